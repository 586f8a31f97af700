// Prefill GEMM for Q4_K weights on gfx950, LDS-ring kernel (the MFMA batches of the linear):
// Y[m, n] = X[m, k] . W[n, k]^T (+ bias), the arithmetic of QLinear::forward with a batch
// of tokens (crates/nn-core/src/layers/quantized/linear.rs:366-400).
//
// Stage s = 64 k = byte group p = s % 4 of super-block sb = s / 4: sub-blocks 2p (the low
// nibbles of the group's 32 bytes per row) and 2p + 1 (the high nibbles).  A ring of NBUF
// LDS buffers holds consecutive stages, copied NBUF - 1 stages ahead by every thread with
// global_load_lds (16 bytes per lane, no register round trip):
//   A: BM rows (32, 64 or 128) x 8 chunks of 8 f16; chunk c of row r sits at slot c ^ ((r >> 1) & 7), so
//      the 16-byte fragment reads of 16 consecutive rows fall in distinct banks;
//   B: the raw tile16 bytes of group p: tile x plane x 16 rows x 16 bytes;
// and the super-block headers ride along with the first stage of each super-block.
//
// NW waves (4 or 8) in WGN wave columns: four side by side, each a BM x BN/4 wave tile
// (WGN = 4; WGN = 2 gives 2 x 2 waves of BM/2 x BN/2), or eight as 2 x 4 of BM/2 x BN/4;
// every wave dequantizes the raw bytes of its own columns in registers (no dequantized
// copy through LDS):
// consumer lane 16G + r takes bytes 8G .. 8G + 7 of row r's group (plane G >> 1), whose
// low nibbles are k = 64p + 8G + i of sub-block 2p and high nibbles k = 64p + 32 + 8G + i
// of sub-block 2p + 1, so each stage is two MFMA steps of 32 k, one sub-block each, and
// the A fragment of lane group G is chunk G (step 0) or 4 + G (step 1) of the row.
// B = sc * q is an exact f16: the masked nibble pairs are f16 subnormals q * 2^-24 (low
// nibbles) or 16 q * 2^-24 (high nibbles), times sc or sc / 16 (exact f16 products).
//
// The per-super-block factor d: the MFMAs of a super-block accumulate from zero into
// AGPR partial sums (so the dequantization VALU work issues beside the MFMAs), and at the
// super-block's end every lane adds d_n * partial into its f32 totals.  The min term
// dmin * m_j * sum(x over the sub-block) is one more MFMA per tile and super-block
// (in its third stage), into accumulators of its own, from the weight's aux plane
// (dmin * m_j * s_n precomputed at upload as exact f16 hi + lo) and the staged
// sub-block sums of x (hi + lo), both carried by the super-block's first stage.
//
// Split-K (KS > 1, when the output tiles alone would leave CUs idle): workgroup (tile,
// ks) covers super-blocks [ks * nblk / KS, (ks + 1) * nblk / KS) and stores its partial
// result in f32 slab ks of the scratch; a finalize kernel sums the slabs in order
// (deterministic), adds the bias and converts.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// f16 pair product a * (s.lo, s.lo) (HI = 0) or a * (s.hi, s.hi) (HI = 1)
template <int HI>
__device__ __forceinline__ uint32_t pk_mul_bcast(uint32_t a, uint32_t s) {
    const half2v sv = __builtin_bit_cast(half2v, s);
    const half2v b = HI ? half2v{sv[1], sv[1]} : half2v{sv[0], sv[0]};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) * b);
}

#define NNQ_GPTR(p) ((const __attribute__((address_space(1))) void *)(p))
#define NNQ_LPTR(p) ((__attribute__((address_space(3))) void *)(p))

template <int BN, int NBUF, int WGN, int BM_, int NW>
struct RK {
    // NW waves: WGN wave columns x (NW / WGN) wave rows, wave tile WM x (BN / WGN)
    static constexpr int BM = BM_, NTH = NW * 64, NTILE = BN / 16, NT = NTILE / WGN;
    static constexpr int WM = BM * WGN / NW, MT = WM / 16;
    static constexpr int A_CH = BM * 8, B_CH = NTILE * 32, CH = A_CH + B_CH;
    static constexpr int LPT = (CH + NTH - 1) / NTH;  // copy instructions per thread and stage
    static constexpr int BUF = LPT * NTH * 16;
    // per super-block (two areas, by parity): headers (NTILE x 16 rows x 16 B), the
    // staged sub-block sums of x (BM rows x hi / lo x 16 B, in an area of one granule
    // per thread), the weight's min-term operands (NTILE x hi / lo x 16 rows x 16 B)
    static constexpr int AUX_CH = NTILE * 32, AUXI = (AUX_CH + NTH - 1) / NTH;
    static constexpr int SB_EXTRA = 2 + AUXI;  // copy instructions per thread and super-block
    static constexpr int HDR_OFF = 0, XS_OFF = NTH * 16, AUX_OFF = XS_OFF + NTH * 16;
    static constexpr int SBA = AUX_OFF + AUXI * NTH * 16;
    // epilogue factors: 2^-s_row of the BM rows, s_n of the BN columns (f32)
    static constexpr int EPI_CH = (BM + BN) / 4;
    static constexpr size_t LDS = (size_t)NBUF * BUF + 2 * SBA + NTH * 16;
    static_assert(EPI_CH <= NTH, "one epilogue-factor copy per thread");
    static_assert((size_t)BM * (BN * 4 + 16) <= (size_t)NBUF * BUF + 2 * SBA, "the f32 output tile fits below the factors");
    static_assert(NTILE % WGN == 0, "column tiles split evenly over the wave columns");
    static_assert(MT * 16 == WM && MT >= 1, "wave rows");
    static_assert(A_CH % NTH == 0, "a copy instruction is all A or all B");
    static_assert(NTILE * 16 <= NTH && BM * 2 <= NTH, "one header and one sums copy per thread");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
    static_assert((NBUF - 1) * (LPT + SB_EXTRA) < 64, "vmcnt range");
    // the super-block areas alternate by parity: the copy issued in iteration s (stage
    // s + NBUF - 1) may start a super-block of the current one's parity only after the
    // current one's last read of its area (stage p = 2), i.e. 4 sb + 2 + NBUF - 1 < 4 (sb + 2)
    static_assert(NBUF <= 6, "a deeper ring would overwrite the current super-block's area");
};

// VMEM instructions a thread issues after the batch of stage s and before the wait in
// iteration s: the batches of stages s + 1 .. s + NBUF - 2, those that start a
// super-block carrying SBX extra copies.  p = s % 4 fixes the count.
template <int NBUF, int LPT, int SBX>
constexpr int rk_wait(int p) {
    int n = (NBUF - 2) * LPT;
    for (int t = p + 1; t <= p + NBUF - 2; t++)
        if (t % 4 == 0) n += SBX;
    return n;
}

template <int BN, int NBUF, int WGN, int BM_, int NW>
__global__ __launch_bounds__(NW * 64) void gemm_q4k_rk_kernel(GemmArgs a, GemmScratch sc) {
    using C = RK<BN, NBUF, WGN, BM_, NW>;
    constexpr int MT = C::MT, NT = C::NT, LPT = C::LPT, NTH = C::NTH, BM = C::BM;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    unsigned char *ring = smem;
    unsigned char *sba = smem + (size_t)NBUF * C::BUF;  // the two per-super-block areas
    float *epi = reinterpret_cast<float *>(sba + 2 * C::SBA);  // [BM] 2^-s_row, [BN] s_n
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv / WGN, wn = wv % WGN;
    const int G = lane >> 4, c16 = lane & 15;
    const int K = (int)a.k, M = (int)a.m, nblk_all = (int)a.nblk, ntile = (int)a.ntile;
    const int KS = sc.ksplit;
    // f32 activations: the staged hi and lo planes are two halves of the work, like two
    // more K parts (slabs KS .. 2 KS - 1 hold the lo plane; the min term goes with hi)
    const int NPL = a.x_bf16 ? 1 : 2, NS = KS * NPL;
    const int nsub = K / 32;

    // Tile order: workgroup ids go round-robin over the 8 XCDs, so when the count
    // allows, each XCD gets a contiguous run of tiles (same activation rows and K range,
    // L2-shared); column tiles vary fastest, then row tiles, then the K split.
    const int nct = (int)((a.ntile * 16 + BN - 1) / BN), nrt = (M + BM - 1) / BM;
    const int total = nct * nrt * NS, bid = (int)blockIdx.x;
    const int T = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
    const int ksp = T / (nct * nrt), Tt = T % (nct * nrt);  // slab: plane ksp / KS, K part ksp % KS
    const int plane = ksp / KS, ks = ksp % KS;
    const int m0 = (Tt / nct) * BM, t0 = (Tt % nct) * (BN / 16);
    const int nblk = nblk_all / KS, sb0 = ks * nblk;  // this workgroup's super-blocks
    const int nstage = nblk * 4;

    // epilogue factors, copied to LDS now (read back after the main loop): 2^-s_row of
    // the tile's rows, s_n (the power of two of the min-term operands) of its columns.
    // A ragged last row tile clamps to the granule holding row M - 1; the scratch that
    // holds 2^-s_row is padded to 256 bytes, so that granule is inside it.
    {
        const float *s_rows = reinterpret_cast<const float *>(a.aux + (size_t)ntile * nblk_all * 512);
        const int g = min(tid, C::EPI_CH - 1);
        const float *esrc = g < BM / 4 ? sc.rowback + 4 * min(m0 / 4 + g, (M - 1) / 4)
                                       : s_rows + (size_t)t0 * 16 + 4 * (g - BM / 4);
        __builtin_amdgcn_global_load_lds(NNQ_GPTR(esrc), NNQ_LPTR(reinterpret_cast<unsigned char *>(epi) + wv * 64 * 16),
                                         16, 0, 0);
    }

    // ---- copy sources (every thread copies LPT granules per stage) ----
    const uint8_t *src[LPT];
#pragma unroll
    for (int j = 0; j < LPT; j++) {
        const int c = j * NTH + tid;
        if (j * NTH < C::A_CH) {
            const int r = c >> 3, kc = (c & 7) ^ ((r >> 1) & 7);
            const int row = min(m0 + r, M - 1);
            src[j] = reinterpret_cast<const uint8_t *>(sc.xh) +
                     ((size_t)plane * M * K + (size_t)row * K + (size_t)sb0 * 256 + 8 * kc) * 2;
        } else {
            // granules past B_CH re-copy the last one into slots nobody reads
            const int cb = min(c - C::A_CH, C::B_CH - 1);
            const int tile = min(t0 + (cb >> 5), ntile - 1);
            src[j] = a.qs + ((size_t)tile * nblk_all + sb0) * 2048 + ((cb >> 4) & 1) * 1024 + (cb & 15) * 16;
        }
    }
    // per super-block: header granule (tile, row), sums granule (row, hi / lo), min-term
    // operand granules (tile, hi / lo, row); all advance by one super-block at a time
    const uint8_t *hsrc, *xsrc, *asrc[C::AUXI];
    {
        const int cc = min(tid, C::NTILE * 16 - 1);
        hsrc = a.hdr + ((size_t)min(t0 + cc / 16, ntile - 1) * nblk_all + sb0) * 256 + (cc % 16) * 16;
        const int row = min(m0 + (tid >> 1), M - 1);
        xsrc = reinterpret_cast<const uint8_t *>(sc.xs) +
               ((size_t)(tid & 1) * M * nsub + (size_t)row * nsub + (size_t)sb0 * 8) * 2;
#pragma unroll
        for (int i = 0; i < C::AUXI; i++) {
            const int c = min(i * NTH + tid, C::AUX_CH - 1);
            asrc[i] = a.aux + ((size_t)min(t0 + (c >> 5), ntile - 1) * nblk_all + sb0) * 512 + ((c >> 4) & 1) * 256 +
                      (c & 15) * 16;
        }
    }
    // stage s: its A and B granules, plus (first stage of a super-block) the super-block's
    // header, sums and min-term operands; stages past the end re-copy the last one into a
    // buffer nobody reads any more
    auto issue = [&](int s) {
        const int sv = min(s, nstage - 1);
        const uint32_t offa = (uint32_t)sv * 128u, offb = (uint32_t)sv * 256u + (uint32_t)(sv >> 2) * 1024u;
        unsigned char *buf = ring + (size_t)(s % NBUF) * C::BUF;
#pragma unroll
        for (int j = 0; j < LPT; j++)
            __builtin_amdgcn_global_load_lds(NNQ_GPTR(src[j] + (j * NTH < C::A_CH ? offa : offb)),
                                             NNQ_LPTR(buf + (size_t)(j * NTH + wv * 64) * 16), 16, 0, 0);
        if ((s & 3) == 0) {
            const int sb = s >> 2, sbc = min(sb, nblk - 1);
            unsigned char *area = sba + (size_t)(sb & 1) * C::SBA;
            __builtin_amdgcn_global_load_lds(NNQ_GPTR(hsrc + (size_t)sbc * 256),
                                             NNQ_LPTR(area + C::HDR_OFF + (size_t)(wv * 64) * 16), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(NNQ_GPTR(xsrc + (size_t)sbc * 16),
                                             NNQ_LPTR(area + C::XS_OFF + (size_t)(wv * 64) * 16), 16, 0, 0);
#pragma unroll
            for (int i = 0; i < C::AUXI; i++)
                __builtin_amdgcn_global_load_lds(NNQ_GPTR(asrc[i] + (size_t)sbc * 512),
                                                 NNQ_LPTR(area + C::AUX_OFF + (size_t)(i * NTH + wv * 64) * 16), 16, 0,
                                                 0);
        }
    };

    // ---- per-lane state ----
    floatx4 part[MT][NT];  // this super-block's sums of x * sc * q (MFMA accumulators)
    floatx4 mins[MT][NT];  // min term, all super-blocks (MFMA accumulators)
    float tot[MT][NT][4];  // sum over super-blocks of d_n * part
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            part[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
            mins[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++) tot[i][j][e] = 0.f;
        }
    float dcol[NT];
    uint32_t scw[NT][4];  // per byte group p: f16 (sc_2p, sc_2p+1 / 16)
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = wm * C::WM + mt * 16 + c16;

#pragma unroll
    for (int t = 0; t < NBUF - 1; t++) issue(t);

    for (int sb = 0; sb < nblk; sb++) {
        const unsigned char *area = sba + (size_t)(sb & 1) * C::SBA;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * sb + p;
            // this thread's copies of stage s (p is a constant once the loop is unrolled)
            if (p == 0)
                wait_vmcnt<rk_wait<NBUF, LPT, C::SB_EXTRA>(0)>();
            else if (p == 1)
                wait_vmcnt<rk_wait<NBUF, LPT, C::SB_EXTRA>(1)>();
            else if (p == 2)
                wait_vmcnt<rk_wait<NBUF, LPT, C::SB_EXTRA>(2)>();
            else
                wait_vmcnt<rk_wait<NBUF, LPT, C::SB_EXTRA>(3)>();
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage s - 1
            __builtin_amdgcn_s_barrier();        // everyone's copies of stage s have landed
            __builtin_amdgcn_sched_barrier(0);
            issue(s + NBUF - 1);                 // into the buffer of stage s - 1
            const unsigned char *buf = ring + (size_t)(s % NBUF) * C::BUF;
            u32x2 braw[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                braw[nt] = *reinterpret_cast<const u32x2 *>(
                    buf + C::A_CH * 16 + ((((wn * NT + nt) * 2 + (G >> 1)) * 16 + c16) * 16) + 8 * (G & 1));
            u32x4 af[2][MT];
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const int r = arow[mt], kc = 4 * j + G;
                    af[j][mt] = *reinterpret_cast<const u32x4 *>(buf + (size_t)(r * 8 + (kc ^ ((r >> 1) & 7))) * 16);
                }
            if (p == 0) {
                // BlockQ4K header: d | dmin, scales[12] (get_scale_min_k4,
                // crates/nn-core/src/layers/quantized/linear.rs:166-176)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const u32x4 h = *reinterpret_cast<const u32x4 *>(area + C::HDR_OFF +
                                                                     (size_t)((wn * NT + nt) * 16 + c16) * 16);
                    dcol[nt] = f16_to_f32(h[0] & 0xFFFFu);
                    const uint32_t sc03 = h[1] & 0x3F3F3F3Fu;
                    const uint32_t sc47 = (h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint32_t w = q < 2 ? sc03 : sc47;
                        const uint32_t lo = (w >> (16 * (q & 1))) & 0xFFu, hi = (w >> (16 * (q & 1) + 8)) & 0xFFu;
                        scw[nt][q] = f32_to_f16_bits((float)lo) | (f32_to_f16_bits(0.0625f * (float)hi) << 16);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const uint32_t w0 = braw[nt][0], w1 = braw[nt][1];
                    const uint32_t w0s = w0 >> 8, w1s = w1 >> 8;
                    u32x4 b;
                    if (j == 0)
                        b = u32x4{pk_mul_bcast<0>(w0 & 0x000F000Fu, scw[nt][p]),
                                  pk_mul_bcast<0>(w0s & 0x000F000Fu, scw[nt][p]),
                                  pk_mul_bcast<0>(w1 & 0x000F000Fu, scw[nt][p]),
                                  pk_mul_bcast<0>(w1s & 0x000F000Fu, scw[nt][p])};
                    else
                        b = u32x4{pk_mul_bcast<1>(w0 & 0x00F000F0u, scw[nt][p]),
                                  pk_mul_bcast<1>(w0s & 0x00F000F0u, scw[nt][p]),
                                  pk_mul_bcast<1>(w1 & 0x00F000F0u, scw[nt][p]),
                                  pk_mul_bcast<1>(w1s & 0x00F000F0u, scw[nt][p])};
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
                        part[mt][nt] = mfma16x16x32_f16(af[j][mt], b,
                                                        (p == 0 && j == 0) ? floatx4{0.f, 0.f, 0.f, 0.f} : part[mt][nt]);
                }
            }
            if (p == 2 && plane == 0) {  // workgroup-uniform
                // min term of the super-block: one MFMA per tile whose 32 k are the four
                // (x hi / lo) x (w hi / lo) cross products of its 8 sub-blocks: lane group G
                // takes x part G & 1 (staged negated: the min term is subtracted) and w part G >> 1
                u32x4 xa[MT], wb[NT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    xa[mt] = *reinterpret_cast<const u32x4 *>(area + C::XS_OFF + (size_t)(arow[mt] * 2 + (G & 1)) * 16);
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    wb[nt] = *reinterpret_cast<const u32x4 *>(
                        area + C::AUX_OFF + (size_t)(((wn * NT + nt) * 2 + (G >> 1)) * 16 + c16) * 16);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) mins[mt][nt] = mfma16x16x32_f16(xa[mt], wb[nt], mins[mt][nt]);
            }
            if (p == 3) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
#pragma unroll
                        for (int e = 0; e < 4; e++) tot[mt][nt][e] += dcol[nt] * part[mt][nt][e];
            }
        }
    }
    wait_vmcnt<0>();  // the trailing (unused) copies
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // every wave is done with the ring: it becomes the output tile

    // y = (tot * 2^24 (the f16-subnormal codes) * 2^-8 * s_n + mins) * (2^8 / s_n) * 2^-s_row:
    // the staged sums carry 2^-8 and the min-term operands s_n.  The tile is assembled in
    // LDS (rows padded by 16 bytes, so the four row groups of a store land in distinct
    // banks) and written out as 16-byte row chunks.
    const bool f32out = NS > 1 || !a.y_bf16;
    const int es = f32out ? 4 : 2, rs = BN * es + 16;
    unsigned char *stg = smem;
    // every factor is read before the first tile write (the compiler cannot tell the
    // two LDS regions apart, so a read after a write would wait for it)
    float rb[MT][4], f1[NT], f2[NT], bc[NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int e = 0; e < 4; e++) rb[mt][e] = epi[wm * C::WM + mt * 16 + 4 * G + e];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int cl = (wn * NT + nt) * 16 + c16;
        // s_n = 2^e is a normal power of two: 2^16 * s_n and 2^8 / s_n are exact
        const uint32_t eb = __float_as_uint(epi[BM + cl]) >> 23;
        f1[nt] = __uint_as_float((eb + 16u) << 23);
        f2[nt] = __uint_as_float((262u - eb) << 23);
        bc[nt] = (a.bias && NS == 1) ? a.bias[(int64_t)t0 * 16 + cl] : 0.0f;
    }
    float yv[MT][NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                yv[mt][nt][e] = (tot[mt][nt][e] * f1[nt] + mins[mt][nt][e]) * f2[nt] * rb[mt][e] + bc[nt];
    if (f32out) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<float *>(stg + (wm * C::WM + mt * 16 + 4 * G + e) * rs +
                                               ((wn * NT + nt) * 16 + c16) * 4) = yv[mt][nt][e];
    } else {
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<uint16_t *>(stg + (wm * C::WM + mt * 16 + 4 * G + e) * rs +
                                                  ((wn * NT + nt) * 16 + c16) * 2) =
                        (uint16_t)f32_to_bf16_bits(yv[mt][nt][e]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    const int cpr = BN * es / 16;  // 16-byte chunks per row
    unsigned char *ybase = NS > 1 ? reinterpret_cast<unsigned char *>(sc.ysplit + (int64_t)ksp * M * a.n)
                                  : reinterpret_cast<unsigned char *>(a.y);
    for (int c = tid; c < BM * cpr; c += NTH) {
        const int rl = c / cpr, ch = c - rl * cpr;
        if (m0 + rl >= M) break;  // rows run in order: the rest are past M as well
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + rl * rs + ch * 16);
        *reinterpret_cast<u32x4 *>(ybase + ((int64_t)(m0 + rl) * a.n + (int64_t)t0 * 16) * es + ch * 16) = v;
    }
}

// split-K result: the partial slabs summed in order plus the bias, stored as f32 or bf16;
// four consecutive elements per thread (n is a multiple of 128)
__global__ __launch_bounds__(256) void gemm_finalize_kernel(const float *ys, int ks, const float *bias, void *y,
                                                            int y_bf16, int64_t m, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= m * n) return;
    floatx4 v = *reinterpret_cast<const floatx4 *>(ys + i);
    for (int j = 1; j < ks; j++) v += *reinterpret_cast<const floatx4 *>(ys + (int64_t)j * m * n + i);
    if (bias) v += *reinterpret_cast<const floatx4 *>(bias + i % n);
    if (y_bf16)
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(y) + i) =
            u32x2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16), f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
    else
        *reinterpret_cast<floatx4 *>(reinterpret_cast<float *>(y) + i) = v;
}

template <int BN, int NBUF, int WGN, int BM, int NW>
int launch_rk(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    using C = RK<BN, NBUF, WGN, BM, NW>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_rk_kernel<BN, NBUF, WGN, BM, NW>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const int nct = (int)((a.ntile * 16 + BN - 1) / BN), nrt = (int)((a.m + C::BM - 1) / C::BM);
    const int ns = sc.ksplit * (a.x_bf16 ? 1 : 2);  // f32 activations: hi and lo plane slabs
    hipLaunchKernelGGL((gemm_q4k_rk_kernel<BN, NBUF, WGN, BM, NW>), dim3((unsigned)(nct * nrt * ns)), dim3(C::NTH), C::LDS,
                       st, a, sc);
    int e = (int)hipGetLastError();
    if (e || ns == 1) return e;
    const int64_t cnt = a.m * a.n / 4;
    hipLaunchKernelGGL(gemm_finalize_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, st, sc.ysplit, ns, a.bias,
                       a.y, a.y_bf16, a.m, a.n);
    return (int)hipGetLastError();
}

}  // namespace

// Shapes the ring kernel takes (N % 128 == 0, a 16-byte aligned output; f32 activations run
// their staged hi and lo planes as two halves of the work, summed by the finalize):
// BM x BN tiles, BM the smallest of 32, 64, 128 holding M (128 beyond), BN 192 or 128
// (dividing N), K split 1, 2, 4, 8 or 16 ways (a divisor of the super-block count leaving
// at least 4 super-blocks per workgroup, 2 with BM < 128).  Of these, the plan with the
// least estimated time: rounds of workgroups (one resident per CU: the rings of the small
// row tiles are deepened to 6 stages, which LDS holds once) times stages per workgroup, a 128-wide
// stage at 0.8 of a 192-wide one, plus one stage for the split-K finalize.  (Assuming two
// resident workgroups with shallower rings measured 5-25% slower at M = 16 to 64.)
// Returns the K split, or 0 when the shape does not fit.
int gemm_ring_plan(const GemmArgs &a, int *bn, int *bm) {
    // (the output tile is written in 16-byte chunks of whole rows: no partial last tile)
    if (a.m < 1 || a.nblk < 1 || a.n != a.ntile * 16 || (reinterpret_cast<uintptr_t>(a.y) & 15)) return 0;
    const int npl = a.x_bf16 ? 1 : 2;  // f32 activations: hi and lo planes, each a full pass
    const int rows = a.m <= 32 ? 32 : (a.m <= 64 ? 64 : 128);
    const int64_t ncols = a.ntile * 16, nrt = (a.m + rows - 1) / rows;
    const int min_sb = rows == 128 ? 4 : 2, per_cu = 1;
    double best_cost = 0.0;
    int best_bn = 0, best_ks = 0;
    for (int cand : {192, 128}) {
        if (ncols % cand) continue;
        for (int ks = 1; ks <= 16; ks *= 2) {
            if (a.nblk % ks || (ks > 1 && a.nblk / ks < min_sb)) continue;
            const int64_t wgs = nrt * (ncols / cand) * ks * npl;
            const int64_t rounds = (wgs + 256 * per_cu - 1) / (256 * per_cu);
            const double cost =
                (double)rounds * (double)(a.nblk / ks) * (cand == 192 ? 1.0 : 0.8) + (ks * npl > 1 ? 1.0 : 0.0);
            if (best_bn == 0 || cost < best_cost) {
                best_cost = cost;
                best_bn = cand;
                best_ks = ks;
            }
        }
    }
    if (best_bn == 0) return 0;
    if (bn) *bn = best_bn;
    if (bm) *bm = rows;
    return best_ks;
}

int launch_gemm_finalize(const float *ys, int ks, const float *bias, void *y, int y_bf16, int64_t m, int64_t n,
                         void *stream) {
    const int64_t cnt = m * n / 4;
    hipLaunchKernelGGL(gemm_finalize_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, (hipStream_t)stream, ys,
                       ks, bias, y, y_bf16, m, n);
    return (int)hipGetLastError();
}

int launch_gemm_ring(const GemmArgs &a, const GemmScratch &sc, void *stream) {
    int bn = 0, bm = 0;
    const int ksplit = gemm_ring_plan(a, &bn, &bm);
    if (ksplit == 0 || sc.ksplit != ksplit || (ksplit * (a.x_bf16 ? 1 : 2) > 1 && !sc.ysplit))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    // four waves side by side (BM rows x BN / 4 columns each): measured 4-5% faster on
    // MI355X than 2 x 2 (BM / 2 x BN / 2), which halves the A reads from LDS but doubles
    // the dequantization of every column.  128 x 192 tiles take eight waves (2 x 4 of
    // 64 x 48, two per SIMD, 178 registers each): 3-7% faster at M = 128 and 512; the
    // 128-wide tiles measured 3% slower with eight, and 4 x 2 waves of 32 x 96 (four
    // dequantizations per column) 30-40% slower.
    // The smaller row tiles leave LDS for a deeper ring (more stages in flight).
    if (bm == 32) return bn == 192 ? launch_rk<192, 6, 4, 32, 4>(a, sc, st) : launch_rk<128, 6, 4, 32, 4>(a, sc, st);
    if (bm == 64) return bn == 192 ? launch_rk<192, 6, 4, 64, 4>(a, sc, st) : launch_rk<128, 6, 4, 64, 4>(a, sc, st);
    return bn == 192 ? launch_rk<192, 4, 4, 128, 8>(a, sc, st) : launch_rk<128, 4, 4, 128, 4>(a, sc, st);
}

}  // namespace nnq
