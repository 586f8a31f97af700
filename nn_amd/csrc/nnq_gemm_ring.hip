// Prefill GEMM for Q4_K weights on gfx950, ring kernel (M >= 128):
// Y[m, n] = X[m, k] . W[n, k]^T (+ bias), the same arithmetic as gemm_q4k_kernel
// (QLinear::forward with a batch of tokens, crates/nn-core/src/layers/quantized/linear.rs:366-400).
//
// Stage s = 64 k = byte group p = s % 4 of super-block sb = s / 4, i.e. sub-blocks 2p
// (low nibbles: k 0..31 of the stage) and 2p + 1 (high nibbles: k 32..63).  A ring of
// NBUF LDS buffers holds consecutive stages:
//   A: P planes x BM rows x 8 chunks of 8 f16; chunk c of row r sits at slot
//      c ^ ((r >> 1) & 7), so the 16-byte fragment reads of 16 consecutive rows fall
//      in distinct banks;
//   B: NTILE tiles x 2 planes x 16 rows x 16 bytes (the tile16 bytes of group p).
// Stages are copied NBUF - 1 ahead with global_load_lds (16 bytes per lane, no
// register round trip).  Every thread issues LPT copies per stage (copies past the
// stage's chunks land in a pad), so one vmcnt immediate per iteration holds for every
// wave; the super-block headers are copied the same way (one copy per thread, one
// super-block ahead, just before a stage's copies), so the loop has no other
// vector-memory loads.
//
// Per iteration: the high-nibble A fragments of stage s are read while the low-nibble
// MFMAs run; then one barrier (stage s + 1 has landed for every wave, and every wave
// is done with the buffer refilled next); then the copies of stage s + NBUF - 1 go
// out and the fragments of stage s + 1 are read while the high-nibble MFMAs run.
//
// The waves split N only (wave tile BM x WN, MT x NT MFMA tiles of 16 x 16), so each B
// fragment is dequantized once per workgroup and reused over BM / 16 rows.  B is
// sc * q as an exact f16: the masked low nibbles q * 2^-24 (subnormals) times sc, and
// the masked high nibbles (16 q) * 2^-24 times sc, with the staged activation of the
// odd sub-blocks pre-scaled by 2^-4 to match (gemm_prep_kernel<P, true>).  The
// accumulator of column n is kept in units of u_n, the latest non-zero d of the
// column, and rescaled by u_prev / u_next when a super-block starts.  The min term runs
// after the main loop from the weight's aux plane (dmin * m_j * s_n precomputed at
// upload as exact f16 hi + lo), so it costs MFMAs and loads but no VALU.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) * __builtin_bit_cast(half2v, b));
}

// f16 pair (v, v) of a small non-negative integer v (exact)
__device__ __forceinline__ uint32_t f16_pair_int(uint32_t v) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)(float)v);
    return h | (h << 16);
}

// s_waitcnt vmcnt(N) only (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

#define NNQ_GPTR(p) ((const __attribute__((address_space(1))) void *)(p))
#define NNQ_LPTR(p) ((__attribute__((address_space(3))) void *)(p))

template <int BM, int BN, int NW, int P, int NBUF>
struct Ring {
    static constexpr int NTH = NW * 64;
    static constexpr int WN = BN / NW, MT = BM / 16, NT = WN / 16;
    static constexpr int NTILE = BN / 16;
    static constexpr int A_CH = P * BM * 8, B_CH = NTILE * 32, CH = A_CH + B_CH;
    static constexpr int LPT = (CH + NTH - 1) / NTH;
    static constexpr int BUF = LPT * NTH * 16;
    static constexpr size_t LDS = (size_t)NBUF * BUF + 2 * NTH * 16;  // ring + two header areas
    static_assert(WN % 16 == 0 && BM % 16 == 0, "16 x 16 MFMA tiles");
    static_assert(A_CH % NTH == 0, "copies of a thread are all A or all B");
    static_assert(NBUF >= 4, "the pipeline needs NBUF - 3 >= 1 stage of slack");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
    static_assert((NBUF - 2) * LPT + 1 < 64, "vmcnt range");
    static_assert(NTILE * 16 <= NTH, "one header copy per thread");
};

// Header batches (issued at iterations t = 3 mod 4, before that iteration's copies)
// that go out after the copies of stage s + 1 and before the mid-iteration wait of
// iteration s: iterations t in [s + 3 - NBUF, s - 1].
constexpr int batches_after(int p, int nbuf) {
    int n = 0;
    for (int d = 3 - nbuf; d <= -1; d++)
        if ((((p + d) % 4) + 4) % 4 == 3) n++;
    return n;
}

template <int BM, int BN, int NW, int P, int NBUF>
__global__ __launch_bounds__(NW * 64) void gemm_q4k_ring_kernel(GemmArgs a, GemmScratch sc) {
    using C = Ring<BM, BN, NW, P, NBUF>;
    constexpr int NTH = C::NTH, MT = C::MT, NT = C::NT, LPT = C::LPT;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, c16 = lane & 15;
    const int K = (int)a.k, M = (int)a.m, nblk = (int)a.nblk, ntile = (int)a.ntile;
    const int nstage = nblk * 4;

    // Tile order: workgroup ids go round-robin over the 8 XCDs, so when the count
    // allows, each XCD gets a contiguous run of tiles (same activation rows, L2-shared).
    const int nct = (int)((a.ntile * 16 + BN - 1) / BN), nrt = (M + BM - 1) / BM;
    const int total = nct * nrt, bid = (int)blockIdx.x;
    const int T = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
    const int m0 = (T / nct) * BM, t0 = (T % nct) * (BN / 16);

    // per-thread copy sources of stage 0; A advances 128 bytes per stage, B
    // 256 bytes per stage plus 1024 per super-block (tile16: 2048 bytes per block)
    const uint8_t *src[LPT];
#pragma unroll
    for (int j = 0; j < LPT; j++) {
        const int c = j * NTH + tid;
        if (j * NTH < C::A_CH) {
            const int pl = c / (BM * 8), rem = c % (BM * 8), r = rem >> 3, kc = (rem & 7) ^ ((r >> 1) & 7);
            const int row = min(m0 + r, M - 1);
            src[j] = reinterpret_cast<const uint8_t *>(sc.xh) + ((size_t)pl * M * K + (size_t)row * K + 8 * kc) * 2;
        } else {
            const int cb = min(c - C::A_CH, C::B_CH - 1);
            const int tile = min(t0 + (cb >> 5), ntile - 1);
            src[j] = a.qs + (size_t)tile * nblk * 2048 + ((cb >> 4) & 1) * 1024 + (cb & 15) * 16;
        }
    }
    auto issue = [&](int s) {  // stages past the end re-copy the last one into a free buffer
        const int sv = min(s, nstage - 1);
        const uint32_t offa = (uint32_t)sv * 128u, offb = (uint32_t)sv * 256u + (uint32_t)(sv >> 2) * 1024u;
        unsigned char *buf = smem + (size_t)(s % NBUF) * C::BUF;
#pragma unroll
        for (int j = 0; j < LPT; j++)
            __builtin_amdgcn_global_load_lds(NNQ_GPTR(src[j] + (j * NTH < C::A_CH ? offa : offb)),
                                             NNQ_LPTR(buf + (size_t)(j * NTH + wn * 64) * 16), 16, 0, 0);
    };

    // this lane's columns: running unit u (latest non-zero d)
    float ucur[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) ucur[nt] = 1.0f;
    // Super-block headers are copied like the stages, one copy per thread, into two LDS
    // areas by super-block parity: chunk c < NTILE * 16 is row c % 16 of tile c / 16,
    // the rest is pad.
    unsigned char *hdr_lds = smem + (size_t)NBUF * C::BUF;
    const uint8_t *hcsrc;
    {
        const int cc = min(tid, C::NTILE * 16 - 1);
        hcsrc = a.hdr + (size_t)min(t0 + cc / 16, ntile - 1) * nblk * 256 + (cc % 16) * 16;
    }
    auto hload = [&](int sb) {
        __builtin_amdgcn_global_load_lds(NNQ_GPTR(hcsrc + (size_t)min(sb, nblk - 1) * 256),
                                         NNQ_LPTR(hdr_lds + (size_t)((sb & 1) * NTH + wn * 64) * 16), 16, 0, 0);
    };
    uint32_t scw[NT][2];  // sc[0..3], sc[4..7] bytes of the current super-block (0 when d == 0)
    float ratio[NT];
    // super-block header: d | dmin, scales (BlockQ4K packing, get_scale_min_k4,
    // crates/nn-core/src/layers/quantized/linear.rs:166-176)
    auto decode = [&](int sb) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const u32x4 h = *reinterpret_cast<const u32x4 *>(hdr_lds + (size_t)(sb & 1) * NTH * 16 +
                                                              ((wn * NT + nt) * 16 + c16) * 16);
            const float d = f16_to_f32(h[0] & 0xFFFFu);
            const uint32_t S1 = h[1], S3 = h[3];
            const uint32_t nzm = d != 0.0f ? 0xFFFFFFFFu : 0u;
            scw[nt][0] = S1 & 0x3F3F3F3Fu & nzm;
            scw[nt][1] = ((S3 & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) & nzm;
            const float un = d != 0.0f ? d : ucur[nt];
            ratio[nt] = ucur[nt] * __builtin_amdgcn_rcpf(un);
            ucur[nt] = un;
        }
    };

    floatx4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // LDS read offsets inside a ring buffer: A chunk (row 16 mt + c16, k-chunk 4 hf + q),
    // whose swizzle key (row >> 1) & 7 does not depend on mt; the 8 raw bytes of (tile
    // wn * NT + nt, row c16, bytes 8q .. 8q + 7)
    int abase[2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) abase[hf] = (c16 * 8 + ((4 * hf + q) ^ ((c16 >> 1) & 7))) * 16;
    const int bbase = C::A_CH * 16 + (wn * NT * 32 + (q >> 1) * 16 + c16) * 16 + 8 * (q & 1);

    // A fragments of a stage in consumption order f = hf * P * MT + pl * MT + mt
    // (hf 0: low-nibble k 0..31, hf 1: high-nibble k 32..63), read D positions ahead.
    constexpr int F = 2 * P * MT, D = 4;
    static_assert(F >= 2 * D, "prefetch distance");
    auto read_frag = [&](const unsigned char *buf, int f) -> u32x4 {
        const int hf = f / (P * MT), pl = (f / MT) % P, mt = f % MT;
        return *reinterpret_cast<const u32x4 *>(buf + pl * BM * 128 + mt * 2048 + abase[hf]);
    };
    u32x2 rawb[NT];
    auto read_b = [&](const unsigned char *buf) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) rawb[nt] = *reinterpret_cast<const u32x2 *>(buf + bbase + nt * 512);
    };
    // B fragments of byte group p from the raw bytes: low nibbles (hf 0) and high (hf 1)
    auto dq_lo = [&](int p, int nt) -> u32x4 {
        const uint32_t w0 = rawb[nt][0], w1 = rawb[nt][1];
        const uint32_t sl = f16_pair_int((scw[nt][p >> 1] >> (16 * (p & 1))) & 0xFFu);
        return u32x4{pk_mul_f16(w0 & 0x000F000Fu, sl), pk_mul_f16((w0 >> 8) & 0x000F000Fu, sl),
                     pk_mul_f16(w1 & 0x000F000Fu, sl), pk_mul_f16((w1 >> 8) & 0x000F000Fu, sl)};
    };
    auto dq_hi = [&](int p, int nt) -> u32x4 {
        const uint32_t w0 = rawb[nt][0], w1 = rawb[nt][1];
        const uint32_t sh = f16_pair_int((scw[nt][p >> 1] >> (16 * (p & 1) + 8)) & 0xFFu);
        return u32x4{pk_mul_f16(w0 & 0x00F000F0u, sh), pk_mul_f16((w0 >> 8) & 0x00F000F0u, sh),
                     pk_mul_f16(w1 & 0x00F000F0u, sh), pk_mul_f16((w1 >> 8) & 0x00F000F0u, sh)};
    };

    // prologue: the header of super-block 0 (decoded at once), then the copies as if
    // iterations -(NBUF - 1) .. -1 had run, with the header batch of super-block 1
    // before the copies of iteration -1
    hload(0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    decode(0);
#pragma unroll
    for (int t = -(NBUF - 1); t <= -1; t++) {
        if (t == -1) hload(1);
        issue(t + NBUF - 1);
    }
    wait_vmcnt<(NBUF - 2) * LPT + 1>();  // stage 0 landed (later: NBUF - 2 stages, one header copy)
    __builtin_amdgcn_s_barrier();
    u32x4 af[F], blo[NT], bhi[NT];
    read_b(smem);
#pragma unroll
    for (int f = 0; f < D; f++) af[f] = read_frag(smem, f);
#pragma unroll
    for (int nt = 0; nt < NT; nt++) blo[nt] = dq_lo(0, nt);

    // The order inside an iteration is pinned with scheduling barriers: groups of
    // (one fragment read D ahead, NT MFMAs, a few VALU), so LDS latency hides under
    // MFMAs with one wave per SIMD.
    for (int sb = 0; sb < nblk; sb++) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * sb + p;
            const unsigned char *buf = smem + (size_t)(s % NBUF) * C::BUF;
            const unsigned char *nbuf = smem + (size_t)((s + 1) % NBUF) * C::BUF;
            u32x4 an[D];
#pragma unroll
            for (int f = 0; f < F; f++) {
                if (f + D < F)
                    af[f + D] = read_frag(buf, f + D);
                else
                    an[f + D - F] = read_frag(nbuf, f + D - F);
                const int hf = f / (P * MT), mt = f % MT;
                if (p == 0 && hf == 0 && f < P * MT && (f / MT) == 0) {
                    // the super-block's first MFMA on acc[mt][*]: rescale to the new unit
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[mt][nt][e] *= ratio[nt];
                }
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    acc[mt][nt] = mfma16x16x32_f16(af[f], hf ? bhi[nt] : blo[nt], acc[mt][nt]);
                if (hf == 0 && f < NT) bhi[f] = dq_hi(p, f);  // needed from f = F / 2 on
                __builtin_amdgcn_sched_barrier(0);
                if (f == F / 2 - 1) {
                    // stage s + 1 landed (for this wave, then for all), buffer of s - 1 retired
                    static_assert(batches_after(0, NBUF) <= 1 && batches_after(1, NBUF) <= 1 &&
                                      batches_after(2, NBUF) <= 1 && batches_after(3, NBUF) <= 1,
                                  "at most one header batch in flight past a stage");
                    if (batches_after(p, NBUF) == 1)  // p is a constant once the loop is unrolled
                        wait_vmcnt<(NBUF - 3) * LPT + 1>();
                    else
                        wait_vmcnt<(NBUF - 3) * LPT>();
                    __builtin_amdgcn_s_barrier();
                    if (p == 3) {
                        decode(sb + 1);  // its copy went out before the copies of stage s + 1
                        hload(sb + 2);   // into the area of super-block sb, decoded one super-block ago
                    }
                    issue(s + NBUF - 1);
                    read_b(nbuf);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (hf == 1 && f >= F / 2 + 2 && f < F / 2 + 2 + NT) blo[f - F / 2 - 2] = dq_lo((p + 1) & 3, f - F / 2 - 2);
            }
#pragma unroll
            for (int f = 0; f < D; f++) af[f] = an[f];
        }
    }
    wait_vmcnt<0>();

    // Back to true scale (times 2^-8 * s_n, s_n the column's power of two for the min
    // term, stored in the aux plane), then subtract the min term on the MFMA: A = the
    // staged sub-block sums (hi, lo), B = dmin * m_j * s_n (hi, lo) from the aux plane.
    const float *s_rows = reinterpret_cast<const float *>(a.aux + (size_t)ntile * nblk * 512);
    float colf[NT];
    const uint8_t *msrc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = min(t0 + wn * NT + nt, ntile - 1);
        const float s_n = s_rows[tile * 16 + c16];
        const float f = ucur[nt] * 16777216.0f * 0.00390625f * s_n;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[mt][nt][e] *= f;
        colf[nt] = 256.0f / s_n;  // exact: s_n is a power of two
        msrc[nt] = a.aux + (size_t)tile * nblk * 512 + c16 * 16;
    }
    // min-term steps: 32 sub-blocks each (lane group q: the 8 sub-blocks of super-block
    // 4 it + q); B is fetched two steps ahead and A one step ahead, so the loads of
    // this latency-bound phase overlap its MFMAs
    const int nsub = K / 32, nit = (nsub + 31) / 32;
    auto load_b = [&](int it, u32x4 (&bh)[NT], u32x4 (&bl)[NT]) {
        const int sb = min(4 * it + q, nblk - 1);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            bh[nt] = ldg128(msrc[nt] + (size_t)sb * 512);
            bl[nt] = ldg128(msrc[nt] + (size_t)sb * 512 + 256);
        }
    };
    auto load_a = [&](int it, u32x4 (&ah)[MT], u32x4 (&al)[MT]) {
        const int sb = min(4 * it + q, nblk - 1);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int row = min(m0 + mt * 16 + c16, M - 1);
            ah[mt] = *reinterpret_cast<const u32x4 *>(sc.xs + (size_t)row * nsub + 8 * sb);
            al[mt] = *reinterpret_cast<const u32x4 *>(sc.xs + (size_t)M * nsub + (size_t)row * nsub + 8 * sb);
        }
    };
    u32x4 bh0[NT], bl0[NT], bh1[NT], bl1[NT], ah[MT], al[MT];
    load_b(0, bh0, bl0);
    load_b(1, bh1, bl1);
    load_a(0, ah, al);
    for (int it = 0; it < nit; it++) {
        u32x4 bh[NT], bl[NT], ahc[MT], alc[MT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            bh[nt] = bh0[nt];
            bl[nt] = bl0[nt];
            bh0[nt] = bh1[nt];
            bl0[nt] = bl1[nt];
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            ahc[mt] = ah[mt];
            alc[mt] = al[mt];
        }
        load_b(it + 2, bh1, bl1);  // clamped past the end: rows of the last super-block, unused
        load_a(it + 1, ah, al);
        // sub-blocks past K (a partial last step) and rows past M contribute zero
        const bool kin = 4 * it + q < nblk;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const bool ok = kin && m0 + mt * 16 + c16 < M;
            // negated: the min term is subtracted
            const u32x4 a1 = ok ? (ahc[mt] ^ 0x80008000u) : u32x4{0u, 0u, 0u, 0u};
            const u32x4 a2 = ok ? (alc[mt] ^ 0x80008000u) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                acc[mt][nt] = mfma16x16x32_f16(a1, bh[nt], acc[mt][nt]);
                acc[mt][nt] = mfma16x16x32_f16(a1, bl[nt], acc[mt][nt]);
                acc[mt][nt] = mfma16x16x32_f16(a2, bh[nt], acc[mt][nt]);
            }
        }
    }

    // store: lane holds rows 4q + e of each 16 x 16 tile, column c16
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int64_t col = (int64_t)(t0 + wn * NT + nt) * 16 + c16;
        if (col >= a.n) continue;
        const float bcol = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t row = m0 + mt * 16 + 4 * q + e;
                if (row >= M) continue;
                const float y = acc[mt][nt][e] * colf[nt] * sc.rowback[row] + bcol;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[row * a.n + col] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[row * a.n + col] = y;
            }
    }
}

template <int BM, int BN, int NW, int P, int NBUF>
int launch_ring(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    using C = Ring<BM, BN, NW, P, NBUF>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_ring_kernel<BM, BN, NW, P, NBUF>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const int nct = (int)((a.ntile * 16 + BN - 1) / BN), nrt = (int)((a.m + BM - 1) / BM);
    hipLaunchKernelGGL((gemm_q4k_ring_kernel<BM, BN, NW, P, NBUF>), dim3((unsigned)(nct * nrt)), dim3(C::NTH), C::LDS,
                       st, a, sc);
    return (int)hipGetLastError();
}

}  // namespace

// bf16 activations, 128 x 192 tiles, one workgroup per CU at least (256 CUs)
bool gemm_ring_fits(const GemmArgs &a) {
    const int64_t ncols = a.ntile * 16;
    return a.x_bf16 && a.m >= 128 && ncols % 192 == 0 && ((a.m + 127) / 128) * (ncols / 192) >= 256;
}

int launch_gemm_ring(const GemmArgs &a, const GemmScratch &sc, void *stream) {
    if (!gemm_ring_fits(a)) return (int)hipErrorInvalidValue;
    return launch_ring<128, 192, 4, 1, 6>(a, sc, (hipStream_t)stream);
}

}  // namespace nnq
