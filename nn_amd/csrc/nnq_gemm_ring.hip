// Prefill GEMM for Q4_K weights on gfx950, warp-specialized ring kernel (bf16
// activations, M >= 128): Y[m, n] = X[m, k] . W[n, k]^T (+ bias), the same arithmetic
// as gemm_q4k_kernel (QLinear::forward with a batch of tokens,
// crates/nn-core/src/layers/quantized/linear.rs:366-400).
//
// Stage s = 64 k = byte group p = s % 4 of super-block sb = s / 4, i.e. sub-blocks 2p
// (low nibbles: k 0..31 of the stage) and 2p + 1 (high nibbles: k 32..63).  A ring of
// NBUF LDS buffers holds consecutive stages:
//   A: BM rows x 8 chunks of 8 f16; chunk c of row r sits at slot c ^ ((r >> 1) & 7),
//      so the 16-byte fragment reads of 16 consecutive rows fall in distinct banks;
//   B: NTILE tiles x 2 planes x 16 rows x 16 bytes (the tile16 bytes of group p).
// Stages are copied NBUF - 1 ahead with global_load_lds (16 bytes per lane, no
// register round trip); the super-block headers are copied the same way, one
// super-block ahead, into two LDS areas by super-block parity.
//
// Eight waves: 0..3 consume (MFMA only, wave tile BM x BN / 4), 4..7 produce, one of
// each per SIMD, so the producers' dequantization VALU runs beside the consumers'
// MFMAs.  Per iteration s, after one barrier:
//   producers: copy stage s + NBUF - 1, wait for their own copies of stage s + 1, and
//     dequantize the raw B bytes they copied themselves into the f16 buffer (s + 1) & 1
//     ([tile][hf][lane] x 16 bytes: the consumers' B fragments), sc folded in;
//   consumers: the MFMAs of stage s (A from the ring, B from f16 buffer s & 1).
// B is sc * q as an exact f16: the masked low nibbles q * 2^-24 (subnormals) times sc,
// and the masked high nibbles (16 q) * 2^-24 times sc, with the staged activation of
// the odd sub-blocks pre-scaled by 2^-4 to match (gemm_prep_kernel<P, true>).  The
// accumulator of column n is kept in units of u_n, the latest non-zero d of the
// column, and rescaled by u_prev / u_next when a super-block starts.  The min term runs
// after the main loop from the weight's aux plane (dmin * m_j * s_n precomputed at
// upload as exact f16 hi + lo).
//
// Split-K (KS > 1, when the output tiles alone would leave CUs idle): workgroup
// (tile, ks) covers super-blocks [ks * nblk / KS, (ks + 1) * nblk / KS) and stores its
// partial result in f32 slab ks of the scratch; a finalize kernel sums the slabs in
// order (deterministic), adds the bias and converts.
#include <cstdlib>

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


// ---------------------------------------------------------------------------------
template <int BN, int NBUF>
struct WS {
    static constexpr int BM = 128, NTILE = BN / 16, NC = 4, NP = 4;
    static constexpr int NTH = (NC + NP) * 64, PTH = NP * 64;
    static constexpr int MT = BM / 16, NT = NTILE / NC;
    static constexpr int A_CH = BM * 8, B_CH = NTILE * 32, CH = A_CH + B_CH;
    static constexpr int LPT = (CH + PTH - 1) / PTH;
    static constexpr int NO = (B_CH + PTH - 1) / PTH;  // raw B chunks dequantized per producer thread
    static constexpr int BUF = LPT * PTH * 16;
    static constexpr int F16B = NTILE * 2 * 64 * 16;
    static constexpr int HDR = PTH * 16;
    static constexpr size_t LDS = (size_t)NBUF * BUF + 2 * F16B + 2 * HDR;
    static_assert(NTILE % NC == 0, "tiles split evenly over the consumers");
    static_assert(A_CH % PTH == 0, "a copy instruction is all A or all B");
    static_assert(NTILE * 16 <= PTH, "one header copy per producer thread");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
    static_assert(NBUF >= 4 && (NBUF - 2) * LPT + 2 < 64, "vmcnt range");
};

// header batches (at iterations t = 3 mod 4, before that iteration's copies) issued
// after the copies of stage s + 1 and before the producers' wait in iteration s
constexpr int ws_batches(int p, int nbuf) {
    int n = 0;
    for (int d = 3 - nbuf; d <= 0; d++)
        if ((((p + d) % 4) + 4) % 4 == 3) n++;
    return n;
}

template <int BN, int NBUF>
__global__ __launch_bounds__(512) void gemm_q4k_ws_kernel(GemmArgs a, GemmScratch sc) {
    using C = WS<BN, NBUF>;
    constexpr int MT = C::MT, NT = C::NT, LPT = C::LPT, PTH = C::PTH, BM = C::BM, NO = C::NO;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    unsigned char *ring = smem;
    unsigned char *f16b = smem + (size_t)NBUF * C::BUF;
    unsigned char *hdr_lds = f16b + 2 * C::F16B;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = (int)a.k, M = (int)a.m, nblk_all = (int)a.nblk, ntile = (int)a.ntile;
    const int KS = sc.ksplit;

    // Tile order: workgroup ids go round-robin over the 8 XCDs, so when the count
    // allows, each XCD gets a contiguous run of tiles (same activation rows and K range,
    // L2-shared); column tiles vary fastest, then row tiles, then the K split.
    const int nct = (int)((a.ntile * 16 + BN - 1) / BN), nrt = (M + BM - 1) / BM;
    const int total = nct * nrt * KS, bid = (int)blockIdx.x;
    const int T = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
    const int ks = T / (nct * nrt), Tt = T % (nct * nrt);
    const int m0 = (Tt / nct) * BM, t0 = (Tt % nct) * (BN / 16);
    const int nblk = nblk_all / KS, sb0 = ks * nblk;  // this workgroup's super-blocks
    const int nstage = nblk * 4;

    if (wv >= C::NC) {
        // ================================ producers ================================
        const int pw = wv - C::NC, pj = tid - C::NC * 64;
        const uint8_t *src[LPT];
#pragma unroll
        for (int j = 0; j < LPT; j++) {
            const int c = j * PTH + pj;
            if (j * PTH < C::A_CH) {
                const int r = c >> 3, kc = (c & 7) ^ ((r >> 1) & 7);
                const int row = min(m0 + r, M - 1);
                src[j] = reinterpret_cast<const uint8_t *>(sc.xh) + ((size_t)row * K + (size_t)sb0 * 256 + 8 * kc) * 2;
            } else {
                const int cb = min(c - C::A_CH, C::B_CH - 1);
                const int tile = min(t0 + (cb >> 5), ntile - 1);
                src[j] = a.qs + ((size_t)tile * nblk_all + sb0) * 2048 + ((cb >> 4) & 1) * 1024 + (cb & 15) * 16;
            }
        }
        auto issue = [&](int s) {  // stages past the end re-copy the last one into a free buffer
            const int sv = min(s, nstage - 1);
            const uint32_t offa = (uint32_t)sv * 128u, offb = (uint32_t)sv * 256u + (uint32_t)(sv >> 2) * 1024u;
            unsigned char *buf = ring + (size_t)(s % NBUF) * C::BUF;
#pragma unroll
            for (int j = 0; j < LPT; j++)
                __builtin_amdgcn_global_load_lds(NNQ_GPTR(src[j] + (j * PTH < C::A_CH ? offa : offb)),
                                                 NNQ_LPTR(buf + (size_t)(j * PTH + pw * 64) * 16), 16, 0, 0);
        };
        const uint8_t *hcsrc;
        {
            const int cc = min(pj, C::NTILE * 16 - 1);
            hcsrc = a.hdr + ((size_t)min(t0 + cc / 16, ntile - 1) * nblk_all + sb0) * 256 + (cc % 16) * 16;
        }
        auto hload = [&](int sb) {
            __builtin_amdgcn_global_load_lds(NNQ_GPTR(hcsrc + (size_t)min(sb, nblk - 1) * 256),
                                             NNQ_LPTR(hdr_lds + (size_t)((sb & 1) * PTH + pw * 64) * 16), 16, 0, 0);
        };
        // dequantization ownership: raw B chunks cb = o * 256 + pj (when < B_CH): tile
        // cb >> 5, plane (cb >> 4) & 1, row cb & 15; the column is tile * 16 + row
        int cbo[NO];
        bool own[NO];
#pragma unroll
        for (int o = 0; o < NO; o++) {
            cbo[o] = min(o * PTH + pj, C::B_CH - 1);
            own[o] = o * PTH + pj < C::B_CH;
        }
        uint32_t scw[NO][2];
        auto decode = [&](int sb) {
#pragma unroll
            for (int o = 0; o < NO; o++) {
                const int col = (cbo[o] >> 5) * 16 + (cbo[o] & 15);
                const u32x4 h = *reinterpret_cast<const u32x4 *>(hdr_lds + (size_t)(sb & 1) * PTH * 16 + col * 16);
                // BlockQ4K header (get_scale_min_k4, crates/nn-core/src/layers/quantized/linear.rs:166-176)
                const uint32_t nzm = (h[0] & 0x7FFFu) != 0u ? 0xFFFFFFFFu : 0u;  // d != 0
                scw[o][0] = h[1] & 0x3F3F3F3Fu & nzm;
                scw[o][1] = ((h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u)) & nzm;
            }
        };
        auto dequant = [&](int s) {  // stage s: raw bytes (ring) -> f16 fragments (buffer s & 1)
            const int p = s & 3;
            const unsigned char *raw = ring + (size_t)(s % NBUF) * C::BUF + C::A_CH * 16;
            unsigned char *dst = f16b + (size_t)(s & 1) * C::F16B;
#pragma unroll
            for (int o = 0; o < NO; o++) {
                if (!own[o]) continue;
                const int cb = cbo[o], t = cb >> 5, h = (cb >> 4) & 1, r = cb & 15;
                const u32x4 w = *reinterpret_cast<const u32x4 *>(raw + cb * 16);
                const uint32_t sw = scw[o][p >> 1];
                const uint32_t sl = f16_pair_int((sw >> (16 * (p & 1))) & 0xFFu);
                const uint32_t sh = f16_pair_int((sw >> (16 * (p & 1) + 8)) & 0xFFu);
#pragma unroll
                for (int half = 0; half < 2; half++) {  // bytes 8 half .. + 7: consumer lane (2h + half) * 16 + r
                    const uint32_t w0 = w[2 * half], w1 = w[2 * half + 1], w0s = w0 >> 8, w1s = w1 >> 8;
                    const int L = (2 * h + half) * 16 + r;
                    const u32x4 lo = {pk_mul_f16(w0 & 0x000F000Fu, sl), pk_mul_f16(w0s & 0x000F000Fu, sl),
                                      pk_mul_f16(w1 & 0x000F000Fu, sl), pk_mul_f16(w1s & 0x000F000Fu, sl)};
                    const u32x4 hi = {pk_mul_f16(w0 & 0x00F000F0u, sh), pk_mul_f16(w0s & 0x00F000F0u, sh),
                                      pk_mul_f16(w1 & 0x00F000F0u, sh), pk_mul_f16(w1s & 0x00F000F0u, sh)};
                    *reinterpret_cast<u32x4 *>(dst + ((t * 2 + 0) * 64 + L) * 16) = lo;
                    *reinterpret_cast<u32x4 *>(dst + ((t * 2 + 1) * 64 + L) * 16) = hi;
                }
            }
        };

        hload(0);
#pragma unroll
        for (int t = -(NBUF - 1); t <= -1; t++) {
            if (t == -1) hload(1);
            issue(t + NBUF - 1);
        }
        wait_vmcnt<(NBUF - 2) * LPT + 1>();  // header 0 and stage 0 (own copies)
        __builtin_amdgcn_s_barrier();        // every producer's header copy is visible
        decode(0);
        dequant(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the f16 fragments are written
        for (int sb = 0; sb < nblk; sb++) {
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int s = 4 * sb + p;
                __builtin_amdgcn_s_barrier();
                if (p == 3) hload(sb + 2);  // into the area of super-block sb: decoded already
                issue(s + NBUF - 1);
                if (ws_batches(p, NBUF) == 1)  // p is a constant once the loop is unrolled
                    wait_vmcnt<(NBUF - 2) * LPT + 1>();
                else
                    wait_vmcnt<(NBUF - 2) * LPT>();
                if (p == 3) decode(sb + 1);  // visible since the barrier of iteration s - 1
                dequant(s + 1);
                __builtin_amdgcn_s_waitcnt(0xC07F);
            }
        }
        wait_vmcnt<0>();
        return;
    }

    // ================================== consumers ==================================
    const int wn = wv;
    const int q = lane >> 4, c16 = lane & 15;
    float ucur[NT], ratio[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) ucur[nt] = 1.0f;
    auto decode_d = [&](int sb) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int col = (wn * NT + nt) * 16 + c16;
            const uint32_t h0 = *reinterpret_cast<const uint32_t *>(hdr_lds + (size_t)(sb & 1) * PTH * 16 + col * 16);
            const float d = f16_to_f32(h0 & 0xFFFFu);
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
    int abase[2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) abase[hf] = (c16 * 8 + ((4 * hf + q) ^ ((c16 >> 1) & 7))) * 16;
    // A fragments of a stage in consumption order f = hf * MT + mt, read D ahead
    constexpr int F = 2 * MT, D = 4;
    auto read_frag = [&](const unsigned char *buf, int f) -> u32x4 {
        return *reinterpret_cast<const u32x4 *>(buf + (f % MT) * 2048 + abase[f / MT]);
    };

    __builtin_amdgcn_s_barrier();  // the producers' prologue barrier
    for (int sb = 0; sb < nblk; sb++) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 4 * sb + p;
            __builtin_amdgcn_s_barrier();  // stage s: copied, dequantized
            const unsigned char *buf = ring + (size_t)(s % NBUF) * C::BUF;
            const unsigned char *fb = f16b + (size_t)(s & 1) * C::F16B;
            u32x4 bfr[2][NT], af[F];
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
                    bfr[hf][nt] = *reinterpret_cast<const u32x4 *>(fb + (((wn * NT + nt) * 2 + hf) * 64 + lane) * 16);
#pragma unroll
            for (int f = 0; f < D; f++) af[f] = read_frag(buf, f);
            if (p == 0) decode_d(sb);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int f = 0; f < F; f++) {
                if (f + D < F) af[f + D] = read_frag(buf, f + D);
                const int hf = f / MT, mt = f % MT;
                if (p == 0 && hf == 0) {  // a new super-block: rescale to its unit first
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[mt][nt][e] *= ratio[nt];
                }
#pragma unroll
                for (int nt = 0; nt < NT; nt++) acc[mt][nt] = mfma16x16x32_f16(af[f], bfr[hf][nt], acc[mt][nt]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // Back to true scale (times 2^-8 * s_n, s_n the column's power of two for the min
    // term, stored in the aux plane), then subtract the min term on the MFMA: A = the
    // staged sub-block sums (hi, lo), B = dmin * m_j * s_n (hi, lo) from the aux plane.
    const float *s_rows = reinterpret_cast<const float *>(a.aux + (size_t)ntile * nblk_all * 512);
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
        msrc[nt] = a.aux + ((size_t)tile * nblk_all + sb0) * 512 + c16 * 16;
    }
    // min-term steps: 32 sub-blocks each (lane group q: the 8 sub-blocks of super-block
    // 4 it + q of this workgroup's range); B two steps ahead, A one step ahead
    const int nsub = K / 32, nit = (nblk + 3) / 4;
    auto load_b = [&](int it, u32x4 (&bh)[NT], u32x4 (&bl)[NT]) {
        const int sb = min(4 * it + q, nblk - 1);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            bh[nt] = ldg128(msrc[nt] + (size_t)sb * 512);
            bl[nt] = ldg128(msrc[nt] + (size_t)sb * 512 + 256);
        }
    };
    auto load_a = [&](int it, u32x4 (&ah)[MT], u32x4 (&al)[MT]) {
        const int sb = sb0 + min(4 * it + q, nblk - 1);
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
        load_b(it + 2, bh1, bl1);  // clamped past the end: unused
        load_a(it + 1, ah, al);
        // sub-blocks past the range (a partial last step) and rows past M contribute zero
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
        const float bcol = (a.bias && KS == 1) ? a.bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t row = m0 + mt * 16 + 4 * q + e;
                if (row >= M) continue;
                const float y = acc[mt][nt][e] * colf[nt] * sc.rowback[row] + bcol;
                if (KS > 1)
                    sc.ysplit[((int64_t)ks * M + row) * a.n + col] = y;
                else if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[row * a.n + col] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[row * a.n + col] = y;
            }
    }
}

// split-K result: the partial slabs summed in order plus the bias, stored as f32 or bf16
__global__ __launch_bounds__(256) void gemm_finalize_kernel(const float *ys, int ks, const float *bias, void *y,
                                                            int y_bf16, int64_t m, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= m * n) return;
    float v = ys[i];
    for (int j = 1; j < ks; j++) v += ys[(int64_t)j * m * n + i];
    v += bias ? bias[i % n] : 0.0f;
    if (y_bf16)
        reinterpret_cast<uint16_t *>(y)[i] = (uint16_t)f32_to_bf16_bits(v);
    else
        reinterpret_cast<float *>(y)[i] = v;
}

template <int BN, int NBUF>
int launch_ws(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    using C = WS<BN, NBUF>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_ws_kernel<BN, NBUF>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const int nct = (int)((a.ntile * 16 + BN - 1) / BN), nrt = (int)((a.m + C::BM - 1) / C::BM);
    hipLaunchKernelGGL((gemm_q4k_ws_kernel<BN, NBUF>), dim3((unsigned)(nct * nrt * sc.ksplit)), dim3(C::NTH), C::LDS,
                       st, a, sc);
    int e = (int)hipGetLastError();
    if (e || sc.ksplit == 1) return e;
    const int64_t cnt = a.m * a.n;
    hipLaunchKernelGGL(gemm_finalize_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, st, sc.ysplit, sc.ksplit,
                       a.bias, a.y, a.y_bf16, a.m, a.n);
    return (int)hipGetLastError();
}

}  // namespace

// Shapes the ring kernel takes (bf16 activations, M >= 128): 128 x 192 tiles when
// N % 192 == 0, else 128 x 128 tiles (N % 128 == 0).  K is split 2 or 4 ways (a
// divisor of the super-block count leaving at least 4 super-blocks per workgroup)
// until there are at least 256 workgroups (one per CU), or as far as it goes.
// Returns the K split, or 0 when the shape does not fit.
int gemm_ring_plan(const GemmArgs &a, int *bn) {
    if (!a.x_bf16 || a.m < 128 || a.nblk < 1) return 0;
    const int64_t ncols = a.ntile * 16, nrt = (a.m + 127) / 128;
    int b = 0;
    if (ncols % 192 == 0)
        b = 192;
    else if (ncols % 128 == 0)
        b = 128;
    else
        return 0;
    if (bn) *bn = b;
    const int64_t wgs = nrt * (ncols / b);
    int best = 1;
    for (int ks = 2; ks <= 4 && wgs * best < 256; ks *= 2)
        if (a.nblk % ks == 0 && a.nblk / ks >= 4) best = ks;
    return best;
}

int launch_gemm_ring(const GemmArgs &a, const GemmScratch &sc, void *stream) {
    int bn = 0;
    const int ksplit = gemm_ring_plan(a, &bn);
    if (ksplit == 0 || sc.ksplit != ksplit || (ksplit > 1 && !sc.ysplit)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    return bn == 192 ? launch_ws<192, 4>(a, sc, st) : launch_ws<128, 4>(a, sc, st);
}

}  // namespace nnq
