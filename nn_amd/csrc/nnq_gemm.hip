// Prefill GEMM for Q4_K weights on gfx950: Y[m, n] = X[m, k] . W[n, k]^T (+ bias),
// f32 accumulation, f32 or bf16 output (QLinear::forward with a batch of tokens,
// crates/nn-core/src/layers/quantized/linear.rs:366-400; the bf16 result dtype
// follows crates/nn-core/src/dyn_tensor/ops/matmul.rs:37-38).
//
// Arithmetic.  A Q4_K weight is w = d*sc_j*q - dmin*m_j (d, dmin f16 per 256-element
// super-block, sc_j / m_j 6-bit per 32-element sub-block, q 4-bit).  The main term
// runs on the 16x16x32 f16 MFMA with B = sc_j*q (an integer <= 945, exact in f16)
// and A = x staged in f16.  The per-super-block factor d is applied without extra
// accumulators: the accumulator of column n is kept in units of u_n, the most recent
// non-zero d of that column, and rescaled by u_prev / u_next when a super-block
// starts (one multiply per accumulator element every 256 k; rounding ~2^-24 per
// step).  The min term dmin*m_j*sum(x over the sub-block) is a GEMM over k/32 run
// after the main loop with both operands split into exact f16 hi + lo parts.
//
// Activation staging (gemm_prep_kernel, once per call): each row of x is scaled by a
// power of two so that max|x| lands in [2^14, 2^15) and converted to f16 (bf16 input
// converts exactly; f32 input is split into hi + lo planes, K-stacked in the MFMA),
// and its 32-element sums are stored negated, as f16 hi + lo of -sum * 2^-8.
//
// Tiling.  A workgroup computes a BM x BN output tile with WGM x WGN waves (wave tile
// WM x WN of 16x16 MFMA tiles).  K advances one super-block (256 k) per stage: the
// staged activation rows and the raw tile16 weight bytes of the stage are copied to
// LDS (the next stage is prefetched into registers during the current compute), each
// wave dequantizes its own B fragments from the raw nibbles (mask into f16-subnormal
// pairs, one packed f16 multiply by the sub-block scale) and reuses each across its
// WM / 16 A rows.
#include <cstdlib>

#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

namespace {

inline size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

// the LDS-ring kernel (nnq_gemm_ring.hip) takes every Q4_K shape its plan accepts
bool use_ring(const GemmArgs &a) { return !a.blk && gemm_ring_plan(a, nullptr) > 0; }

}  // namespace

// scratch layout: xh | xs | rowback | ysplit; base null: offsets from 0 (sizing)
GemmScratch gemm_carve(void *base, const GemmArgs &a, size_t *bytes) {
    const int P = a.x_bf16 ? 1 : 2;
    uint8_t *b = reinterpret_cast<uint8_t *>(base);
    if (gemm_thin_plan(a, nullptr, nullptr)) {
        if (bytes) *bytes = 0;
        return GemmScratch{};
    }
    if (!a.blk && (gemm_skinny_plan(a, nullptr, nullptr) || gemm_wide_plan(a, nullptr))) {
        GemmScratch s{};
        const size_t off = gemm_wide_scratch(a, &s, b);
        if (bytes) *bytes = off;
        return s;
    }
    if (gemm_wide8_plan(a, nullptr)) {
        GemmScratch s{};
        const size_t off = gemm_wide8_scratch(a, &s, b);
        if (bytes) *bytes = off;
        return s;
    }
    size_t off = 0;
    GemmScratch s;
    s.xh = reinterpret_cast<uint16_t *>(b + off);
    off += al256((size_t)P * a.m * a.k * 2);
    s.xs = reinterpret_cast<uint16_t *>(b + off);
    off += al256((size_t)2 * a.m * (a.k / 32) * 2);
    s.rowback = reinterpret_cast<float *>(b + off);
    off += al256((size_t)a.m * 4);
    s.ksplit = a.blk ? gemm_blk_plan(a, nullptr) : (use_ring(a) ? gemm_ring_plan(a, nullptr) : 1);
    // slabs: one per K part; the ring kernel runs f32 activations' two planes as two sets
    const int nslab = s.ksplit * ((!a.blk && !a.x_bf16 && use_ring(a)) ? 2 : 1);
    s.ysplit = nullptr;
    if (nslab > 1) {
        s.ysplit = reinterpret_cast<float *>(b + off);
        off += al256((size_t)nslab * a.m * a.n * 4);
    }
    if (bytes) *bytes = off;
    return s;
}

namespace {

__device__ __forceinline__ void load8(const void *x, int x_bf16, int64_t off, float v[8]) {
    if (x_bf16) {
        const u32x4 w = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(x) + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = bf16_to_f32(w[i] & 0xFFFFu);
            v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        }
    } else {
        const float *p = reinterpret_cast<const float *>(x) + off;
        const floatx4 a = *reinterpret_cast<const floatx4 *>(p), b = *reinterpret_cast<const floatx4 *>(p + 4);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    }
}

__device__ __forceinline__ uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) * __builtin_bit_cast(half2v, b));
}

}  // namespace

// ---------------------------------------------------------------------------------
// Activation staging: one workgroup per row.  NG > 0: the row is read once into
// registers (NG groups of 8 per thread, K <= 2048 NG), its max found, then converted
// from the registers; NG = 0: any K, the row is read twice.
// ---------------------------------------------------------------------------------
template <int P, int NG>
__global__ __launch_bounds__(256) void gemm_prep_kernel(const void *x, int x_bf16, int64_t m, int64_t k,
                                                        GemmScratch sc) {
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    __shared__ float wred[4];
    __shared__ float scale_s;
    const int64_t ng = k / 8;
    const int64_t xoff = row * k;
    constexpr int NR = NG > 0 ? NG : 1;
    float vr[NR][8];
    float amax = 0.0f;
    if (NG > 0) {
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int64_t g = tid + 256 * j;
            if (g < ng) load8(x, x_bf16, xoff + 8 * g, vr[j]);
        }
#pragma unroll
        for (int j = 0; j < NR; j++) {
            if (tid + 256 * j >= ng) break;
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                amax = fmaxf(amax, fabsf(vr[j][i]));
                sum += vr[j][i];
            }
            if (!(fabsf(sum) <= 3.0e38f)) amax = INFINITY;  // NaN / inf in the row
        }
    } else {
        for (int64_t g = tid; g < ng; g += 256) {
            float v[8];
            load8(x, x_bf16, xoff + 8 * g, v);
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                amax = fmaxf(amax, fabsf(v[i]));
                sum += v[i];
            }
            if (!(fabsf(sum) <= 3.0e38f)) amax = INFINITY;
        }
    }
    amax = wave_max(amax);
    if (lane == 0) wred[wv] = amax;
    __syncthreads();
    if (tid == 0) {
        const float mm = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
        float s, back;
        f16_prescale(mm, s, back);
        scale_s = s;
        sc.rowback[row] = back;
    }
    __syncthreads();
    const float s = scale_s;
    uint16_t *xh0 = sc.xh + row * k;
    uint16_t *xh1 = sc.xh + m * k + row * k;
    const int64_t nsub = k / 32;
    // the four lanes of a quad hold one 32-element block (ng is a multiple of 4 and the
    // stride 256 keeps quads aligned), so the DPP sum only reads lanes of the same quad
    auto convert = [&](int64_t g, const float (&v)[8]) {
        u32x4 H, L;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a0 = v[2 * i] * s, a1 = v[2 * i + 1] * s;
            uint32_t h0, l0, h1, l1;
            split_f16(a0, h0, l0);
            split_f16(a1, h1, l1);
            H[i] = h0 | (h1 << 16);
            L[i] = l0 | (l1 << 16);
            sum += a0 + a1;
        }
        *reinterpret_cast<u32x4 *>(xh0 + 8 * g) = H;
        if (P == 2) *reinterpret_cast<u32x4 *>(xh1 + 8 * g) = L;
        float tot = sum + dpp_xor1(sum);
        tot += dpp_xor2(tot);
        if ((g & 3) == 0) {
            uint32_t th, tl;
            split_f16(tot * 0.00390625f, th, tl);  // 2^-8 keeps 32 * 2^15 inside f16
            // stored negated (sign bits flipped, exact): the min term is subtracted
            sc.xs[row * nsub + g / 4] = (uint16_t)(th ^ 0x8000u);
            sc.xs[m * nsub + row * nsub + g / 4] = (uint16_t)(tl ^ 0x8000u);
        }
    };
    if (NG > 0) {
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int64_t g = tid + 256 * j;
            if (g >= ng) break;  // uniform across each quad (ng % 4 == 0)
            convert(g, vr[j]);
        }
    } else {
        for (int64_t g = tid; g < ng; g += 256) {
            float v[8];
            load8(x, x_bf16, xoff + 8 * g, v);
            convert(g, v);
        }
    }
}

// ---------------------------------------------------------------------------------
// Main kernel
// ---------------------------------------------------------------------------------
template <int BM, int BN, int WGM, int WGN, int P>
struct GemmCfg {
    static constexpr int NTH = WGM * WGN * 64;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int MT = WM / 16, NT = WN / 16;
    static constexpr int AST = 264;  // LDS row stride of the staged activation (f16): 256 + 8 pad
    static constexpr int NTILE = BN / 16;
    static constexpr size_t A_BYTES = (size_t)P * BM * AST * 2;
    static constexpr size_t B_BYTES = (size_t)NTILE * 2048;
    static constexpr size_t SCP_BYTES = (size_t)BN * 8 * 4;
    static constexpr size_t LDS = A_BYTES + B_BYTES + SCP_BYTES + 3 * BN * 4;
    static constexpr int ACH = P * BM * 32;  // 16-byte activation chunks per stage
    static constexpr int APT = (ACH + NTH - 1) / NTH;
    static constexpr int BCH = NTILE * 128;  // 16-byte weight chunks per stage
    static constexpr int BPT = (BCH + NTH - 1) / NTH;
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be 16-aligned");
    static_assert(BN <= NTH, "one thread per column decodes the super-block header");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
};

template <int BM, int BN, int WGM, int WGN, int P>
__global__ __launch_bounds__(WGM *WGN * 64) void gemm_q4k_kernel(GemmArgs a, GemmScratch sc) {
    using C = GemmCfg<BM, BN, WGM, WGN, P>;
    constexpr int NTH = C::NTH, MT = C::MT, NT = C::NT, AST = C::AST;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint16_t *As = reinterpret_cast<uint16_t *>(smem);
    uint8_t *Bs = smem + C::A_BYTES;
    uint32_t *scp = reinterpret_cast<uint32_t *>(Bs + C::B_BYTES);  // [BN][8] packed f16 (sc*2^10 | sc*2^6)
    float *ucur = reinterpret_cast<float *>(scp + BN * 8);          // [BN] current unit u_n
    float *ratio = ucur + BN;                                        // [BN] u_prev / u_next
    float *dminmax = ratio + BN;                                     // [BN] max |dmin| so far

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv / WGN, wn = wv % WGN;
    const int p = lane >> 4, l16 = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
    const int64_t t0 = n0 / 16;
    const int64_t K = a.k, M = a.m;

    if (tid < BN) {
        ucur[tid] = 1.0f;
        dminmax[tid] = 0.0f;
    }

    floatx4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    u32x4 ra[C::APT], rb[C::BPT], rh = u32x4{0u, 0u, 0u, 0u};
    const int64_t nstage = a.nblk;

    // global -> registers for super-block sb (activation rows, raw weight bytes, headers)
    auto gload = [&](int64_t sb) {
#pragma unroll
        for (int i = 0; i < C::APT; i++) {
            const int c = tid + i * NTH;
            ra[i] = u32x4{0u, 0u, 0u, 0u};
            if (c < C::ACH) {
                const int pl = c / (BM * 32), rem = c % (BM * 32), row = rem / 32, c16 = rem % 32;
                if (m0 + row < M)
                    ra[i] = *reinterpret_cast<const u32x4 *>(sc.xh + (int64_t)pl * M * K + (m0 + row) * K + sb * 256 +
                                                             c16 * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < C::BPT; i++) {
            const int c = tid + i * NTH;
            rb[i] = u32x4{0u, 0u, 0u, 0u};
            if (c < C::BCH) {
                const int tt = c / 128, w = c % 128;
                if (t0 + tt < a.ntile) rb[i] = ldg128(a.qs + ((t0 + tt) * a.nblk + sb) * 2048 + w * 16);
            }
        }
        if (tid < BN) {
            const int64_t tt = t0 + tid / 16;
            rh = tt < a.ntile ? ldg128(a.hdr + (tt * a.nblk + sb) * 256 + 16 * (tid % 16)) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    // registers -> LDS, and the per-column tables of the super-block
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < C::APT; i++) {
            const int c = tid + i * NTH;
            if (c < C::ACH) {
                const int pl = c / (BM * 32), rem = c % (BM * 32), row = rem / 32, c16 = rem % 32;
                *reinterpret_cast<u32x4 *>(As + (pl * BM + row) * AST + c16 * 8) = ra[i];
            }
        }
#pragma unroll
        for (int i = 0; i < C::BPT; i++) {
            const int c = tid + i * NTH;
            if (c < C::BCH) *reinterpret_cast<u32x4 *>(Bs + c * 16) = rb[i];
        }
        if (tid < BN) {
            // BlockQ4K header: d | dmin, scales[12] (get_scale_min_k4,
            // crates/nn-core/src/layers/quantized/linear.rs:166-176)
            const float d = f16_to_f32(rh[0] & 0xFFFFu), dmin = f16_to_f32(rh[0] >> 16);
            const uint32_t S1 = rh[1], S2 = rh[2], S3 = rh[3];
            const uint32_t sc03 = S1 & 0x3F3F3F3Fu;
            const uint32_t sc47 = (S3 & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
            const float uo = ucur[tid];
            const bool nz = d != 0.0f;
            const float un = nz ? d : uo;
            ucur[tid] = un;
            ratio[tid] = uo / un;
            dminmax[tid] = fmaxf(dminmax[tid], fabsf(dmin));
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t scj = ((j < 4 ? sc03 : sc47) >> (8 * (j & 3))) & 0xFFu;
                // low nibbles are read as q * 2^-24, high nibbles as 16 q * 2^-24
                const float f = nz ? (float)scj * ((j & 1) ? 64.0f : 1024.0f) : 0.0f;
                const uint32_t h = f32_to_f16_bits(f);
                scp[tid * 8 + j] = h | (h << 16);
            }
        }
    };

    gload(0);
    for (int64_t st = 0; st < nstage; st++) {
        __syncthreads();  // the previous stage's fragments have been read
        sstore();
        __syncthreads();
        if (st + 1 < nstage) gload(st + 1);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const float r = ratio[wn * C::WN + nt * 16 + l16];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mt][nt][i] *= r;
        }
#pragma unroll
        for (int g = 0; g < 4; g++) {  // byte group: sub-blocks 2g (low nibbles), 2g + 1 (high)
            u32x4 ae[P][MT], ao[P][MT];
#pragma unroll
            for (int pl = 0; pl < P; pl++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const uint16_t *ar = As + (pl * BM + wm * C::WM + mt * 16 + l16) * AST + 64 * g + 8 * p;
                    ae[pl][mt] = *reinterpret_cast<const u32x4 *>(ar);
                    ao[pl][mt] = *reinterpret_cast<const u32x4 *>(ar + 32);
                }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int cl = wn * C::WN + nt * 16 + l16;
                const u32x2 raw = *reinterpret_cast<const u32x2 *>(Bs + (cl / 16) * 2048 + 1024 * (p >> 1) +
                                                                   16 * (16 * g + l16) + 8 * (p & 1));
                const u32x2 sp = *reinterpret_cast<const u32x2 *>(scp + cl * 8 + 2 * g);
                const uint32_t w0 = raw[0], w1 = raw[1], w0s = w0 >> 8, w1s = w1 >> 8;
                const u32x4 be = {pk_mul_f16(w0 & 0x000F000Fu, sp[0]), pk_mul_f16(w0s & 0x000F000Fu, sp[0]),
                                  pk_mul_f16(w1 & 0x000F000Fu, sp[0]), pk_mul_f16(w1s & 0x000F000Fu, sp[0])};
                const u32x4 bo = {pk_mul_f16(w0 & 0x00F000F0u, sp[1]), pk_mul_f16(w0s & 0x00F000F0u, sp[1]),
                                  pk_mul_f16(w1 & 0x00F000F0u, sp[1]), pk_mul_f16(w1s & 0x00F000F0u, sp[1])};
#pragma unroll
                for (int pl = 0; pl < P; pl++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        acc[mt][nt] = mfma16x16x32_f16(ae[pl][mt], be, acc[mt][nt]);
                        acc[mt][nt] = mfma16x16x32_f16(ao[pl][mt], bo, acc[mt][nt]);
                    }
            }
        }
    }
    __syncthreads();

    // Back to true scale (times 2^-8 * s_n, s_n the column's power-of-two for the min
    // term), then subtract the min term on the MFMA.
    float colf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int cl = wn * C::WN + nt * 16 + l16;
        float s_n, back_n;
        f16_prescale(dminmax[cl] * 63.0f, s_n, back_n);
        const float f = ucur[cl] * 16384.0f * 0.00390625f * s_n;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[mt][nt][i] *= f;
        colf[nt] = 256.0f * back_n;
    }
    const int64_t nsub = K / 32;
    for (int64_t jg0 = 0; jg0 < nsub; jg0 += 32) {
        const int64_t sb = jg0 / 8 + p;  // super-block of this lane's 8 sub-block sums
        const bool kin = sb < a.nblk;
        u32x4 ah[MT], al[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int64_t row = m0 + wm * C::WM + mt * 16 + l16;
            ah[mt] = al[mt] = u32x4{0u, 0u, 0u, 0u};
            if (kin && row < M) {
                // the sums are staged negated: the min term is subtracted
                ah[mt] = *reinterpret_cast<const u32x4 *>(sc.xs + row * nsub + jg0 + 8 * p);
                al[mt] = *reinterpret_cast<const u32x4 *>(sc.xs + M * nsub + row * nsub + jg0 + 8 * p);
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int cl = wn * C::WN + nt * 16 + l16;
            const int64_t tt = t0 + cl / 16;
            u32x4 bh = {0u, 0u, 0u, 0u}, bl = {0u, 0u, 0u, 0u};
            if (kin && tt < a.ntile) {
                const u32x4 h = ldg128(a.hdr + (tt * a.nblk + sb) * 256 + 16 * l16);
                float s_n, back_n;
                f16_prescale(dminmax[cl] * 63.0f, s_n, back_n);
                const float dm = f16_to_f32(h[0] >> 16) * s_n;
                const uint32_t S1 = h[1], S2 = h[2], S3 = h[3];
                const uint32_t mn03 = S2 & 0x3F3F3F3Fu;
                const uint32_t mn47 = ((S3 >> 4) & 0x0F0F0F0Fu) | ((S2 >> 2) & 0x30303030u);
                uint32_t hh[8], ll[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t mj = ((j < 4 ? mn03 : mn47) >> (8 * (j & 3))) & 0xFFu;
                    split_f16(dm * (float)mj, hh[j], ll[j]);  // dmin * m_j * s_n: 17 bits, exact as hi + lo
                }
                (void)S1;
                bh = u32x4{hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16), hh[4] | (hh[5] << 16), hh[6] | (hh[7] << 16)};
                bl = u32x4{ll[0] | (ll[1] << 16), ll[2] | (ll[3] << 16), ll[4] | (ll[5] << 16), ll[6] | (ll[7] << 16)};
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                acc[mt][nt] = mfma16x16x32_f16(ah[mt], bh, acc[mt][nt]);
                acc[mt][nt] = mfma16x16x32_f16(ah[mt], bl, acc[mt][nt]);
                acc[mt][nt] = mfma16x16x32_f16(al[mt], bh, acc[mt][nt]);
            }
        }
    }

    // store: lane holds rows 4p + i of each 16 x 16 tile, column l16
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int64_t col = n0 + wn * C::WN + nt * 16 + l16;
        if (col >= a.n) continue;
        const float bcol = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t row = m0 + wm * C::WM + mt * 16 + 4 * p + i;
                if (row >= M) continue;
                const float y = acc[mt][nt][i] * colf[nt] * sc.rowback[row] + bcol;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[row * a.n + col] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[row * a.n + col] = y;
            }
    }
}

// ---------------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------------
size_t gemm_scratch_bytes(const GemmArgs &a) {
    size_t bytes = 0;
    gemm_carve(nullptr, a, &bytes);
    return bytes;
}

template <int BM, int BN, int WGM, int WGN, int P>
static int launch_cfg(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    using C = GemmCfg<BM, BN, WGM, WGN, P>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_kernel<BM, BN, WGM, WGN, P>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const dim3 grid((unsigned)((a.ntile * 16 + BN - 1) / BN), (unsigned)((a.m + BM - 1) / BM));
    hipLaunchKernelGGL((gemm_q4k_kernel<BM, BN, WGM, WGN, P>), grid, dim3(C::NTH), C::LDS, st, a, sc);
    return (int)hipGetLastError();
}

template <int P>
static int launch_p(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    const int64_t ncols = a.ntile * 16;
    auto wgs = [&](int64_t bm, int64_t bn) { return ((a.m + bm - 1) / bm) * ((ncols + bn - 1) / bn); };
    if (use_ring(a)) return launch_gemm_ring(a, sc, st);
    if constexpr (P == 1) {  // the f32 (hi + lo) staging doubles the activation LDS
        if (a.m >= 128 && ncols % 192 == 0 && wgs(128, 192) >= 256) return launch_cfg<128, 192, 2, 2, P>(a, sc, st);
        if (a.m >= 128 && wgs(128, 128) >= 256) return launch_cfg<128, 128, 2, 2, P>(a, sc, st);
    }
    if (a.m >= 64 && wgs(64, 128) >= 256) return launch_cfg<64, 128, 2, 2, P>(a, sc, st);
    if (a.m >= 64) return launch_cfg<64, 64, 2, 2, P>(a, sc, st);
    return launch_cfg<32, 64, 2, 2, P>(a, sc, st);
}

template <int P, int NG>
static void launch_prep_ng(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    hipLaunchKernelGGL((gemm_prep_kernel<P, NG>), dim3((unsigned)a.m), dim3(256), 0, st, a.x, a.x_bf16, a.m, a.k, sc);
}
// the row in registers when K <= 2048 * 6 (Qwen3-8B: 4096 and 12288)
template <int P>
static void launch_prep(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    const int64_t per = (a.k / 8 + 255) / 256;  // groups of 8 per thread
    if (per <= 2) return launch_prep_ng<P, 2>(a, sc, st);
    if (per <= 6) return launch_prep_ng<P, 6>(a, sc, st);
    return launch_prep_ng<P, 0>(a, sc, st);
}

int launch_gemm_prep(const GemmArgs &a, const GemmScratch &sc, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    if (a.x_bf16)
        launch_prep<1>(a, sc, st);
    else
        launch_prep<2>(a, sc, st);
    return (int)hipGetLastError();
}

int launch_gemm_q4k(const GemmArgs &a, void *stream) {
    if (a.m <= 0) return 0;
    if (gemm_thin_plan(a, nullptr, nullptr)) return launch_gemm_thin(a, stream);
    const GemmScratch sc = gemm_carve(a.scratch, a, nullptr);
    if (gemm_skinny_plan(a, nullptr, nullptr) || gemm_wide_plan(a, nullptr)) return launch_gemm_wide(a, sc, stream);
    hipStream_t st = (hipStream_t)stream;
    int e = launch_gemm_prep(a, sc, st);
    if (e) return e;
    return a.x_bf16 ? launch_p<1>(a, sc, st) : launch_p<2>(a, sc, st);
}

}  // namespace nnq
