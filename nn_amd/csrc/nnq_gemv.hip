// Decode GEMV (m <= 8 tokens) for Q4_K / Q8_0 / Q6_K weights on gfx950.
//
// One workgroup owns a tile of 16 weight rows and all of K.  Its waves split K
// into 256-element units (unit u goes to wave u % WAVES).  Per unit a wave
// issues coalesced 16-byte loads whose bytes are, lane by lane, the B operand
// of a 16x16x32 f16 MFMA (the tile16 repack puts them there), turns nibbles /
// bytes into packed f16 values with one mask per pair (the integer q is read as
// an f16 subnormal q * 2^-24, exact), and multiplies against the activation.
// The activation is staged once per workgroup in LDS as f16 hi + lo parts of
// x * 2^s (s per token, chosen so max|x| lands in [2^14, 2^15)), so the f16 MFMA
// sees x to ~22 significant bits and every product is exact in the f32
// accumulator.  Per-sub-block scales and mins are applied to the MFMA results
// in f32; waves are combined through LDS at the end.
//
// A-operand rows: Q4_K / Q8_0 use rows (2t, 2t+1) = (hi, lo) of token t (8 tokens);
// Q6_K uses rows 4t..4t+3 = (hi, lo) x (first / second 16-value sub-block).
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

enum { FQ4K = 12, FQ80 = 8, FQ6K = 14 };

template <int FMT>
struct Fmt;
template <>
struct Fmt<FQ4K> {
    static constexpr int kMaxTok = 8, kSumGran = 32;
};
template <>
struct Fmt<FQ80> {
    static constexpr int kMaxTok = 8, kSumGran = 32;
};
template <>
struct Fmt<FQ6K> {
    static constexpr int kMaxTok = 4, kSumGran = 16;
};

struct LdsPlan {
    int kc;          // staged K per chunk
    size_t bytes;
};

static inline size_t lds_bytes_for(int mt, int kc, int gran, int waves) {
    size_t stage = (size_t)mt * kc * 4 + (size_t)mt * (kc / gran) * 4;
    size_t red = (size_t)waves * 8 * 16 * 2 * 4;
    return (stage > red ? stage : red) + 64;
}

// ---------------------------------------------------------------------------------
// Activation staging: x[t][k0 .. k0+kc) -> LDS hi/lo f16 planes + sub-block sums.
// ---------------------------------------------------------------------------------
// `kcur` elements are staged (k >= a.k reads as zero: Q8_0 pads to 256), `kc` is the
// plane stride.
template <int GRAN>
__device__ __forceinline__ void stage_x(const GemvArgs &a, int mt, int64_t k0, int kcur, int kc, const float *scl,
                                        uint16_t *xs, float *xsum) {
    const int tid = threadIdx.x, nth = blockDim.x;
    const int per_tok = kcur / 8;
    for (int idx = tid; idx < mt * per_tok; idx += nth) {
        int t = idx / per_tok, g8 = idx - t * per_tok;
        int64_t kk = k0 + 8 * g8;
        float v[8];
        if (kk >= a.k) {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        } else if (a.x_bf16) {
            const uint16_t *xp = (const uint16_t *)a.x + (int64_t)t * a.k + kk;
            u32x4 w = *reinterpret_cast<const u32x4 *>(xp);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[2 * i] = bf16_to_f32(w[i] & 0xFFFFu);
                v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
            }
        } else {
            const float *xp = (const float *)a.x + (int64_t)t * a.k + kk;
            floatx4 w0 = *reinterpret_cast<const floatx4 *>(xp);
            floatx4 w1 = *reinterpret_cast<const floatx4 *>(xp + 4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = w0[i];
                v[4 + i] = w1[i];
            }
        }
        float s = scl[t];
        uint32_t hi[8], lo[8];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            split_f16(v[i] * s, hi[i], lo[i]);
            sum += v[i];
        }
        u32x4 H = {hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)};
        u32x4 L = {lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)};
        *reinterpret_cast<u32x4 *>(xs + ((size_t)t * 2 + 0) * kc + 8 * g8) = H;
        *reinterpret_cast<u32x4 *>(xs + ((size_t)t * 2 + 1) * kc + 8 * g8) = L;
        // sums over GRAN consecutive k: combine GRAN/8 neighbouring lanes
        float tot = sum;
#pragma unroll
        for (int o = 1; o < GRAN / 8; o <<= 1) tot += __shfl_xor(tot, o, 64);
        if ((g8 & (GRAN / 8 - 1)) == 0) xsum[(size_t)t * (kc / GRAN) + g8 / (GRAN / 8)] = tot;
    }
}

// per-token prescale factors 2^s (max over the whole row of x)
__device__ __forceinline__ void token_scales(const GemvArgs &a, int mt, float *scl, float *wred) {
    const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, wv = tid >> 6, nw = nth >> 6;
    for (int t = 0; t < mt; t++) {
        float m = 0.0f;
        if (a.x_bf16) {
            const uint16_t *xp = (const uint16_t *)a.x + (int64_t)t * a.k;
            for (int64_t i = (int64_t)tid * 8; i < a.k; i += (int64_t)nth * 8) {
                u32x4 w = *reinterpret_cast<const u32x4 *>(xp + i);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    m = fmaxf(m, fabsf(bf16_to_f32(w[j] & 0xFFFFu)));
                    m = fmaxf(m, fabsf(bf16_to_f32(w[j] >> 16)));
                }
                // NaN propagation: fmaxf drops NaN, so test explicitly
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (((w[j] & 0x7FFFu) > 0x7F80u) || (((w[j] >> 16) & 0x7FFFu) > 0x7F80u)) m = INFINITY;
            }
        } else {
            const float *xp = (const float *)a.x + (int64_t)t * a.k;
            for (int64_t i = (int64_t)tid * 4; i < a.k; i += (int64_t)nth * 4) {
                floatx4 w = *reinterpret_cast<const floatx4 *>(xp + i);
#pragma unroll
                for (int j = 0; j < 4; j++) m = (fabsf(w[j]) <= m) ? m : (fabsf(w[j]) > m ? fabsf(w[j]) : INFINITY);
            }
        }
        m = wave_max(m);
        if (lane == 0) wred[wv] = m;
        __syncthreads();
        if (tid == 0) {
            float mm = 0.0f;
            for (int i = 0; i < nw; i++) mm = fmaxf(mm, wred[i]);
            scl[t] = f16_prescale(mm);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------
// Per-format unit processing (256 k of one 16-row tile), accumulating
// acc1 (scaled MFMA sums) and acc2 (sub-block-sum terms) for this lane's tokens.
// ---------------------------------------------------------------------------------
struct UnitQ4K {
    u32x4 q0, q1, h;
};
struct UnitQ80 {
    u32x4 q[4];
    u32x4 h;
};
struct UnitQ6K {
    u32x3 q[4];
    u32x4 s;
    uint32_t d;
};

__device__ __forceinline__ void load_unit(const GemvArgs &a, int64_t tile, int64_t unit, UnitQ4K &u) {
    const int lane = threadIdx.x & 63;
    const uint8_t *qb = a.qs + (tile * a.nblk + unit) * 2048 + 16 * lane;
    u.q0 = ldg128(qb);
    u.q1 = ldg128(qb + 1024);
    u.h = ldg128(a.hdr + (tile * a.nblk + unit) * 256 + 16 * (lane & 15));
}
__device__ __forceinline__ void load_unit(const GemvArgs &a, int64_t tile, int64_t unit, UnitQ80 &u) {
    const int lane = threadIdx.x & 63;
    const int64_t npair = a.nblk / 2, ngrp = a.nblk / 8;
#pragma unroll
    for (int i = 0; i < 4; i++) u.q[i] = ldg128(a.qs + (tile * npair + unit * 4 + i) * 1024 + 16 * lane);
    u.h = ldg128(a.hdr + (tile * ngrp + unit) * 256 + 16 * (lane & 15));
}
__device__ __forceinline__ void load_unit(const GemvArgs &a, int64_t tile, int64_t unit, UnitQ6K &u) {
    const int lane = threadIdx.x & 63;
    const uint8_t *qb = a.qs + (tile * a.nblk + unit) * 3072 + 12 * lane;
#pragma unroll
    for (int c = 0; c < 4; c++) u.q[c] = ldg96(qb + 768 * c);
    const uint8_t *hb = a.hdr + (tile * a.nblk + unit) * 288;
    u.s = ldg128(hb + 16 * (lane & 15));
    u.d = *reinterpret_cast<const uint16_t *>(hb + 256 + 2 * (lane & 15));
}

// A operand for the two-rows-per-token layout (Q4_K, Q8_0): row m = lane&15 -> token m>>1, part m&1
__device__ __forceinline__ u32x4 a_operand2(const uint16_t *xs, int kc, int mt, int kk) {
    const int lane = threadIdx.x & 63, m = lane & 15, p = lane >> 4, t = m >> 1, part = m & 1;
    if (t < mt) return *reinterpret_cast<const u32x4 *>(xs + ((size_t)t * 2 + part) * kc + kk + 8 * p);
    return u32x4{0u, 0u, 0u, 0u};
}
// A operand for Q6_K: row m -> token m>>2, half (m>>1)&1 selects which 16-k sub-block, part m&1
__device__ __forceinline__ u32x4 a_operand4(const uint16_t *xs, int kc, int mt, int kk) {
    const int lane = threadIdx.x & 63, m = lane & 15, p = lane >> 4, t = m >> 2, part = m & 1, half = (m >> 1) & 1;
    if (t < mt && (p >> 1) == half)
        return *reinterpret_cast<const u32x4 *>(xs + ((size_t)t * 2 + part) * kc + kk + 8 * p);
    return u32x4{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ void compute_unit(const UnitQ4K &u, const uint16_t *xs, const float *xsum, int kc, int mt,
                                             int kk, float acc1[2], float acc2[2]) {
    const int g = (threadIdx.x & 63) >> 4;
    // header: d | dmin, scales[0..3], scales[4..7], scales[8..11] (BlockQ4K packing)
    const float d = f16_to_f32(u.h[0] & 0xFFFFu), dmin = f16_to_f32(u.h[0] >> 16);
    const uint32_t S1 = u.h[1], S2 = u.h[2], S3 = u.h[3];
    const uint32_t sc03 = S1 & 0x3F3F3F3Fu, mn03 = S2 & 0x3F3F3F3Fu;
    const uint32_t sc47 = (S3 & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    const uint32_t mn47 = ((S3 >> 4) & 0x0F0F0F0Fu) | ((S2 >> 2) & 0x30303030u);
    float t1e[2] = {0.f, 0.f}, t1o[2] = {0.f, 0.f}, t2[2] = {0.f, 0.f};
    const float *xs0 = xsum + (size_t)(2 * g) * (kc / 32) + kk / 32;
    const float *xs1 = xsum + (size_t)(2 * g + 1) * (kc / 32) + kk / 32;
    const bool tok0 = 2 * g < mt, tok1 = 2 * g + 1 < mt;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const u32x4 q = h ? u.q1 : u.q0;
        const uint32_t scb = h ? sc47 : sc03, mnb = h ? mn47 : mn03;
#pragma unroll
        for (int gg = 0; gg < 2; gg++) {
            const uint32_t w0 = q[2 * gg], w1 = q[2 * gg + 1];
            const uint32_t w0s = w0 >> 8, w1s = w1 >> 8;
            const u32x4 blo = {w0 & 0x000F000Fu, w0s & 0x000F000Fu, w1 & 0x000F000Fu, w1s & 0x000F000Fu};
            const u32x4 bhi = {w0 & 0x00F000F0u, w0s & 0x00F000F0u, w1 & 0x00F000F0u, w1s & 0x00F000F0u};
            const int jl = 4 * h + 2 * gg, jh = jl + 1;  // sub-block indices (low / high nibbles)
            const int klo = kk + 64 * (2 * h + gg), khi = klo + 32;
            floatx4 cl = mfma16x16x32_f16(a_operand2(xs, kc, mt, klo), blo, floatx4{0.f, 0.f, 0.f, 0.f});
            floatx4 ch = mfma16x16x32_f16(a_operand2(xs, kc, mt, khi), bhi, floatx4{0.f, 0.f, 0.f, 0.f});
            const float scl = (float)((scb >> (16 * gg)) & 0xFFu), sch = (float)((scb >> (16 * gg + 8)) & 0xFFu);
            const float mnl = (float)((mnb >> (16 * gg)) & 0xFFu), mnh = (float)((mnb >> (16 * gg + 8)) & 0xFFu);
            t1e[0] += scl * (cl[0] + cl[1]);
            t1e[1] += scl * (cl[2] + cl[3]);
            t1o[0] += sch * (ch[0] + ch[1]);
            t1o[1] += sch * (ch[2] + ch[3]);
            const float x0l = tok0 ? xs0[jl] : 0.f, x0h = tok0 ? xs0[jh] : 0.f;
            const float x1l = tok1 ? xs1[jl] : 0.f, x1h = tok1 ? xs1[jh] : 0.f;
            t2[0] += mnl * x0l + mnh * x0h;
            t2[1] += mnl * x1l + mnh * x1h;
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        acc1[i] += d * (t1e[i] + 0.0625f * t1o[i]);
        acc2[i] += dmin * t2[i];
    }
}

__device__ __forceinline__ void compute_unit(const UnitQ80 &u, const uint16_t *xs, const float *xsum, int kc, int mt,
                                             int kk, float acc1[2], float acc2[2]) {
    const int g = (threadIdx.x & 63) >> 4;
    const float *xs0 = xsum + (size_t)(2 * g) * (kc / 32) + kk / 32;
    const float *xs1 = xsum + (size_t)(2 * g + 1) * (kc / 32) + kk / 32;
    const bool tok0 = 2 * g < mt, tok1 = 2 * g + 1 < mt;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
            const int j = 2 * i + hb;  // block within the unit
            const uint32_t w0 = u.q[i][2 * hb] ^ 0x80808080u, w1 = u.q[i][2 * hb + 1] ^ 0x80808080u;
            const u32x4 b = {w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu, (w1 >> 8) & 0x00FF00FFu};
            floatx4 c = mfma16x16x32_f16(a_operand2(xs, kc, mt, kk + 32 * j), b, floatx4{0.f, 0.f, 0.f, 0.f});
            const float dj = f16_to_f32((u.h[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
            acc1[0] += dj * (c[0] + c[1]);
            acc1[1] += dj * (c[2] + c[3]);
            acc2[0] += dj * (tok0 ? xs0[j] : 0.f);
            acc2[1] += dj * (tok1 ? xs1[j] : 0.f);
        }
    }
}

__device__ __forceinline__ void compute_unit(const UnitQ6K &u, const uint16_t *xs, const float *xsum, int kc, int mt,
                                             int kk, float acc1[2], float acc2[2]) {
    const int g = (threadIdx.x & 63) >> 4;  // token of this lane group
    const bool tok = g < mt;
    const float *xsg = xsum + (size_t)g * (kc / 16) + kk / 16;
    const float d = f16_to_f32(u.d);
    float t1 = 0.f, t2 = 0.f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t A = u.q[c][0], B = u.q[c][1], C = u.q[c][2];
        const u32x4 ba = {((A)&0x000F000Fu) | ((C << 4) & 0x00300030u),
                          ((A >> 4) & 0x000F000Fu) | ((C << 2) & 0x00300030u),
                          ((A >> 8) & 0x000F000Fu) | ((C)&0x00300030u),
                          ((A >> 12) & 0x000F000Fu) | ((C >> 2) & 0x00300030u)};
        const u32x4 bb = {((B)&0x000F000Fu) | ((C >> 4) & 0x00300030u),
                          ((B >> 4) & 0x000F000Fu) | ((C >> 6) & 0x00300030u),
                          ((B >> 8) & 0x000F000Fu) | ((C >> 8) & 0x00300030u),
                          ((B >> 12) & 0x000F000Fu) | ((C >> 10) & 0x00300030u)};
        floatx4 ca = mfma16x16x32_f16(a_operand4(xs, kc, mt, kk + 64 * c), ba, floatx4{0.f, 0.f, 0.f, 0.f});
        floatx4 cb = mfma16x16x32_f16(a_operand4(xs, kc, mt, kk + 64 * c + 32), bb, floatx4{0.f, 0.f, 0.f, 0.f});
        // sub-blocks 4c .. 4c+3 of this 256-value block
        const uint32_t sw = u.s[c];
        const float s0 = (float)(int8_t)(sw & 0xFF), s1 = (float)(int8_t)((sw >> 8) & 0xFF);
        const float s2 = (float)(int8_t)((sw >> 16) & 0xFF), s3 = (float)(int8_t)(sw >> 24);
        t1 += s0 * (ca[0] + ca[1]) + s1 * (ca[2] + ca[3]) + s2 * (cb[0] + cb[1]) + s3 * (cb[2] + cb[3]);
        if (tok) t2 += s0 * xsg[4 * c] + s1 * xsg[4 * c + 1] + s2 * xsg[4 * c + 2] + s3 * xsg[4 * c + 3];
    }
    acc1[0] += d * t1;
    acc2[0] += d * t2;
}

template <int FMT>
struct UnitOf;
template <>
struct UnitOf<FQ4K> {
    using T = UnitQ4K;
};
template <>
struct UnitOf<FQ80> {
    using T = UnitQ80;
};
template <>
struct UnitOf<FQ6K> {
    using T = UnitQ6K;
};

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    uint32_t b = __float_as_uint(v);
    uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

template <int FMT, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    using Unit = typename UnitOf<FMT>::T;
    constexpr int GRAN = Fmt<FMT>::kSumGran;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t tile = blockIdx.x;
    const int mt = (int)a.m;
    const int kc = a.kc;
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)mt * kc * 4);
    __shared__ float scl[8];
    __shared__ float wred[WAVES];

    const int64_t kpad = a.nblk * (FMT == FQ80 ? 32 : 256);  // K rounded up to whole 256-element units

    // issue the first unit's weight loads before touching x
    Unit cur;
    int kcur0 = (int)(kpad < kc ? kpad : kc);
    if (wv < kcur0 / 256) load_unit(a, tile, wv, cur);

    token_scales(a, mt, scl, wred);

    float acc1[2] = {0.f, 0.f}, acc2[2] = {0.f, 0.f};
    for (int64_t k0 = 0; k0 < kpad; k0 += kc) {
        const int kcur = (int)((kpad - k0) < kc ? (kpad - k0) : kc);
        const int64_t u0 = k0 / 256;
        const int ucnt = kcur / 256;
        if (k0 > 0 && wv < ucnt) load_unit(a, tile, u0 + wv, cur);
        __syncthreads();
        stage_x<GRAN>(a, mt, k0, kcur, kc, scl, xs, xsum);
        __syncthreads();
        for (int ul = wv; ul < ucnt; ul += WAVES) {
            Unit nxt;
            const bool has = ul + WAVES < ucnt;
            if (has) load_unit(a, tile, u0 + ul + WAVES, nxt);
            compute_unit(cur, xs, xsum, kc, mt, ul * 256, acc1, acc2);
            if (has) cur = nxt;
        }
    }
    __syncthreads();

    // combine waves: red[w][slot][n], slot = token
    float *red1 = reinterpret_cast<float *>(smem);
    float *red2 = red1 + WAVES * 8 * 16;
    const int g = lane >> 4, n = lane & 15;
    if (FMT == FQ6K) {
        red1[(wv * 8 + g) * 16 + n] = acc1[0];
        red2[(wv * 8 + g) * 16 + n] = acc2[0];
    } else {
        red1[(wv * 8 + 2 * g) * 16 + n] = acc1[0];
        red1[(wv * 8 + 2 * g + 1) * 16 + n] = acc1[1];
        red2[(wv * 8 + 2 * g) * 16 + n] = acc2[0];
        red2[(wv * 8 + 2 * g + 1) * 16 + n] = acc2[1];
    }
    __syncthreads();
    if (tid < mt * 16) {
        const int t = tid >> 4, nn = tid & 15;
        float s1 = 0.f, s2 = 0.f;
        for (int w = 0; w < WAVES; w++) {
            s1 += red1[(w * 8 + t) * 16 + nn];
            s2 += red2[(w * 8 + t) * 16 + nn];
        }
        const float back = 16777216.0f / scl[t];  // 2^(24 - s)
        const float bias_k = FMT == FQ4K ? 1.0f : (FMT == FQ80 ? 128.0f : 32.0f);
        float y = s1 * back - bias_k * s2;
        const int64_t row = tile * 16 + nn;
        if (row < a.n) {
            if (a.bias) y += a.bias[row];
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
            else
                reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
        }
        if (a.argmax_partial && t == 0) {
            // first-index argmax of this tile's 16 logits (row-major order), NaN -> max key
            uint64_t key = row < a.n ? (y != y ? ~0ull : argmax_key(y, (uint32_t)row)) : 0ull;
            for (int o = 8; o > 0; o >>= 1) {
                uint64_t other = __shfl_xor(key, o, 16);
                key = other > key ? other : key;
            }
            if (nn == 0) a.argmax_partial[tile] = key;
        }
    }
}

// ---------------------------------------------------------------------------------
// Bit-exact dequantization from the device layout (the parity gate for decode).
// One wave per (tile, unit); lane l = 16p + n decodes its bytes for row n.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_q4k_kernel(const uint8_t *qs, const uint8_t *hdr, int64_t n, int64_t k,
                                                          int64_t ntile, int64_t nblk, float *out) {
    const int lane = threadIdx.x & 63;
    const int64_t job = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= ntile * nblk) return;
    const int64_t tile = job / nblk, b = job % nblk;
    const int r = lane & 15, p = lane >> 4;
    const int64_t row = tile * 16 + r;
    const uint8_t *qb = qs + job * 2048 + 16 * lane;
    const u32x4 h = ldg128(hdr + job * 256 + 16 * r);
    if (row >= n) return;
    const float d = f16_to_f32(h[0] & 0xFFFFu), dmin = f16_to_f32(h[0] >> 16);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(&h) + 4;
    float *o = out + row * k + b * 256;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const u32x4 q = ldg128(qb + 1024 * hh);
#pragma unroll
        for (int gg = 0; gg < 2; gg++) {
            const int gidx = 2 * hh + gg;
            int jl = 2 * gidx, jh = jl + 1;
            uint32_t scl, ml, sch, mh;
            // get_scale_min_k4 (crates/nn-core/src/layers/quantized/linear.rs:166-176)
            auto gsm = [&](int j, uint32_t &s, uint32_t &m) {
                if (j < 4) {
                    s = sb[j] & 63;
                    m = sb[j + 4] & 63;
                } else {
                    s = (sb[j + 4] & 0xF) | ((sb[j - 4] >> 6) << 4);
                    m = (sb[j + 4] >> 4) | ((sb[j] >> 6) << 4);
                }
            };
            gsm(jl, scl, ml);
            gsm(jh, sch, mh);
            const float d1 = d * (float)scl, m1 = dmin * (float)ml;
            const float d2 = d * (float)sch, m2 = dmin * (float)mh;
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const uint32_t word = q[2 * gg + w];
                // stored byte order (e0, e2, e1, e3) of elements i0..i0+3
                const uint32_t e[4] = {word & 0xFF, (word >> 16) & 0xFF, (word >> 8) & 0xFF, word >> 24};
                const int i0 = 8 * p + 4 * w;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    o[64 * gidx + i0 + c] = d1 * (float)(e[c] & 0xF) - m1;
                    o[64 * gidx + 32 + i0 + c] = d2 * (float)(e[c] >> 4) - m2;
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void dequant_q80_kernel(const uint8_t *qs, const uint8_t *hdr, int64_t n, int64_t k,
                                                          int64_t ntile, int64_t nblk, float *out) {
    // one wave per (tile, block pair)
    const int lane = threadIdx.x & 63;
    const int64_t npair = nblk / 2, ngrp = nblk / 8;
    const int64_t job = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= ntile * npair) return;
    const int64_t tile = job / npair, bp = job % npair;
    const int r = lane & 15, p = lane >> 4;
    const int64_t row = tile * 16 + r;
    const u32x4 q = ldg128(qs + job * 1024 + 16 * lane);
    const u32x4 h = ldg128(hdr + (tile * ngrp + bp / 4) * 256 + 16 * r);
    if (row >= n) return;
    const int64_t nb = k / 32;
#pragma unroll
    for (int hb = 0; hb < 2; hb++) {
        const int64_t blk = 2 * bp + hb;
        if (blk >= nb) continue;
        const int jj = (int)(blk % 8);
        const float dj = f16_to_f32((h[jj >> 1] >> (16 * (jj & 1))) & 0xFFFFu);
        float *o = out + row * k + blk * 32 + 8 * p;
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t word = q[2 * hb + w];
            const uint32_t e[4] = {word & 0xFF, (word >> 16) & 0xFF, (word >> 8) & 0xFF, word >> 24};
#pragma unroll
            for (int c = 0; c < 4; c++) o[4 * w + c] = dj * (float)(int8_t)e[c];
        }
    }
}

__global__ __launch_bounds__(256) void dequant_q6k_kernel(const uint8_t *qs, const uint8_t *hdr, int64_t n, int64_t k,
                                                          int64_t ntile, int64_t nblk, float *out) {
    const int lane = threadIdx.x & 63;
    const int64_t job = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= ntile * nblk) return;
    const int64_t tile = job / nblk, b = job % nblk;
    const int r = lane & 15, p = lane >> 4;
    const int64_t row = tile * 16 + r;
    const uint8_t *hb = hdr + job * 288;
    if (row >= n) return;
    const float d = f16_to_f32(*reinterpret_cast<const uint16_t *>(hb + 256 + 2 * r));
    const int8_t *sc = reinterpret_cast<const int8_t *>(hb + 16 * r);
    float *o = out + row * k + b * 256;
    for (int c = 0; c < 4; c++) {
        const u32x3 q = ldg96(qs + (job * 4 + c) * 768 + 12 * lane);
        for (int s = 0; s < 16; s++) {
            const int j = s / 2, which = s % 2, jj = j % 4;
            const uint32_t src = j < 4 ? q[0] : q[1];
            const uint32_t nib = (src >> (4 * jj + 16 * which)) & 0xF;
            const uint32_t crumb = (q[2] >> (2 * j + 16 * which)) & 0x3;
            const int q6 = (int)(nib | (crumb << 4));
            const int kk = s < 8 ? 64 * c + 8 * p + s : 64 * c + 32 + 8 * p + (s - 8);
            // dequantize_q6_k: (d * sc) * (q6 - 32), crates/nn-gguf/src/dequant.rs:453
            const float ds = d * (float)sc[kk / 16];
            o[kk] = ds * (float)(q6 - 32);
        }
    }
}

__global__ void argmax_final_kernel(const unsigned long long *partial, int64_t count, uint32_t *idx,
                                    int32_t *status) {
    __shared__ unsigned long long red[16];
    unsigned long long key = 0;
    for (int64_t i = threadIdx.x; i < count; i += blockDim.x) key = partial[i] > key ? partial[i] : key;
    for (int o = 32; o > 0; o >>= 1) {
        unsigned long long other = __shfl_xor(key, o, 64);
        key = other > key ? other : key;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long k = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) k = red[i] > k ? red[i] : k;
        const bool nan = (k == ~0ull);
        *idx = nan ? 0u : 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu);
        if (status) *status = nan ? NNQ_ERR_NON_FINITE : NNQ_OK;
    }
}

// standalone argmax over a device f32 vector: per-block keys then final reduce
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *v, int64_t n, unsigned long long *partial) {
    __shared__ unsigned long long red[4];
    unsigned long long key = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        float x = v[i];
        unsigned long long kx = x != x ? ~0ull : argmax_key(x, (uint32_t)i);
        key = kx > key ? kx : key;
    }
    for (int o = 32; o > 0; o >>= 1) {
        unsigned long long other = __shfl_xor(key, o, 64);
        key = other > key ? other : key;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long k = red[0];
        for (int i = 1; i < 4; i++) k = red[i] > k ? red[i] : k;
        partial[blockIdx.x] = k;
    }
}

// ---------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------
template <int FMT, int WAVES>
static int launch_gemv_t(const GemvArgs &a0, void *stream) {
    GemvArgs a = a0;
    const int mt = (int)a.m;
    // largest K chunk (multiple of 256) whose staging fits in 64 KB
    const int64_t kpad = a.nblk * (FMT == FQ80 ? 32 : 256);
    int kc = (int)((65536 / ((size_t)mt * (4 + 4 * 1.0 / Fmt<FMT>::kSumGran))) / 256 * 256);
    if (kc < 256) kc = 256;
    if (kc > kpad) kc = (int)kpad;
    a.kc = kc;
    size_t lds = lds_bytes_for(mt, kc, Fmt<FMT>::kSumGran, WAVES);
    hipLaunchKernelGGL((gemv_kernel<FMT, WAVES>), dim3((unsigned)a.ntile), dim3(WAVES * 64), lds,
                       (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_gemv(int fmt, const GemvArgs &a, void *stream) {
    // fewer waves when K is short so that every wave owns at least one unit
    const int64_t units = (a.k + 255) / 256;
    switch (fmt) {
    case FQ4K:
        if (units >= 16) return launch_gemv_t<FQ4K, 16>(a, stream);
        if (units >= 8) return launch_gemv_t<FQ4K, 8>(a, stream);
        return launch_gemv_t<FQ4K, 4>(a, stream);
    case FQ80:
        if (units >= 16) return launch_gemv_t<FQ80, 16>(a, stream);
        if (units >= 8) return launch_gemv_t<FQ80, 8>(a, stream);
        return launch_gemv_t<FQ80, 4>(a, stream);
    case FQ6K:
        if (units >= 16) return launch_gemv_t<FQ6K, 16>(a, stream);
        if (units >= 8) return launch_gemv_t<FQ6K, 8>(a, stream);
        return launch_gemv_t<FQ6K, 4>(a, stream);
    }
    return (int)hipErrorInvalidValue;
}

int launch_dequant(int fmt, const uint8_t *qs, const uint8_t *hdr, int64_t n, int64_t k, int64_t ntile, int64_t nblk,
                   float *out, void *stream) {
    int64_t jobs = 0;
    switch (fmt) {
    case FQ4K:
        jobs = ntile * nblk;
        hipLaunchKernelGGL(dequant_q4k_kernel, dim3((unsigned)((jobs + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                           qs, hdr, n, k, ntile, nblk, out);
        break;
    case FQ80:
        jobs = ntile * (nblk / 2);
        hipLaunchKernelGGL(dequant_q80_kernel, dim3((unsigned)((jobs + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                           qs, hdr, n, k, ntile, nblk, out);
        break;
    case FQ6K:
        jobs = ntile * nblk;
        hipLaunchKernelGGL(dequant_q6k_kernel, dim3((unsigned)((jobs + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                           qs, hdr, n, k, ntile, nblk, out);
        break;
    default:
        return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int launch_argmax_final(const unsigned long long *partial, int64_t count, uint32_t *idx, int32_t *status,
                        void *stream) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, partial, count, idx, status);
    return (int)hipGetLastError();
}

int launch_argmax_reduce(const float *v, int64_t n, uint32_t *idx, int32_t *status, void *scratch,
                         size_t scratch_bytes, void *stream) {
    int64_t blocks = (n + 255) / 256;
    int64_t cap = (int64_t)(scratch_bytes / sizeof(unsigned long long));
    if (blocks > 1024) blocks = 1024;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) return (int)hipErrorInvalidValue;
    unsigned long long *partial = reinterpret_cast<unsigned long long *>(scratch);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, v, n, partial);
    int e = (int)hipGetLastError();
    if (e) return e;
    return launch_argmax_final(partial, blocks, idx, status, stream);
}

}  // namespace nnq
