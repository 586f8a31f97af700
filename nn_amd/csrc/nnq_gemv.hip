// Decode GEMV (up to 8 tokens per launch: Q4_K and Q6_K 4, Q8_0 8) for Q4_K / Q8_0 / Q6_K
// weights on gfx950.
//
// One workgroup owns a tile of 16 weight rows.  Its waves split K into units (256
// elements; 8 blocks for Q8_0) and issue the activation slices and the weight loads of
// all their units of a pass up front, so a whole K pass of the tile is in flight at
// once.  Per unit a wave's coalesced loads are, lane by lane, the B operand of a
// 16x16x32 f16 MFMA (the tile16 repack puts them there); nibbles / bytes become packed
// f16 values with one mask per pair (the integer q is read as an f16 subnormal
// q * 2^-24, exact) and are multiplied against the activation.
// The decode kernels stage each unit's activation slice in a wave-private LDS buffer as
// f16 hi + lo parts of x * 2^s (s per token and 32-element block, chosen so the block's
// max|x| lands in [2^14, 2^15)), so the f16 MFMA sees x to ~22 significant bits and every
// product is exact in the f32 accumulator; the blocks' powers of two and sums of x stay
// in registers (wave-uniform scalars) or, for batches, in a small per-wave LDS table.
// Scales and mins are applied to the MFMA results in f32; waves meet in LDS at the end.
// The streaming kernels (many tiles per CU: the LM head, the fused gate | up) stage the
// activation once per workgroup and loop over tiles.
//
// A-operand rows: Q4_K / Q8_0 use rows (2t, 2t+1) = (hi, lo) of token t;
// Q6_K uses rows 4t..4t+3 = (hi, lo) x (first / second 16-value sub-block).
#include <algorithm>

#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

// silu(g) * u for four f32 values (g, u as raw bits): SiLU as x / (1 + e^-x)
// (crates/nn-core/src/dyn_tensor/ops/math.rs:140), the product in f32, as
// Qwen3MLP::forward (crates/nn-qwen3/src/layers.rs:40-47) forms it.
__device__ __forceinline__ u32x4 swiglu4(const u32x4 &g, const u32x4 &u) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float gv = __uint_as_float(g[i]);
        r[i] = __float_as_uint(gv / (1.0f + expf(-gv)) * __uint_as_float(u[i]));
    }
    return r;
}

// Output status of a GEMV pass: mode 1 clears it (one thread of the grid), mode 2
// flags a non-finite output (every writer stores the same value).
__device__ __forceinline__ void gemv_status(const GemvArgs &a, float y, bool first) {
    if (a.status_mode == 1 && first) *a.status = NNQ_OK;
    if (a.status_mode == 2 && !(fabsf(y) <= 3.402823466e38f)) *a.status = NNQ_ERR_NON_FINITE;
}

// SwiGLU epilogue of a gate | up GEMV whose 16-row tiles hold 8 gate rows and then the
// 8 matching up rows: the 16 lanes of a tile (nn = row in tile) exchange halves, and
// lane nn < 8 stores silu(gate) * up (f32, as Qwen3MLP::forward, crates/nn-qwen3/src/
// layers.rs:40-47) at column 8 * tile + nn of y [m, n / 2].  Every lane of the 16 calls it.
__device__ __forceinline__ void store_swiglu_pair(const GemvArgs &a, float y, int t, int64_t tile, int nn,
                                                  bool first) {
    const float other = __shfl_xor(y, 8, 16);
    if (a.status_mode == 1 && first) *a.status = NNQ_OK;
    if (nn < 8) {
        const float h = y / (1.0f + expf(-y)) * other;
        if (a.status_mode == 2 && !(fabsf(h) <= 3.402823466e38f)) *a.status = NNQ_ERR_NON_FINITE;
        const int64_t col = tile * 8 + nn, cols = a.n / 2;
        if (a.y_bf16)
            reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * cols + col] = (uint16_t)f32_to_bf16_bits(h);
        else
            reinterpret_cast<float *>(a.y)[(int64_t)t * cols + col] = h;
    }
}

enum { FQ4K = 12, FQ80 = 8, FQ6K = 14 };

template <int FMT>
struct Fmt;
template <>
struct Fmt<FQ4K> {
    static constexpr int kSumGran = 32;
};
template <>
struct Fmt<FQ80> {
    static constexpr int kSumGran = 32;
};
template <>
struct Fmt<FQ6K> {
    static constexpr int kSumGran = 16;
};

// Largest number of 8-element activation groups one thread stages per chunk.
constexpr int kXGroups = 3;

// ---------------------------------------------------------------------------------
// Activation staging: x[t][k0 .. k0+kc) -> LDS hi/lo f16 planes of x * 2^s(t,b),
// sums of the unscaled x over GRAN consecutive k, and the factor 2^-s(t,b) of every
// 32-element block b (four consecutive lanes hold one block of one token, so its
// max is two DPP steps away and no whole-row pass over x is needed).  Staging is
// split in two: the raw loads (issued before the weight loads of the chunk, so that
// waiting for them does not wait for the weights) and the conversion.
// ---------------------------------------------------------------------------------
struct XRaw {
    u32x4 r[kXGroups][2];
    int t[kXGroups], g8[kXGroups];
    bool valid[kXGroups];  // the group exists in this chunk
    bool in[kXGroups];     // ... and lies inside x (Q8_0 pads K to whole 256-element units)
};

// Every thread issues the same two 16-byte loads per group whatever the group's
// validity (out-of-range groups read x[0]; bf16 reads its one vector twice), so the
// load sequence is branch-free and the wait for these loads does not extend to the
// weight loads issued after them.
__device__ __forceinline__ void stage_x_load(const GemvArgs &a, int mt, int64_t k0, int kcur, float inv_per_tok,
                                             XRaw &raw) {
    const int tid = threadIdx.x, nth = blockDim.x;
    const int per_tok = kcur / 8;
#pragma unroll
    for (int j = 0; j < kXGroups; j++) {
        const int idx = tid + j * nth;
        const bool valid = idx < mt * per_tok;
        // idx / per_tok without an integer division (exact: idx < 2^15, per_tok >= 32)
        const int t = valid ? (int)(((float)idx + 0.5f) * inv_per_tok) : 0;
        const int g8 = valid ? idx - t * per_tok : 0;
        const int64_t kk = k0 + 8 * g8;
        raw.valid[j] = valid;
        raw.t[j] = t;
        raw.g8[j] = g8;
        raw.in[j] = valid && kk < a.k;
        const int64_t off = raw.in[j] ? (int64_t)t * a.k + kk : 0;
        const uint8_t *p0 = reinterpret_cast<const uint8_t *>(a.x) + off * (a.x_bf16 ? 2 : 4);
        const uint8_t *p1 = a.x_bf16 ? p0 : p0 + 16;
        raw.r[j][0] = *reinterpret_cast<const u32x4 *>(p0);
        raw.r[j][1] = *reinterpret_cast<const u32x4 *>(p1);
    }
}

template <int GRAN, bool PADDED>
__device__ __forceinline__ void stage_x_store(const GemvArgs &a, int kc, const XRaw &raw, uint16_t *xs, float *xsum,
                                              float *backs) {
#pragma unroll
    for (int j = 0; j < kXGroups; j++) {
        // the four lanes of one 32-element block are all valid or all invalid (mt * per_tok
        // is a multiple of 32 groups and nth a multiple of 64), so the DPP steps below only
        // read active lanes; waves without a valid group skip the conversion
        if (!raw.valid[j]) continue;
        float v[8];
        if (a.x_bf16) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[2 * i] = bf16_to_f32(raw.r[j][0][i] & 0xFFFFu);
                v[2 * i + 1] = bf16_to_f32(raw.r[j][0][i] >> 16);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = __uint_as_float(raw.r[j][0][i]);
                v[4 + i] = __uint_as_float(raw.r[j][1][i]);
            }
        }
        if (PADDED) {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = raw.in[j] ? v[i] : 0.0f;
        }
        float amax = 0.0f, sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            amax = fmaxf(amax, fabsf(v[i]));
            sum += v[i];
        }
        if (!(fabsf(sum) <= 3.0e38f)) amax = INFINITY;  // NaN / inf in this group
        amax = fmaxf(amax, dpp_xor1(amax));
        amax = fmaxf(amax, dpp_xor2(amax));
        float s, back;
        f16_prescale(amax, s, back);
        u32x4 H, L;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t h0, l0, h1, l1;
            split_f16(v[2 * i] * s, h0, l0);
            split_f16(v[2 * i + 1] * s, h1, l1);
            H[i] = h0 | (h1 << 16);
            L[i] = l0 | (l1 << 16);
        }
        float tot = sum + dpp_xor1(sum);
        if (GRAN == 32) tot += dpp_xor2(tot);
        {
            const int t = raw.t[j], g8 = raw.g8[j];
            *reinterpret_cast<u32x4 *>(xs + ((size_t)t * 2 + 0) * kc + 8 * g8) = H;
            *reinterpret_cast<u32x4 *>(xs + ((size_t)t * 2 + 1) * kc + 8 * g8) = L;
            if ((g8 & (GRAN / 8 - 1)) == 0) xsum[(size_t)t * (kc / GRAN) + g8 / (GRAN / 8)] = tot;
            if ((g8 & 3) == 0) backs[t * (kc / 32) + g8 / 4] = back;
        }
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
__device__ __forceinline__ void compute_unit(const UnitQ80 &u, const uint16_t *xs, const float *xsum, int kc, int mt,
                                             int kk, const float *bku, float acc1[2], float acc2[2]) {
    const int g = (threadIdx.x & 63) >> 4;
    const float *xs0 = xsum + (size_t)(2 * g) * (kc / 32) + kk / 32;
    const float *xs1 = xsum + (size_t)(2 * g + 1) * (kc / 32) + kk / 32;
    const bool tok0 = 2 * g < mt, tok1 = 2 * g + 1 < mt;
    float t1[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
            const int j = 2 * i + hb;  // block within the unit
            const uint32_t w0 = u.q[i][2 * hb] ^ 0x80808080u, w1 = u.q[i][2 * hb + 1] ^ 0x80808080u;
            const u32x4 b = {w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu, (w1 >> 8) & 0x00FF00FFu};
            floatx4 c = mfma16x16x32_f16(a_operand2(xs, kc, mt, kk + 32 * j), b, floatx4{0.f, 0.f, 0.f, 0.f});
            const float dj = f16_to_f32((u.h[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
            const float b0 = tok0 ? bku[(2 * g) * (kc / 32) + j] : 0.f;
            const float b1 = tok1 ? bku[(2 * g + 1) * (kc / 32) + j] : 0.f;
            t1[0] += (dj * b0) * (c[0] + c[1]);
            t1[1] += (dj * b1) * (c[2] + c[3]);
            acc2[0] += dj * (tok0 ? xs0[j] : 0.f);
            acc2[1] += dj * (tok1 ? xs1[j] : 0.f);
        }
    }
    acc1[0] += t1[0];
    acc1[1] += t1[1];
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

// ---------------------------------------------------------------------------------
// Streaming decode GEMV over many tiles (m <= 2, Q8_0 / Q6_K; the LM head).  Each
// workgroup loops over tiles blockIdx.x, + gridDim.x, ...  The activation (all of K)
// is staged once per workgroup into LDS as in gemv_kernel, and every wave loads its
// units of the next tile into registers before it computes the current one, so the
// weight stream of one tile overlaps the unit math of the previous one.  The waves
// of a tile meet in one of two reduction buffers (one barrier per tile).
// ---------------------------------------------------------------------------------
template <int FMT, int WAVES, int UPW>
__global__ __launch_bounds__(WAVES * 64) void gemv_stream_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    using Unit = typename UnitOf<FMT>::T;
    constexpr int GRAN = Fmt<FMT>::kSumGran;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int mt = (int)a.m;
    const int units = (int)(FMT == FQ80 ? a.nblk / 8 : a.nblk);
    const int kc = units * 256;  // K padded to whole units (the host checks mt * kc fits)
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)mt * kc * 4);
    float *backs = xsum + (size_t)mt * (kc / GRAN);
    __shared__ float red[2][2][WAVES][2][16];  // [tile parity][acc1 / acc2][wave][token][row]

    const int64_t ntile = a.ntile, step = gridDim.x;
    int64_t tile = blockIdx.x;  // the host launches at most ntile workgroups
    // every load below is issued unconditionally (a clamped unit or tile re-reads valid
    // bytes), so the in-order wait for one batch never covers a later one
    auto load = [&](int64_t t, Unit (&u)[UPW]) {
#pragma unroll
        for (int i = 0; i < UPW; i++) {
            const int ul = wv + i * WAVES;
            load_unit(a, t, ul < units ? ul : units - 1, u[i]);
        }
    };
    XRaw raw;
    stage_x_load(a, mt, 0, kc, 1.0f / (float)(kc / 8), raw);
    Unit w0[UPW], w1[UPW];
    load(tile, w0);
    stage_x_store<GRAN, FMT == FQ80>(a, kc, raw, xs, xsum, backs);
    __syncthreads();

    int par = 0;
    uint64_t run_key = 0;  // thread 0: the largest argmax key of this workgroup's tiles
    const int g = lane >> 4, n = lane & 15;
    auto body = [&](Unit (&cur)[UPW], Unit (&nxt)[UPW]) {
        const int64_t next = tile + step;
        load(next < ntile ? next : ntile - 1, nxt);
        float acc1[4][2] = {}, acc2[4][2] = {};
#pragma unroll
        for (int i = 0; i < UPW; i++) {
            const int ul = wv + i * WAVES;
            if (ul < units) compute_unit(cur[i], xs, xsum, kc, mt, ul * 256, backs + ul * 8, acc1[0], acc2[0]);
        }
        if constexpr (FMT == FQ6K) {
            // lane group g holds token g
            if (g < 2) {
                red[par][0][wv][g][n] = acc1[0][0];
                red[par][1][wv][g][n] = acc2[0][0];
            }
        } else {
            // lane group 0 holds tokens 0 and 1
            if (g == 0) {
                red[par][0][wv][0][n] = acc1[0][0];
                red[par][0][wv][1][n] = acc1[0][1];
                red[par][1][wv][0][n] = acc2[0][0];
                red[par][1][wv][1][n] = acc2[0][1];
            }
        }
        __syncthreads();  // the other buffer is rewritten only after the next tile's barrier
        if (tid < mt * 16) {
            const int t = tid >> 4, nn = tid & 15;
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < WAVES; w2++) {
                s1 += red[par][0][w2][t][nn];
                s2 += red[par][1][w2][t][nn];
            }
            // s1 carries the f16-subnormal factor 2^-24 of the integer weight codes
            const float bias_k = FMT == FQ80 ? 128.0f : 32.0f;
            float y = s1 * 16777216.0f - bias_k * s2;
            const int64_t row = tile * 16 + nn;
            if (row < a.n) {
                if (a.bias) y += a.bias[row];
                gemv_status(a, y, tile == 0 && tid == 0);
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
                if (nn == 0) run_key = key > run_key ? key : run_key;
            }
        }
        par ^= 1;
        tile = next;
    };
    for (;;) {
        body(w0, w1);
        if (tile >= ntile) break;
        body(w1, w0);
        if (tile >= ntile) break;
    }
    // one argmax key per workgroup (the host reduces gridDim.x keys)
    if (a.argmax_partial && tid == 0) a.argmax_partial[blockIdx.x] = run_key;
    __builtin_amdgcn_s_waitcnt(0);  // the last (unused) prefetch
}

// ---------------------------------------------------------------------------------
// Q6_K streaming decode GEMV (the LM head): gemv_stream_kernel's tile loop with one
// unit (256 k) per wave and K <= 16 units, arranged so that a tile costs little more
// than its weight bytes:
//  * everything that depends only on x is built once per workgroup, before the loop,
//    in registers: the A operands of the unit's 8 MFMAs, its 2^-s block factors, and
//    the A operand of the offset term;
//  * the offset term 32 * sum_j sc_j * sum(x over sub-block j) is one more MFMA per
//    unit: A = the 16 sub-block sums of x (f16 hi + lo under a power of two per token
//    and unit), B = the row's 16 int8 scales as f16 (exact);
//  * the int8 scales become f16 with byte moves and one packed add (1024 + 128 + s is
//    an exact f16 built from the byte s ^ 0x80 under exponent 10), and enter the f32
//    sums through mixed-precision FMAs;
//  * weight pointers are scalar per wave and tile.
// Q6_K codes q (6 bits) enter as f16 subnormals q * 2^-24, exact, as in the decode kernels.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t i8pair_to_f16x2(uint32_t w, int hi) {
    // bytes (2 hi, 2 hi + 1) of w -> f16 (s0, s1): 0x64 | (b ^ 0x80) is 1152 + s exactly
    const uint32_t b = __builtin_amdgcn_perm(0u, w, hi ? 0x0C030C02u : 0x0C010C00u) ^ 0x64806480u;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, b) + h2{(_Float16)-1152.0f, (_Float16)-1152.0f});
}
__device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

template <int MT>
__global__ __launch_bounds__(1024) void gemv_q6k_stream_kernel(GemvArgs a) {
    constexpr int WAVES = 16, GRAN = 16;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int units = (int)a.nblk;  // 1 .. 16 (host-checked)
    const int kc = units * 256;
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)MT * kc * 4);
    float *backs = xsum + (size_t)MT * (kc / GRAN);
    __shared__ float red[2][2][WAVES][2][16];  // [tile parity][main / offset][wave][token][row]
    __shared__ __attribute__((aligned(16))) uint16_t zpad[8];

    const int64_t ntile = a.ntile, step = gridDim.x;
    int64_t tile = blockIdx.x;
    const bool has = wv < units;  // wave-uniform: this wave owns unit wv
    const int ul = has ? wv : 0;
    const int p = lane >> 4, m = lane & 15, n = m, g = p;

    auto qptr = [&](int64_t t) { return a.qs + (size_t)(t * a.nblk + ul) * 3072 + 12 * lane; };
    auto hptr = [&](int64_t t) { return a.hdr + (size_t)(t * a.nblk + ul) * 288; };
    struct W {
        u32x3 q[4];
        u32x4 s;
        uint32_t d;
    };
    auto load = [&](int64_t t, W &w) {
        const uint8_t *qb = qptr(t), *hb = hptr(t);
#pragma unroll
        for (int c = 0; c < 4; c++) w.q[c] = ldg96(qb + 768 * c);
        w.s = ldg128(hb + 16 * n);
        w.d = *reinterpret_cast<const uint16_t *>(hb + 256 + 2 * n);
    };

    XRaw raw;
    stage_x_load(a, MT, 0, kc, 1.0f / (float)(kc / 8), raw);
    W w0, w1;
    if (has) load(tile, w0);
    if (tid < 2) reinterpret_cast<u32x4 *>(zpad)[0] = u32x4{0u, 0u, 0u, 0u};
    stage_x_store<GRAN, false>(a, kc, raw, xs, xsum, backs);
    __syncthreads();

    // ---- per-wave constants (x only) ----
    // A operand of MFMA (c, h): lane (p, m) -> token m >> 2, half (m >> 1) & 1, part m & 1;
    // non-zero only where the lane's k-slice p lies in that 16-k half (p >> 1 == half)
    u32x4 av[4][2];
    {
        const int t = m >> 2, part = m & 1, half = (m >> 1) & 1;
        const bool own = t < MT && (p >> 1) == half;
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint16_t *src = own ? xs + ((size_t)t * 2 + part) * kc + ul * 256 + 64 * c + 32 * h + 8 * p : zpad;
                av[c][h] = *reinterpret_cast<const u32x4 *>(src);
            }
    }
    // 2^-s of the unit's 32-element blocks for this lane group's token
    float xb[8];
#pragma unroll
    for (int i = 0; i < 8; i++) xb[i] = g < MT ? backs[g * (kc / 32) + ul * 8 + i] : 0.0f;
    // offset-term A operand: row m = 4t + part (part < 2) holds the unit's 16 sub-block
    // sums of token t (k-slices p = 0, 1), as f16 hi / lo of sum * 2^so(t)
    u32x4 a2 = {0u, 0u, 0u, 0u};
    float back2 = 0.0f;  // 2^-so of this lane group's token
    {
        // so per token: max |sum| over the unit's 16 sums -> [2^14, 2^15)
        float so_t[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            float mx = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(xsum[t * (kc / GRAN) + ul * 16 + j]));
            float s, b;
            f16_prescale(mx, s, b);
            so_t[t] = s;
            if (g == t) back2 = b;
        }
        const int t = m >> 2, part = m & 3;
        if (t < MT && part < 2 && p < 2) {
            const float s = so_t[t];
            uint32_t hv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t hh, ll;
                split_f16(xsum[t * (kc / GRAN) + ul * 16 + 8 * p + i] * s, hh, ll);
                hv[i] = part ? ll : hh;
            }
            a2 = u32x4{hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16)};
        }
    }

    int par = 0;
    uint64_t run_key = 0;  // thread 0: the largest argmax key of this workgroup's tiles
    auto body = [&](W &cur, W &nxt) {
        const int64_t next = tile + step;
        if (has) load(next < ntile ? next : ntile - 1, nxt);
        float acc1 = 0.0f, acc2 = 0.0f;
        if (has) {
            // the row's 16 scales as f16 pairs: sc[i] = (scale 2i, scale 2i + 1)
            uint32_t sc[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[2 * i] = i8pair_to_f16x2(cur.s[i], 0);
                sc[2 * i + 1] = i8pair_to_f16x2(cur.s[i], 1);
            }
            float t1 = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t A = cur.q[c][0], B = cur.q[c][1], C = cur.q[c][2];
                const u32x4 ba = {((A)&0x000F000Fu) | ((C << 4) & 0x00300030u),
                                  ((A >> 4) & 0x000F000Fu) | ((C << 2) & 0x00300030u),
                                  ((A >> 8) & 0x000F000Fu) | ((C)&0x00300030u),
                                  ((A >> 12) & 0x000F000Fu) | ((C >> 2) & 0x00300030u)};
                const u32x4 bb = {((B)&0x000F000Fu) | ((C >> 4) & 0x00300030u),
                                  ((B >> 4) & 0x000F000Fu) | ((C >> 6) & 0x00300030u),
                                  ((B >> 8) & 0x000F000Fu) | ((C >> 8) & 0x00300030u),
                                  ((B >> 12) & 0x000F000Fu) | ((C >> 10) & 0x00300030u)};
                const floatx4 ca = mfma16x16x32_f16(av[c][0], ba, floatx4{0.f, 0.f, 0.f, 0.f});
                const floatx4 cb = mfma16x16x32_f16(av[c][1], bb, floatx4{0.f, 0.f, 0.f, 0.f});
                // sub-blocks 4c .. 4c + 3: scales sc[2c] (lo, hi), sc[2c + 1] (lo, hi)
                const float ta = f16_lo(sc[2 * c]) * (ca[0] + ca[1]) + f16_hi(sc[2 * c]) * (ca[2] + ca[3]);
                const float tb = f16_lo(sc[2 * c + 1]) * (cb[0] + cb[1]) + f16_hi(sc[2 * c + 1]) * (cb[2] + cb[3]);
                t1 += xb[2 * c] * ta + xb[2 * c + 1] * tb;
            }
            // offset term: B2 lane (p, n) = scales 8 (p & 1) .. + 7 of row n (A2 is zero for p >= 2)
            const u32x4 b2 = (p & 1) ? u32x4{sc[4], sc[5], sc[6], sc[7]} : u32x4{sc[0], sc[1], sc[2], sc[3]};
            const floatx4 c2 = mfma16x16x32_f16(a2, b2, floatx4{0.f, 0.f, 0.f, 0.f});
            const float d = f16_to_f32(cur.d);
            acc1 = d * t1;
            acc2 = d * ((c2[0] + c2[1]) * back2);
        }
        if (g < MT) {
            red[par][0][wv][g][n] = acc1;
            red[par][1][wv][g][n] = acc2;
        }
        __syncthreads();  // the other buffer is rewritten only after the next tile's barrier
        if (tid < MT * 16) {
            const int t = tid >> 4, nn = tid & 15;
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < WAVES; w2++) {
                s1 += red[par][0][w2][t][nn];
                s2 += red[par][1][w2][t][nn];
            }
            float y = s1 * 16777216.0f - 32.0f * s2;
            const int64_t row = tile * 16 + nn;
            if (row < a.n) {
                if (a.bias) y += a.bias[row];
                gemv_status(a, y, tile == 0 && tid == 0);
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
            }
            if (a.argmax_partial && t == 0) {
                uint64_t key = row < a.n ? (y != y ? ~0ull : argmax_key(y, (uint32_t)row)) : 0ull;
                for (int o = 8; o > 0; o >>= 1) {
                    uint64_t other = __shfl_xor(key, o, 16);
                    key = other > key ? other : key;
                }
                if (nn == 0) run_key = key > run_key ? key : run_key;
            }
        }
        par ^= 1;
        tile = next;
    };
    for (;;) {
        body(w0, w1);
        if (tile >= ntile) break;
        body(w1, w0);
        if (tile >= ntile) break;
    }
    // one argmax key per workgroup (the host reduces gridDim.x keys)
    if (a.argmax_partial && tid == 0) a.argmax_partial[blockIdx.x] = run_key;
    __builtin_amdgcn_s_waitcnt(0);  // the last (unused) prefetch
}

// ---------------------------------------------------------------------------------
// Q4_K decode kernel (m <= 2).  One workgroup per 16-row tile, unit u of K to wave
// u % WAVES, every wave issuing the activation slices and the weight loads of all its
// units of a pass up front and then working through its units without a workgroup
// barrier, arranged so that almost nothing but the MFMA inputs goes through LDS:
//  * staging lane 16G + j holds elements 64G + 4j .. 64G + 4j + 3 of the unit, so
//    sub-blocks 2G and 2G + 1 live in the same 16-lane row that consumes them in
//    the MFMA epilogue (compute lane 16G + n, row n of the tile).  The per
//    sub-block power-of-two scale and sum of x are reduced over each half-row with
//    DPP and swapped between the two half-rows with one rotation; they stay in
//    registers;
//  * x * s is split into f16 hi + lo pairs by mixed-precision FMAs that write both
//    halves of a register, so a pair costs two instructions;
//  * the wave index is made scalar, so unit indices and base addresses are scalar;
//  * the four lane groups are summed with the permlane swaps, and each lane folds
//    its two accumulators (codes * 2^-24 sums, min terms) into one value first.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mix_hi2(float a, float b, float s) {
    uint32_t r;  // f16(a * s) | f16(b * s) << 16
    asm("v_fma_mixlo_f16 %0, %1, %2, 0\n\tv_fma_mixhi_f16 %0, %3, %2, 0" : "=&v"(r) : "v"(a), "v"(s), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t mix_lo2(float a, float b, float s, uint32_t hi) {
    uint32_t r;  // f16(a * s - hi.x) | f16(b * s - hi.y) << 16, each residual formed exactly by the FMA
    asm("v_fma_mixlo_f16 %0, %1, %2, -%4 op_sel_hi:[0,0,1]\n\t"
        "v_fma_mixhi_f16 %0, %3, %2, -%4 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=&v"(r)
        : "v"(a), "v"(s), "v"(b), "v"(hi));
    return r;
}
__device__ __forceinline__ float absmax4(float a, float b, float c, float d) {
    float r;
    asm("v_max3_f32 %0, |%1|, |%2|, |%3|\n\tv_max3_f32 %0, %0, |%4|, |%4|" : "=&v"(r) : "v"(a), "v"(b), "v"(c), "v"(d));
    return r;
}
template <int CTRL>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
    return v > o ? v : o;
}
template <int CTRL>
__device__ __forceinline__ float add_dpp(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ float mov_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
// sum over the four 16-lane rows (every lane receives the total of its column)
__device__ __forceinline__ float sum_rows(float v) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Per-lane activation statistics of one token: 1/scale and sum of x for sub-blocks
// 2G (lo) and 2G + 1 (hi) of the lane's row.
struct XStat {
    float b_lo, b_hi, xs_lo, xs_hi;
};

// Stage this lane's 4 activations (f32, or bf16 in raw[0..1]) of one token into
// the hi / lo f16 planes of the wave's unit buffer.
template <bool XB>
__device__ __forceinline__ void stage_q4k(const u32x4 &raw, uint16_t *hi_plane, uint16_t *lo_plane, XStat &st) {
    const int lane = threadIdx.x & 63;
    float v0, v1, v2, v3;
    if (XB) {
        v0 = __uint_as_float(raw[0] << 16);
        v1 = __uint_as_float(raw[0] & 0xFFFF0000u);
        v2 = __uint_as_float(raw[1] << 16);
        v3 = __uint_as_float(raw[1] & 0xFFFF0000u);
    } else {
        v0 = __uint_as_float(raw[0]);
        v1 = __uint_as_float(raw[1]);
        v2 = __uint_as_float(raw[2]);
        v3 = __uint_as_float(raw[3]);
    }
    // max |x| of the lane's 32-element sub-block (8 lanes), compared as bit patterns
    uint32_t m = __float_as_uint(absmax4(v0, v1, v2, v3));
    m = umax_dpp<0xB1>(m);   // lane ^ 1
    m = umax_dpp<0x4E>(m);   // lane ^ 2
    m = umax_dpp<0x141>(m);  // row_half_mirror: the other quad of the 8
    // s = 2^(14 - e) (e = unbiased exponent of the max) capped at 2^126, so max * s
    // lies in [2^14, 2^15); back = 1/s, a normal f32 for every input.  A NaN or inf
    // max gives a finite s and the non-finite value propagates through the products.
    const uint32_t sb = min(0x86000000u - (m & 0x7F800000u), 0x7E800000u);
    const float s = __uint_as_float(sb);
    const uint32_t h01 = mix_hi2(v0, v1, s), h23 = mix_hi2(v2, v3, s);
    const uint32_t l01 = mix_lo2(v0, v1, s, h01), l23 = mix_lo2(v2, v3, s, h23);
    *reinterpret_cast<u32x2 *>(hi_plane + 4 * lane) = u32x2{h01, h23};
    *reinterpret_cast<u32x2 *>(lo_plane + 4 * lane) = u32x2{l01, l23};
    float sum = (v0 + v1) + (v2 + v3);
    sum = add_dpp<0xB1>(sum);
    sum = add_dpp<0x4E>(sum);
    sum = add_dpp<0x141>(sum);
    const float back = __uint_as_float(0x7F000000u - sb);
    const float back_o = mov_dpp<0x128>(back), sum_o = mov_dpp<0x128>(sum);  // row_ror:8, the other half-row
    const bool first = (lane & 8) == 0;
    st.b_lo = first ? back : back_o;
    st.b_hi = first ? back_o : back;
    st.xs_lo = first ? sum : sum_o;
    st.xs_hi = first ? sum_o : sum;
}

// Buffer resources over one tile's planes: SGPR bases, so a load's address is a lane
// offset (VGPR) plus a unit offset (SGPR) with no per-load address arithmetic; reads
// past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gv_rsrc(const void *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)min(bytes, (int64_t)0x7FFFFFF0), 0x00020000);
}
// AUX 2: non-temporal (the weight stream); 0: default (activations, reused from L2)
template <int AUX>
__device__ __forceinline__ u32x4 gv_load4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}
__device__ __forceinline__ u32x2 gv_load2(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// XM: activation kind, 0 f32, 1 bf16, 2 f32 gate | up pairs (SwiGLU prologue).
// The arguments the first loads need come first as scalars: the build preloads the
// leading kernel arguments into SGPRs (-amdgpu-kernarg-preload-count), so a wave issues
// its loads without waiting for the kernel-argument fetch; the rest (outputs, bias,
// status, argmax) sit in GemvArgs and are fetched while the loads are in flight.
// One workgroup per 16-row tile (grid = ntile).
template <int WAVES, int UPW, int XM, int MT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q4k_decode_kernel(const uint8_t *qs, const uint8_t *hdr,
                                                                    const void *x, int units, int mt, GemvArgs a) {
    constexpr bool XB = XM == 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = (int)blockIdx.x;
    const int k = units * 256;             // the host checks k >= 256
    const int xrow = XM == 2 ? 2 * k : k;  // elements per token row of x
    constexpr int xe = XB ? 2 : 4;
    const __amdgpu_buffer_rsrc_t rq = gv_rsrc(qs + (size_t)tile * units * 2048, (int64_t)units * 2048);
    const __amdgpu_buffer_rsrc_t rh = gv_rsrc(hdr + (size_t)tile * units * 256, (int64_t)units * 256);
    const __amdgpu_buffer_rsrc_t rx = gv_rsrc(x, (int64_t)mt * xrow * xe);
    const int l16 = 16 * lane, n16 = 16 * (lane & 15), lx = 4 * lane * xe;

    // A-operand rows of lane group G: 4G + 2t + part (token 2 tp + t of MFMA set tp, hi /
    // lo part) over the k-group of sub-block 2G (low nibbles) or 2G + 1 (high nibbles);
    // other rows zero.  Four tokens take two sets of MFMAs over the same B operands.
    static_assert(MT == 1 || MT == 2 || MT == 4, "token rows");
    constexpr int NTP = (MT + 1) / 2;
    // per wave: one buffer per unit of a pass [token, hi/lo][256] f16, each followed
    // by 64 zero halves that the A operand of the rows without data reads
    constexpr int kBuf = MT * 512 + 64;
    __shared__ __attribute__((aligned(16))) uint16_t xbuf[WAVES][UPW][kBuf];
    __shared__ float red[WAVES][MT][16];
    const int G = lane >> 4, n = lane & 15, i = n & 3;

    float acc1[MT], acc2[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc1[t] = acc2[t] = 0.f;
    int ub0 = 0;
    do {  // passes over K
        // activation slices first (L2 hits), then the weights of every unit of the pass
        u32x4 xr[UPW][MT], xu[XM == 2 ? UPW : 1][MT];
        UnitQ4K w[UPW];
        int uo[UPW];
#pragma unroll
        for (int j = 0; j < UPW; j++) uo[j] = min(ub0 + wv + j * WAVES, units - 1);
#pragma unroll
        for (int j = 0; j < UPW; j++) {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int tr = t < mt ? t : 0;  // rows past the batch read row 0, staged as zeros
                const int so = (tr * xrow + uo[j] * 256) * xe;
                if (XB) {
                    const u32x2 w2 = gv_load2(rx, lx, so);
                    xr[j][t] = u32x4{w2[0], w2[1], 0u, 0u};
                } else {
                    xr[j][t] = gv_load4<0>(rx, lx, so);
                }
                if constexpr (XM == 2) xu[j][t] = gv_load4<0>(rx, lx, so + k * 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep this issue order
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            w[j].q0 = gv_load4<2>(rq, l16, uo[j] * 2048);
            w[j].q1 = gv_load4<2>(rq, l16 + 1024, uo[j] * 2048);
            w[j].h = gv_load4<2>(rh, n16, uo[j] * 256);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ub0 == 0 && lane < 8 * UPW)  // the wave's own pads, read later only by lanes of this wave
            *reinterpret_cast<u32x4 *>(&xbuf[wv][lane >> 3][MT * 512 + 8 * (lane & 7)]) = u32x4{0u, 0u, 0u, 0u};
        // every unit's activation slice is staged first: it needs only the activation
        // loads (issued before the weights), so it runs while the weights stream in
        XStat st_all[UPW][MT];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            if (ub0 + wv + j * WAVES >= units) break;  // wave-uniform
            uint16_t *buf = xbuf[wv][j];
#pragma unroll
            for (int t = 0; t < MT; t++) {
                u32x4 xv = xr[j][t];
                if constexpr (XM == 2) xv = swiglu4(xv, xu[j][t]);
                if (MT > 2 && t >= mt) xv = u32x4{0u, 0u, 0u, 0u};  // rows past the batch
                stage_q4k<XB>(xv, buf + 512 * t, buf + 512 * t + 256, st_all[j][t]);
            }
        }
        // the wave's own LDS writes are read back by other lanes of the same wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        int aoff[NTP];
#pragma unroll
        for (int tp = 0; tp < NTP; tp++) {
            const bool own = G == (n >> 2) && 2 * tp + (i >> 1) < MT;
            aoff[tp] = own ? ((2 * tp + (i >> 1)) * 2 + (i & 1)) * 256 + 64 * G : MT * 512;
        }
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            if (ub0 + wv + j * WAVES >= units) break;  // wave-uniform
            const XStat *st = st_all[j];
            const uint16_t *ap[NTP];
#pragma unroll
            for (int tp = 0; tp < NTP; tp++) ap[tp] = xbuf[wv][j] + aoff[tp];
            // header: d | dmin, scales[0..3], scales[4..7], scales[8..11] (BlockQ4K
            // packing, get_scale_min_k4, crates/nn-core/src/layers/quantized/linear.rs:166-176)
            const u32x4 &h = w[j].h;
            const float d = f16_to_f32(h[0] & 0xFFFFu), dmin = f16_to_f32(h[0] >> 16);
            const uint32_t S1 = h[1], S2 = h[2], S3 = h[3];
            const uint32_t hsel = 0u - (uint32_t)(G >> 1);  // all ones for sub-blocks 4..7
            const uint32_t scw =
                ((S1 & 0x3F3F3F3Fu) & ~hsel) | (((S3 & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) & hsel);
            const uint32_t mnw =
                ((S2 & 0x3F3F3F3Fu) & ~hsel) | ((((S3 >> 4) & 0x0F0F0F0Fu) | ((S2 >> 2) & 0x30303030u)) & hsel);
            const uint32_t scp = scw >> (16 * (G & 1)), mnp = mnw >> (16 * (G & 1));
            const float sc_lo = (float)(scp & 0xFFu), sc_hi = 0.0625f * (float)((scp >> 8) & 0xFFu);
            const float mn_lo = (float)(mnp & 0xFFu), mn_hi = (float)((mnp >> 8) & 0xFFu);

            floatx4 clo[NTP], chi[NTP];
#pragma unroll
            for (int tp = 0; tp < NTP; tp++) clo[tp] = chi[tp] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const u32x4 q = q4 < 2 ? w[j].q0 : w[j].q1;
                const uint32_t w0 = q[2 * (q4 & 1)], w1 = q[2 * (q4 & 1) + 1];
                const uint32_t w0s = w0 >> 8, w1s = w1 >> 8;
                const u32x4 blo = {w0 & 0x000F000Fu, w0s & 0x000F000Fu, w1 & 0x000F000Fu, w1s & 0x000F000Fu};
                const u32x4 bhi = {w0 & 0x00F000F0u, w0s & 0x00F000F0u, w1 & 0x00F000F0u, w1s & 0x00F000F0u};
#pragma unroll
                for (int tp = 0; tp < NTP; tp++) {
                    clo[tp] = mfma16x16x32_f16(*reinterpret_cast<const u32x4 *>(ap[tp] + 8 * q4), blo, clo[tp]);
                    chi[tp] = mfma16x16x32_f16(*reinterpret_cast<const u32x4 *>(ap[tp] + 32 + 8 * q4), bhi, chi[tp]);
                }
            }
            // lane 16G + n now holds, for row n and sub-blocks 2G / 2G + 1, the
            // (hi, lo) partial dot products of token 2 tp (entries 0, 1 of set tp) and
            // token 2 tp + 1 (entries 2, 3)
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const floatx4 &cl = clo[t >> 1], &ch = chi[t >> 1];
                const int e = 2 * (t & 1);
                const float T = (sc_lo * st[t].b_lo) * (cl[e] + cl[e + 1]) + (sc_hi * st[t].b_hi) * (ch[e] + ch[e + 1]);
                acc1[t] += d * T;
                acc2[t] += dmin * (mn_lo * st[t].xs_lo + mn_hi * st[t].xs_hi);
            }
        }
        ub0 += WAVES * UPW;
    } while (ub0 < units);

    // y = 2^24 * (code sums) - (min terms), summed over the lane groups, then the waves
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const float v = sum_rows(acc1[t] * 16777216.0f - acc2[t]);
        if (lane < 16) red[wv][t][lane] = v;
    }
    __syncthreads();
    if (tid < MT * 16) {
        const int t = tid >> 4, nn = tid & 15;
        float y = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) y += red[w2][t][nn];
        const int64_t row = (int64_t)tile * 16 + nn;
        if (a.swiglu_out) {
            // rows nn < 8 are gate rows, nn + 8 their up rows (full tiles: n = 2 * inter, inter % 8 == 0)
            store_swiglu_pair(a, y, t, tile, nn, blockIdx.x == 0 && tid == 0);
        } else if (row < a.n && t < mt) {
            if (a.bias) y += a.bias[row];
            gemv_status(a, y, blockIdx.x == 0 && tid == 0);
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
            else
                reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
        }
        if (a.argmax_partial && t == 0) {
            // first-index argmax of this tile's 16 logits (the 16 lanes hold one tile)
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
// Q8_0 decode kernel (m <= 2).  gemv_q4k_decode_kernel's division of work over the
// Q8_0 tile16 image (a unit is 8 blocks = 256 k of a 16-row tile: four 1024-byte
// block pairs, lane 16p + r holding bytes 8p .. 8p + 7 of both blocks of row r, and
// 16 bytes of row r's eight f16 d), arranged so that a wave waits once per unit:
//  * staging lane l holds elements 4l .. 4l + 3 of the unit (block l / 8); each
//    block's power-of-two scale and sum of x are reduced over its 8 lanes with DPP
//    and read out as wave-uniform scalars, so no statistics go through LDS;
//  * the A operand of block j is one 16-byte LDS read per lane (rows 2t / 2t + 1 =
//    hi / lo of token t; the other rows read a zero pad, without branches); the
//    eight reads of a unit are issued together and its eight MFMAs are independent;
//  * codes enter as f16 subnormals (q ^ 0x80) * 2^-24 = (q + 128) * 2^-24, exact,
//    and the block's 128 * sum(x) offset is subtracted with its d in f32.
// Lanes 0 .. 15 of a wave end with the partial of rows 0 .. 15 for each token.
// ---------------------------------------------------------------------------------
template <bool XB>
__device__ __forceinline__ void stage_q80(const u32x4 &raw, bool in, uint16_t *hi_plane, uint16_t *lo_plane,
                                          float &back, float &sum) {
    const int lane = threadIdx.x & 63;
    float v0, v1, v2, v3;
    if (XB) {
        v0 = __uint_as_float(raw[0] << 16);
        v1 = __uint_as_float(raw[0] & 0xFFFF0000u);
        v2 = __uint_as_float(raw[1] << 16);
        v3 = __uint_as_float(raw[1] & 0xFFFF0000u);
    } else {
        v0 = __uint_as_float(raw[0]);
        v1 = __uint_as_float(raw[1]);
        v2 = __uint_as_float(raw[2]);
        v3 = __uint_as_float(raw[3]);
    }
    if (!in) v0 = v1 = v2 = v3 = 0.0f;  // k beyond K in the last (padded) unit
    // max |x| of the lane's 32-element block (8 lanes), compared as bit patterns;
    // s, back and the non-finite handling as in stage_q4k
    uint32_t m = __float_as_uint(absmax4(v0, v1, v2, v3));
    m = umax_dpp<0xB1>(m);
    m = umax_dpp<0x4E>(m);
    m = umax_dpp<0x141>(m);
    const uint32_t sb = min(0x86000000u - (m & 0x7F800000u), 0x7E800000u);
    const float s = __uint_as_float(sb);
    const uint32_t h01 = mix_hi2(v0, v1, s), h23 = mix_hi2(v2, v3, s);
    const uint32_t l01 = mix_lo2(v0, v1, s, h01), l23 = mix_lo2(v2, v3, s, h23);
    *reinterpret_cast<u32x2 *>(hi_plane + 4 * lane) = u32x2{h01, h23};
    *reinterpret_cast<u32x2 *>(lo_plane + 4 * lane) = u32x2{l01, l23};
    float sm = (v0 + v1) + (v2 + v3);
    sm = add_dpp<0xB1>(sm);
    sm = add_dpp<0x4E>(sm);
    sm = add_dpp<0x141>(sm);
    back = __uint_as_float(0x7F000000u - sb);
    sum = sm;
}

__device__ __forceinline__ float lane_value(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// XM: activation kind, 0 f32, 1 bf16, 2 f32 gate | up pairs (SwiGLU prologue).  Leading
// scalar arguments preloaded into SGPRs and buffer loads, as gemv_q4k_decode_kernel.
template <int WAVES, int UPW, int XM, int MT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q80_decode_kernel(const uint8_t *qs, const uint8_t *hdr,
                                                                    const void *x, int units, int k, int mt,
                                                                    GemvArgs a) {
    constexpr bool XB = XM == 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = (int)blockIdx.x;
    constexpr int xe = XB ? 2 : 4;
    const int xrow = XM == 2 ? 2 * k : k;  // elements per token row of x
    const __amdgpu_buffer_rsrc_t rq = gv_rsrc(qs + (size_t)tile * units * 4096, (int64_t)units * 4096);
    const __amdgpu_buffer_rsrc_t rh = gv_rsrc(hdr + (size_t)tile * units * 256, (int64_t)units * 256);
    const __amdgpu_buffer_rsrc_t rx = gv_rsrc(x, (int64_t)mt * xrow * xe);
    const int l16 = 16 * lane, lx = 4 * lane * xe;
    // per wave and unit of a pass: [token, hi / lo][256] f16, then 256 zero halves
    constexpr int kBuf = MT * 512 + 256;
    __shared__ __attribute__((aligned(16))) uint16_t xbuf[WAVES][UPW][kBuf];
    __shared__ float red[WAVES][MT][16];

    // A-operand row of this lane: lane & 15 = 2t + part (token t, hi / lo part)
    const int r16 = lane & 15, kg = lane >> 4;
    const int aoff = (r16 >> 1) < MT ? r16 * 256 + 8 * kg : MT * 512 + 8 * kg;

    float acc1[MT], acc2[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc1[t] = acc2[t] = 0.f;
    int ub0 = 0;
    do {  // passes over K (units >= 1)
        // activation slices first (L2 hits), then the weights of every unit of the pass
        u32x4 xr[UPW][MT], xu[XM == 2 ? UPW : 1][MT];
        bool xin[UPW];
        int uo[UPW];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            uo[j] = min(ub0 + wv + j * WAVES, units - 1);
            xin[j] = uo[j] * 256 + 4 * lane < k;  // k beyond K in the last (padded) unit: staged as zeros
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int so = (t * xrow + uo[j] * 256) * xe;
                if (XB) {
                    const u32x2 w2 = gv_load2(rx, lx, so);
                    xr[j][t] = u32x4{w2[0], w2[1], 0u, 0u};
                } else {
                    xr[j][t] = gv_load4<0>(rx, lx, so);
                }
                if constexpr (XM == 2) xu[j][t] = gv_load4<0>(rx, lx, so + k * 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep this issue order
        UnitQ80 w[UPW];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
#pragma unroll
            for (int i = 0; i < 4; i++) w[j].q[i] = gv_load4<2>(rq, l16 + 1024 * i, uo[j] * 4096);
            w[j].h = gv_load4<2>(rh, 16 * r16, uo[j] * 256);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ub0 == 0) {  // the wave's own pads, read later only by lanes of this wave
#pragma unroll
            for (int j = 0; j < UPW; j++)
                if (lane < 32) *reinterpret_cast<u32x4 *>(&xbuf[wv][j][MT * 512 + 8 * lane]) = u32x4{0u, 0u, 0u, 0u};
        }
        // staging needs only the activation loads, so it runs while the weights stream in
        float bk[UPW][MT], xs[UPW][MT];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            if (ub0 + wv + j * WAVES >= units) break;  // wave-uniform
            uint16_t *buf = xbuf[wv][j];
#pragma unroll
            for (int t = 0; t < MT; t++) {
                u32x4 xv = xr[j][t];
                if constexpr (XM == 2) xv = swiglu4(xv, xu[j][t]);
                stage_q80<XB>(xv, xin[j], buf + 512 * t, buf + 512 * t + 256, bk[j][t], xs[j][t]);
            }
        }
        // the wave's own LDS writes are read back by other lanes of the same wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            if (ub0 + wv + j * WAVES >= units) break;  // wave-uniform
            const uint16_t *ap = xbuf[wv][j] + aoff;
            u32x4 av[8];
#pragma unroll
            for (int b = 0; b < 8; b++) av[b] = *reinterpret_cast<const u32x4 *>(ap + 32 * b);
            floatx4 c[8];
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint32_t w0 = w[j].q[b >> 1][2 * (b & 1)] ^ 0x80808080u;
                const uint32_t w1 = w[j].q[b >> 1][2 * (b & 1) + 1] ^ 0x80808080u;
                const u32x4 bop = {w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu,
                                   (w1 >> 8) & 0x00FF00FFu};
                c[b] = mfma16x16x32_f16(av[b], bop, floatx4{0.f, 0.f, 0.f, 0.f});
            }
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const float d = f16_to_f32((w[j].h[b >> 1] >> (16 * (b & 1))) & 0xFFFFu);
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const float back = lane_value(bk[j][t], 8 * b), xsum = lane_value(xs[j][t], 8 * b);
                    acc1[t] += (d * back) * (c[b][2 * t] + c[b][2 * t + 1]);
                    acc2[t] += d * xsum;
                }
            }
        }
        ub0 += WAVES * UPW;
    } while (ub0 < units);

    // y = 2^24 * (code sums) - 128 * (offset terms), then summed over the waves
#pragma unroll
    for (int t = 0; t < MT; t++)
        if (lane < 16) red[wv][t][lane] = acc1[t] * 16777216.0f - 128.0f * acc2[t];
    __syncthreads();
    if (tid < MT * 16) {
        const int t = tid >> 4, nn = tid & 15;
        float y = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) y += red[w2][t][nn];
        const int64_t row = (int64_t)tile * 16 + nn;
        if (row < a.n) {
            if (a.bias) y += a.bias[row];
            gemv_status(a, y, blockIdx.x == 0 && tid == 0);
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
            else
                reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
        }
        if (a.argmax_partial && t == 0) {
            // first-index argmax of this tile's 16 logits (the 16 lanes hold one tile)
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
// Q8_0 batched decode (3 <= m <= 8; MT = 4 or 8 token rows, the rows past m zero):
// gemv_q80_decode_kernel's unit math with every A row in use (rows 2t + part), so lane
// group g holds tokens 2g and 2g + 1.  The block statistics of every token go through a
// per-wave LDS table (8 powers of two and 8 sums per token) that each lane group reads
// for its two tokens with broadcast 16-byte reads.  One unit per wave and pass.
// ---------------------------------------------------------------------------------
template <int WAVES, int XM, int MT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q80_batch_kernel(GemvArgs a) {
    constexpr bool XB = XM == 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = (int)blockIdx.x, mt = (int)a.m;
    constexpr int kBuf = MT * 512 + 256;
    __shared__ __attribute__((aligned(16))) uint16_t xbuf[WAVES][kBuf];
    __shared__ __attribute__((aligned(16))) float stats[WAVES][MT][16];  // [token][8 x 2^-s, 8 x sum]
    __shared__ float red[WAVES][MT][16];
    if (lane < 32) *reinterpret_cast<u32x4 *>(&xbuf[wv][MT * 512 + 8 * lane]) = u32x4{0u, 0u, 0u, 0u};

    const int r16 = lane & 15, kg = lane >> 4, g = kg;
    const int aoff = (r16 >> 1) < MT ? r16 * 256 + 8 * kg : MT * 512 + 8 * kg;
    const int t0 = min(2 * g, MT - 1), t1 = min(2 * g + 1, MT - 1);  // this lane group's tokens

    const int units = (int)(a.nblk / 8), k = (int)a.k;
    const uint8_t *qbase = a.qs + (size_t)tile * (size_t)(a.nblk / 2) * 1024 + 16 * lane;
    const uint8_t *hbase = a.hdr + (size_t)tile * units * 256 + 16 * r16;
    constexpr int xe = XB ? 2 : 4;
    const int xrow = XM == 2 ? 2 * k : k;
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.x);
    float acc1[2] = {0.f, 0.f}, acc2[2] = {0.f, 0.f};
    for (int ub0 = 0; ub0 < units; ub0 += WAVES) {
        const int u = min(ub0 + wv, units - 1);
        const int kk = u * 256 + 4 * lane;
        const bool xin = kk < k;
        u32x4 xr[MT], xu[XM == 2 ? MT : 1];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const bool tin = xin && t < mt;
            const uint8_t *p = xb + (size_t)(tin ? t * xrow + kk : 0) * xe;  // out of range: x[0]
            if (XB) {
                const u32x2 w2 = *reinterpret_cast<const u32x2 *>(p);
                xr[t] = u32x4{w2[0], w2[1], 0u, 0u};
            } else {
                xr[t] = *reinterpret_cast<const u32x4 *>(p);
            }
            if constexpr (XM == 2) xu[t] = *reinterpret_cast<const u32x4 *>(p + (size_t)k * 4);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep this issue order
        UnitQ80 w;
#pragma unroll
        for (int i = 0; i < 4; i++) w.q[i] = ldg128(qbase + (size_t)(u * 4 + i) * 1024u);
        w.h = ldg128(hbase + (size_t)u * 256u);
        __builtin_amdgcn_sched_barrier(0);
        if (ub0 + wv >= units) break;  // wave-uniform: no unit left for this wave
#pragma unroll
        for (int t = 0; t < MT; t++) {
            u32x4 xv = xr[t];
            if constexpr (XM == 2) xv = swiglu4(xv, xu[t]);
            float bk, xs;
            stage_q80<XB>(xv, xin && t < mt, xbuf[wv] + 512 * t, xbuf[wv] + 512 * t + 256, bk, xs);
            if ((lane & 7) == 0) {
                stats[wv][t][lane >> 3] = bk;
                stats[wv][t][8 + (lane >> 3)] = xs;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint16_t *ap = xbuf[wv] + aoff;
        u32x4 av[8];
#pragma unroll
        for (int b = 0; b < 8; b++) av[b] = *reinterpret_cast<const u32x4 *>(ap + 32 * b);
        floatx4 s0[4], s1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s0[i] = *reinterpret_cast<const floatx4 *>(&stats[wv][t0][4 * i]);
            s1[i] = *reinterpret_cast<const floatx4 *>(&stats[wv][t1][4 * i]);
        }
        floatx4 c[8];
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const uint32_t w0 = w.q[b >> 1][2 * (b & 1)] ^ 0x80808080u;
            const uint32_t w1 = w.q[b >> 1][2 * (b & 1) + 1] ^ 0x80808080u;
            const u32x4 bop = {w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu, (w1 >> 8) & 0x00FF00FFu};
            c[b] = mfma16x16x32_f16(av[b], bop, floatx4{0.f, 0.f, 0.f, 0.f});
        }
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const float d = f16_to_f32((w.h[b >> 1] >> (16 * (b & 1))) & 0xFFFFu);
            acc1[0] += (d * s0[b >> 2][b & 3]) * (c[b][0] + c[b][1]);
            acc1[1] += (d * s1[b >> 2][b & 3]) * (c[b][2] + c[b][3]);
            acc2[0] += d * s0[2 + (b >> 2)][b & 3];
            acc2[1] += d * s1[2 + (b >> 2)][b & 3];
        }
        // the next pass rewrites this wave's buffers only after these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // y = 2^24 * (code sums) - 128 * (offset terms), then summed over the waves
    if (2 * g < MT) red[wv][2 * g][r16] = acc1[0] * 16777216.0f - 128.0f * acc2[0];
    if (2 * g + 1 < MT) red[wv][2 * g + 1][r16] = acc1[1] * 16777216.0f - 128.0f * acc2[1];
    __syncthreads();
    if (tid < mt * 16) {
        const int t = tid >> 4, nn = tid & 15;
        float y = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) y += red[w2][t][nn];
        const int64_t row = (int64_t)tile * 16 + nn;
        if (row < a.n) {
            if (a.bias) y += a.bias[row];
            gemv_status(a, y, blockIdx.x == 0 && tid == 0);
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
            else
                reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
        }
    }
}

// ---------------------------------------------------------------------------------
// Q6_K decode kernel (m <= 2), gemv_q80_decode_kernel's organisation for the Q6_K tile16
// image (a unit is one 256-k super-block of a 16-row tile: four 768-byte chunks of 64 k,
// lane 16p + r holding 12 bytes of row r per chunk, then 16 int8 sub-block scales and the
// f16 d per row):
//  * staging lane l holds elements 4l .. 4l + 3 (32-block l / 8, 16-sub-block l / 4);
//    the blocks' powers of two and the sub-blocks' sums of x come out of DPP steps and
//    are read as wave-uniform scalars;
//  * MFMA j covers k 32j .. 32j + 31 (sub-blocks 2j, 2j + 1): A rows 4t + 2h + part hold
//    token t's hi / lo parts in the k-groups of half h only (the others read a zero pad),
//    so lane group t ends with the two sub-blocks' partial dots of token t;
//  * the 6-bit codes enter as f16 subnormals q * 2^-24 (exact), the -32 offset is
//    subtracted with the sub-block sums of x, in f32.
// ---------------------------------------------------------------------------------
template <bool XB>
__device__ __forceinline__ void stage_q6k(const u32x4 &raw, uint16_t *hi_plane, uint16_t *lo_plane, float &back,
                                          float &sum16) {
    const int lane = threadIdx.x & 63;
    float v0, v1, v2, v3;
    if (XB) {
        v0 = __uint_as_float(raw[0] << 16);
        v1 = __uint_as_float(raw[0] & 0xFFFF0000u);
        v2 = __uint_as_float(raw[1] << 16);
        v3 = __uint_as_float(raw[1] & 0xFFFF0000u);
    } else {
        v0 = __uint_as_float(raw[0]);
        v1 = __uint_as_float(raw[1]);
        v2 = __uint_as_float(raw[2]);
        v3 = __uint_as_float(raw[3]);
    }
    // max |x| of the 32-block (8 lanes); s, back and non-finite handling as in stage_q4k
    uint32_t m = __float_as_uint(absmax4(v0, v1, v2, v3));
    m = umax_dpp<0xB1>(m);
    m = umax_dpp<0x4E>(m);
    m = umax_dpp<0x141>(m);
    const uint32_t sb = min(0x86000000u - (m & 0x7F800000u), 0x7E800000u);
    const float s = __uint_as_float(sb);
    const uint32_t h01 = mix_hi2(v0, v1, s), h23 = mix_hi2(v2, v3, s);
    const uint32_t l01 = mix_lo2(v0, v1, s, h01), l23 = mix_lo2(v2, v3, s, h23);
    *reinterpret_cast<u32x2 *>(hi_plane + 4 * lane) = u32x2{h01, h23};
    *reinterpret_cast<u32x2 *>(lo_plane + 4 * lane) = u32x2{l01, l23};
    float sm = (v0 + v1) + (v2 + v3);
    sm = add_dpp<0xB1>(sm);
    sm = add_dpp<0x4E>(sm);  // the 16-sub-block's sum (4 lanes)
    back = __uint_as_float(0x7F000000u - sb);
    sum16 = sm;
}

// XM: activation kind, 0 f32, 1 bf16, 2 f32 gate | up pairs (SwiGLU prologue)
template <int WAVES, int UPW, int XM, int MT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q6k_decode_kernel(GemvArgs a) {
    constexpr bool XB = XM == 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = (int)blockIdx.x;
    // per wave and unit of a pass: [token, hi / lo][256] f16, then 256 zero halves
    constexpr int kBuf = MT * 512 + 256;
    __shared__ __attribute__((aligned(16))) uint16_t xbuf[WAVES][UPW][kBuf];
    __shared__ float red[WAVES][MT][16];
#pragma unroll
    for (int j = 0; j < UPW; j++)  // the wave's own pads, read later only by lanes of this wave
        if (lane < 32) *reinterpret_cast<u32x4 *>(&xbuf[wv][j][MT * 512 + 8 * lane]) = u32x4{0u, 0u, 0u, 0u};

    // A-operand row of this lane: lane & 15 = 4t + 2h + part, non-zero in the k-groups of half h
    const int r16 = lane & 15, kg = lane >> 4, g = lane >> 4;
    const int at = r16 >> 2, ah = (r16 >> 1) & 1, apart = r16 & 1;
    const bool own = at < MT && (kg >> 1) == ah;
    const int aoff = own ? (at * 2 + apart) * 256 + 8 * kg : MT * 512 + 8 * kg;

    const int units = (int)a.nblk, k = (int)a.k;
    constexpr int xe = XB ? 2 : 4;
    const int xrow = XM == 2 ? 2 * k : k;  // elements per token row of x
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.x);
    float acc1 = 0.f, acc2 = 0.f;  // lane group g < MT: token g
    int ub0 = 0;
    do {  // passes over K (units >= 1)
        u32x4 xr[UPW][MT], xu[XM == 2 ? UPW : 1][MT];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            const int u = min(ub0 + wv + j * WAVES, units - 1);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const uint8_t *p = xb + (size_t)(t * xrow + u * 256 + 4 * lane) * xe;
                if (XB) {
                    const u32x2 w2 = *reinterpret_cast<const u32x2 *>(p);
                    xr[j][t] = u32x4{w2[0], w2[1], 0u, 0u};
                } else {
                    xr[j][t] = *reinterpret_cast<const u32x4 *>(p);
                }
                if constexpr (XM == 2) xu[j][t] = *reinterpret_cast<const u32x4 *>(p + (size_t)k * 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep this issue order
        UnitQ6K w[UPW];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            load_unit(a, tile, min(ub0 + wv + j * WAVES, units - 1), w[j]);
            __builtin_amdgcn_sched_barrier(0);
        }
        float bk[UPW][MT], xs16[UPW][MT];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            if (ub0 + wv + j * WAVES >= units) break;  // wave-uniform
            uint16_t *buf = xbuf[wv][j];
#pragma unroll
            for (int t = 0; t < MT; t++) {
                u32x4 xv = xr[j][t];
                if constexpr (XM == 2) xv = swiglu4(xv, xu[j][t]);
                stage_q6k<XB>(xv, buf + 512 * t, buf + 512 * t + 256, bk[j][t], xs16[j][t]);
            }
        }
        // the wave's own LDS writes are read back by other lanes of the same wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            if (ub0 + wv + j * WAVES >= units) break;  // wave-uniform
            const uint16_t *ap = xbuf[wv][j] + aoff;
            u32x4 av[8];
#pragma unroll
            for (int b = 0; b < 8; b++) av[b] = *reinterpret_cast<const u32x4 *>(ap + 32 * b);
            floatx4 c[8];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const uint32_t A = w[j].q[cc][0], B = w[j].q[cc][1], C = w[j].q[cc][2];
                const u32x4 ba = {(A & 0x000F000Fu) | ((C << 4) & 0x00300030u), ((A >> 4) & 0x000F000Fu) | ((C << 2) & 0x00300030u),
                                  ((A >> 8) & 0x000F000Fu) | (C & 0x00300030u), ((A >> 12) & 0x000F000Fu) | ((C >> 2) & 0x00300030u)};
                const u32x4 bb = {(B & 0x000F000Fu) | ((C >> 4) & 0x00300030u), ((B >> 4) & 0x000F000Fu) | ((C >> 6) & 0x00300030u),
                                  ((B >> 8) & 0x000F000Fu) | ((C >> 8) & 0x00300030u),
                                  ((B >> 12) & 0x000F000Fu) | ((C >> 10) & 0x00300030u)};
                c[2 * cc] = mfma16x16x32_f16(av[2 * cc], ba, floatx4{0.f, 0.f, 0.f, 0.f});
                c[2 * cc + 1] = mfma16x16x32_f16(av[2 * cc + 1], bb, floatx4{0.f, 0.f, 0.f, 0.f});
            }
            // sub-block scales of row r16 (int8), the d of the super-block
            float t1 = 0.f, t2 = 0.f;
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint32_t sw = w[j].s[b >> 1] >> (16 * (b & 1));
                const float sa = (float)(int8_t)(sw & 0xFFu), sbv = (float)(int8_t)((sw >> 8) & 0xFFu);
                float back = lane_value(bk[j][0], 8 * b), xa = lane_value(xs16[j][0], 8 * b),
                      xbs = lane_value(xs16[j][0], 8 * b + 4);
                if constexpr (MT > 1) {
                    const float back1 = lane_value(bk[j][1], 8 * b), xa1 = lane_value(xs16[j][1], 8 * b),
                                xb1 = lane_value(xs16[j][1], 8 * b + 4);
                    back = g == 1 ? back1 : back;
                    xa = g == 1 ? xa1 : xa;
                    xbs = g == 1 ? xb1 : xbs;
                }
                t1 += back * (sa * (c[b][0] + c[b][1]) + sbv * (c[b][2] + c[b][3]));
                t2 += sa * xa + sbv * xbs;
            }
            const float d = f16_to_f32(w[j].d & 0xFFFFu);
            acc1 += d * t1;
            acc2 += d * t2;
        }
        ub0 += WAVES * UPW;
    } while (ub0 < units);

    // y = 2^24 * (code sums) - 32 * (offset terms), then summed over the waves
    if (g < MT) red[wv][g][r16] = acc1 * 16777216.0f - 32.0f * acc2;
    __syncthreads();
    if (tid < MT * 16) {
        const int t = tid >> 4, nn = tid & 15;
        float y = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) y += red[w2][t][nn];
        const int64_t row = (int64_t)tile * 16 + nn;
        if (row < a.n) {
            if (a.bias) y += a.bias[row];
            gemv_status(a, y, blockIdx.x == 0 && tid == 0);
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
            else
                reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
        }
        if (a.argmax_partial && t == 0) {
            // first-index argmax of this tile's 16 logits (the 16 lanes hold one tile)
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
// Q6_K batched decode (3 <= m <= 4 tokens, the rows past m zero): gemv_q6k_decode_kernel's
// unit math with all four token row groups in use (lane group t holds token t); each
// token's block powers of two and sub-block sums go through a per-wave LDS table (8 + 16
// floats) that its lane group reads with broadcast 16-byte loads.  One unit per wave
// and pass.
// ---------------------------------------------------------------------------------
template <int WAVES, int XM>
__global__ __launch_bounds__(WAVES * 64) void gemv_q6k_batch_kernel(GemvArgs a) {
    constexpr bool XB = XM == 1;
    constexpr int MT = 4;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = (int)blockIdx.x, mt = (int)a.m;
    constexpr int kBuf = MT * 512 + 256;
    __shared__ __attribute__((aligned(16))) uint16_t xbuf[WAVES][kBuf];
    __shared__ __attribute__((aligned(16))) float stats[WAVES][MT][24];  // [token][8 x 2^-s, 16 x sum]
    __shared__ float red[WAVES][MT][16];
    if (lane < 32) *reinterpret_cast<u32x4 *>(&xbuf[wv][MT * 512 + 8 * lane]) = u32x4{0u, 0u, 0u, 0u};

    const int r16 = lane & 15, kg = lane >> 4, g = kg;
    const int at = r16 >> 2, ah = (r16 >> 1) & 1, apart = r16 & 1;
    const int aoff = (kg >> 1) == ah ? (at * 2 + apart) * 256 + 8 * kg : MT * 512 + 8 * kg;

    const int units = (int)a.nblk, k = (int)a.k;
    constexpr int xe = XB ? 2 : 4;
    const int xrow = XM == 2 ? 2 * k : k;
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.x);
    float acc1 = 0.f, acc2 = 0.f;  // token g
    for (int ub0 = 0; ub0 < units; ub0 += WAVES) {
        const int u = min(ub0 + wv, units - 1);
        u32x4 xr[MT], xu[XM == 2 ? MT : 1];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const uint8_t *p = xb + (size_t)(t < mt ? t * xrow + u * 256 + 4 * lane : 0) * xe;  // past m: x[0]
            if (XB) {
                const u32x2 w2 = *reinterpret_cast<const u32x2 *>(p);
                xr[t] = u32x4{w2[0], w2[1], 0u, 0u};
            } else {
                xr[t] = *reinterpret_cast<const u32x4 *>(p);
            }
            if constexpr (XM == 2) xu[t] = *reinterpret_cast<const u32x4 *>(p + (size_t)k * 4);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep this issue order
        UnitQ6K w;
        load_unit(a, tile, u, w);
        __builtin_amdgcn_sched_barrier(0);
        if (ub0 + wv >= units) break;  // wave-uniform: no unit left for this wave
#pragma unroll
        for (int t = 0; t < MT; t++) {
            u32x4 xv = xr[t];
            if constexpr (XM == 2) xv = swiglu4(xv, xu[t]);
            if (t >= mt) xv = u32x4{0u, 0u, 0u, 0u};  // rows past the batch: zeros (bf16 or f32)
            float bk, x16;
            stage_q6k<XB>(xv, xbuf[wv] + 512 * t, xbuf[wv] + 512 * t + 256, bk, x16);
            if ((lane & 7) == 0) stats[wv][t][lane >> 3] = bk;
            if ((lane & 3) == 0) stats[wv][t][8 + (lane >> 2)] = x16;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint16_t *ap = xbuf[wv] + aoff;
        u32x4 av[8];
#pragma unroll
        for (int b = 0; b < 8; b++) av[b] = *reinterpret_cast<const u32x4 *>(ap + 32 * b);
        floatx4 st[6];
#pragma unroll
        for (int i = 0; i < 6; i++) st[i] = *reinterpret_cast<const floatx4 *>(&stats[wv][g][4 * i]);
        floatx4 c[8];
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const uint32_t A = w.q[cc][0], B = w.q[cc][1], C = w.q[cc][2];
            const u32x4 ba = {(A & 0x000F000Fu) | ((C << 4) & 0x00300030u), ((A >> 4) & 0x000F000Fu) | ((C << 2) & 0x00300030u),
                              ((A >> 8) & 0x000F000Fu) | (C & 0x00300030u), ((A >> 12) & 0x000F000Fu) | ((C >> 2) & 0x00300030u)};
            const u32x4 bb = {(B & 0x000F000Fu) | ((C >> 4) & 0x00300030u), ((B >> 4) & 0x000F000Fu) | ((C >> 6) & 0x00300030u),
                              ((B >> 8) & 0x000F000Fu) | ((C >> 8) & 0x00300030u),
                              ((B >> 12) & 0x000F000Fu) | ((C >> 10) & 0x00300030u)};
            c[2 * cc] = mfma16x16x32_f16(av[2 * cc], ba, floatx4{0.f, 0.f, 0.f, 0.f});
            c[2 * cc + 1] = mfma16x16x32_f16(av[2 * cc + 1], bb, floatx4{0.f, 0.f, 0.f, 0.f});
        }
        float t1 = 0.f, t2 = 0.f;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const uint32_t sw = w.s[b >> 1] >> (16 * (b & 1));
            const float sa = (float)(int8_t)(sw & 0xFFu), sbv = (float)(int8_t)((sw >> 8) & 0xFFu);
            const float back = st[b >> 2][b & 3];
            const float xa = st[2 + (2 * b) / 4][(2 * b) & 3], xbs = st[2 + (2 * b + 1) / 4][(2 * b + 1) & 3];
            t1 += back * (sa * (c[b][0] + c[b][1]) + sbv * (c[b][2] + c[b][3]));
            t2 += sa * xa + sbv * xbs;
        }
        const float d = f16_to_f32(w.d & 0xFFFFu);
        acc1 += d * t1;
        acc2 += d * t2;
        // the next pass rewrites this wave's buffers only after these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    red[wv][g][r16] = acc1 * 16777216.0f - 32.0f * acc2;
    __syncthreads();
    if (tid < mt * 16) {
        const int t = tid >> 4, nn = tid & 15;
        float y = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) y += red[w2][t][nn];
        const int64_t row = (int64_t)tile * 16 + nn;
        if (row < a.n) {
            if (a.bias) y += a.bias[row];
            gemv_status(a, y, blockIdx.x == 0 && tid == 0);
            if (a.y_bf16)
                reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
            else
                reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
        }
    }
}

// ---------------------------------------------------------------------------------
// Q4_K streaming decode GEMV (m <= 2, K <= 16 units, many tiles: the fused gate | up
// of an MLP).  gemv_q4k_decode_kernel's unit math inside gemv_stream_kernel's tile
// loop: wave w owns unit w of every tile, stages its activation slice once, keeps the
// 8 A operands and the slice statistics in registers, and loads its unit of the next
// tile before it computes the current one.
// ---------------------------------------------------------------------------------
template <int MT, bool XB>
__global__ __launch_bounds__(1024) void gemv_q4k_stream_kernel(GemvArgs a) {
    constexpr int WAVES = 16, kBuf = MT * 512 + 64;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ __attribute__((aligned(16))) uint16_t xbuf[WAVES][kBuf];
    __shared__ float red[2][WAVES][MT][16];  // [tile parity][wave][token][row]
    if (lane < 8)  // the wave's zero pad, read only by lanes of this wave
        *reinterpret_cast<u32x4 *>(&xbuf[wv][MT * 512 + 8 * lane]) = u32x4{0u, 0u, 0u, 0u};

    const int units = (int)a.nblk, k = (int)a.k;  // units <= 16 (host-checked)
    const bool has = wv < units;                  // wave-uniform
    const int ul = has ? wv : 0;
    const int G = lane >> 4, n = lane & 15, i = n & 3;
    const bool own = G == (n >> 2) && (i >> 1) < MT;
    const int aoff = own ? ((i >> 1) * 2 + (i & 1)) * 256 + 64 * G : MT * 512;
    const int64_t ntile = a.ntile, step = gridDim.x;
    int64_t tile = blockIdx.x;

    struct W {
        u32x4 q0, q1, h;
    };
    auto load = [&](int64_t t, W &w) {
        const uint8_t *qb = a.qs + ((size_t)t * units + ul) * 2048 + 16 * lane;
        w.q0 = ldg128(qb);
        w.q1 = ldg128(qb + 1024);
        w.h = ldg128(a.hdr + ((size_t)t * units + ul) * 256 + 16 * n);
    };
    // activation slice of unit ul (issued before the weights)
    constexpr int xe = XB ? 2 : 4;
    u32x4 xr[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const uint8_t *p = reinterpret_cast<const uint8_t *>(a.x) + ((size_t)t * k + ul * 256 + 4 * lane) * xe;
        if (XB) {
            const u32x2 w2 = *reinterpret_cast<const u32x2 *>(p);
            xr[t] = u32x4{w2[0], w2[1], 0u, 0u};
        } else {
            xr[t] = *reinterpret_cast<const u32x4 *>(p);
        }
    }
    W w0, w1;
    if (has) load(tile, w0);
    XStat st[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) stage_q4k<XB>(xr[t], xbuf[wv] + 512 * t, xbuf[wv] + 512 * t + 256, st[t]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    u32x4 av[4][2];
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
        for (int h = 0; h < 2; h++) av[q4][h] = *reinterpret_cast<const u32x4 *>(xbuf[wv] + aoff + 32 * h + 8 * q4);
    const uint32_t hsel = 0u - (uint32_t)(G >> 1);  // all ones for sub-blocks 4..7

    int par = 0;
    uint64_t run_key = 0;  // thread 0: the largest argmax key of this workgroup's tiles
    auto body = [&](W &cur, W &nxt) {
        const int64_t next = tile + step;
        if (has) load(next < ntile ? next : ntile - 1, nxt);
        float acc1[MT], acc2[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) acc1[t] = acc2[t] = 0.0f;
        if (has) {
            // header: d | dmin, scales[0..3], scales[4..7], scales[8..11] (BlockQ4K packing,
            // get_scale_min_k4, crates/nn-core/src/layers/quantized/linear.rs:166-176)
            const u32x4 &h = cur.h;
            const float d = f16_to_f32(h[0] & 0xFFFFu), dmin = f16_to_f32(h[0] >> 16);
            const uint32_t S1 = h[1], S2 = h[2], S3 = h[3];
            const uint32_t scw =
                ((S1 & 0x3F3F3F3Fu) & ~hsel) | (((S3 & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) & hsel);
            const uint32_t mnw =
                ((S2 & 0x3F3F3F3Fu) & ~hsel) | ((((S3 >> 4) & 0x0F0F0F0Fu) | ((S2 >> 2) & 0x30303030u)) & hsel);
            const uint32_t scp = scw >> (16 * (G & 1)), mnp = mnw >> (16 * (G & 1));
            const float sc_lo = (float)(scp & 0xFFu), sc_hi = 0.0625f * (float)((scp >> 8) & 0xFFu);
            const float mn_lo = (float)(mnp & 0xFFu), mn_hi = (float)((mnp >> 8) & 0xFFu);
            floatx4 clo = {0.f, 0.f, 0.f, 0.f}, chi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const u32x4 q = q4 < 2 ? cur.q0 : cur.q1;
                const uint32_t w0 = q[2 * (q4 & 1)], w1 = q[2 * (q4 & 1) + 1];
                const uint32_t w0s = w0 >> 8, w1s = w1 >> 8;
                const u32x4 blo = {w0 & 0x000F000Fu, w0s & 0x000F000Fu, w1 & 0x000F000Fu, w1s & 0x000F000Fu};
                const u32x4 bhi = {w0 & 0x00F000F0u, w0s & 0x00F000F0u, w1 & 0x00F000F0u, w1s & 0x00F000F0u};
                clo = mfma16x16x32_f16(av[q4][0], blo, clo);
                chi = mfma16x16x32_f16(av[q4][1], bhi, chi);
            }
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const float T = (sc_lo * st[t].b_lo) * (clo[2 * t] + clo[2 * t + 1]) +
                                (sc_hi * st[t].b_hi) * (chi[2 * t] + chi[2 * t + 1]);
                acc1[t] = d * T;
                acc2[t] = dmin * (mn_lo * st[t].xs_lo + mn_hi * st[t].xs_hi);
            }
        }
        // y = 2^24 * (code sums) - (min terms), summed over the lane groups, then the waves
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const float v = sum_rows(acc1[t] * 16777216.0f - acc2[t]);
            if (lane < 16) red[par][wv][t][lane] = v;
        }
        __syncthreads();  // the other buffer is rewritten only after the next tile's barrier
        if (tid < MT * 16) {
            const int t = tid >> 4, nn = tid & 15;
            float y = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < WAVES; w2++) y += red[par][w2][t][nn];
            const int64_t row = tile * 16 + nn;
            if (a.swiglu_out) {
                store_swiglu_pair(a, y, t, tile, nn, tile == 0 && tid == 0);
            } else if (row < a.n) {
                if (a.bias) y += a.bias[row];
                gemv_status(a, y, tile == 0 && tid == 0);
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[(int64_t)t * a.n + row] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[(int64_t)t * a.n + row] = y;
            }
            if (a.argmax_partial && t == 0) {
                uint64_t key = row < a.n ? (y != y ? ~0ull : argmax_key(y, (uint32_t)row)) : 0ull;
                for (int o = 8; o > 0; o >>= 1) {
                    uint64_t other = __shfl_xor(key, o, 16);
                    key = other > key ? other : key;
                }
                if (nn == 0) run_key = key > run_key ? key : run_key;
            }
        }
        par ^= 1;
        tile = next;
    };
    for (;;) {
        body(w0, w1);
        if (tile >= ntile) break;
        body(w1, w0);
        if (tile >= ntile) break;
    }
    // one argmax key per workgroup (the host reduces gridDim.x keys)
    if (a.argmax_partial && tid == 0) a.argmax_partial[blockIdx.x] = run_key;
    __builtin_amdgcn_s_waitcnt(0);  // the last (unused) prefetch
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
    const int r = lane & 15, p = lane >> 4;  // row r of the tile, byte group p (sub-blocks 2p, 2p + 1)
    const int64_t row = tile * 16 + r;
    const uint8_t *qb = qs + job * 2048 + 16 * lane;
    const u32x4 h = ldg128(hdr + job * 256 + 16 * r);
    if (row >= n) return;
    const float d = f16_to_f32(h[0] & 0xFFFFu), dmin = f16_to_f32(h[0] >> 16);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(&h) + 4;
    // get_scale_min_k4 (crates/nn-core/src/layers/quantized/linear.rs:166-176)
    auto gsm = [&](int j, uint32_t &sc, uint32_t &mn) {
        if (j < 4) {
            sc = sb[j] & 63;
            mn = sb[j + 4] & 63;
        } else {
            sc = (sb[j + 4] & 0xF) | ((sb[j - 4] >> 6) << 4);
            mn = (sb[j + 4] >> 4) | ((sb[j] >> 6) << 4);
        }
    };
    uint32_t scl, mnl, sch, mnh;
    gsm(2 * p, scl, mnl);
    gsm(2 * p + 1, sch, mnh);
    // BlockQ4K::dequantize (linear.rs:73-89): d1 = d * sc, m1 = dmin * m, v = d1 * q - m1
    const float d1 = d * (float)scl, m1 = dmin * (float)mnl;
    const float d2 = d * (float)sch, m2 = dmin * (float)mnh;
    float *o = out + row * k + b * 256 + 64 * p;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const u32x4 q = ldg128(qb + 1024 * hh);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t word = q[w];
            // stored byte order (e0, e2, e1, e3) of bytes i0 .. i0 + 3
            const uint32_t e[4] = {word & 0xFF, (word >> 16) & 0xFF, (word >> 8) & 0xFF, word >> 24};
            const int i0 = 16 * hh + 4 * w;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                o[i0 + c] = d1 * (float)(e[c] & 0xF) - m1;
                o[32 + i0 + c] = d2 * (float)(e[c] >> 4) - m2;
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
    // eight independent loads in flight per thread and round (one round up to 8192 keys)
    for (int64_t base = threadIdx.x; base < count; base += 8 * (int64_t)blockDim.x) {
        unsigned long long v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t i = base + (int64_t)u * blockDim.x;
            v[u] = i < count ? partial[i] : 0ull;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) key = v[u] > key ? v[u] : key;
    }
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
// SwiGLU glue of the MLP when the down projection does not take gate | up directly
// (more than 2 tokens): h[t, i] = silu(gu[t, i]) * gu[t, I + i]; thread 0 of block
// 0 clears the status that the output check sets afterwards.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void swiglu_kernel(const float *gu, int64_t m, int64_t inter, float *h,
                                                     int32_t *status, int interleaved8) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (status && i == 0) *status = NNQ_OK;
    if (i >= m * inter) return;
    const int64_t t = i / inter, c = i % inter;
    // gate column and its up column: halves [gate | up], or 8 gate then 8 up per 16
    const int64_t gc = interleaved8 ? (c / 8) * 16 + c % 8 : c, uc = interleaved8 ? gc + 8 : inter + c;
    const float g = gu[t * 2 * inter + gc];
    h[i] = g / (1.0f + expf(-g)) * gu[t * 2 * inter + uc];
}

// check_output_finite (crates/nn-core/src/layers/nan_check.rs:113-140) on the device:
// any NaN or infinite value of y sets *status to NNQ_ERR_NON_FINITE
__global__ __launch_bounds__(256) void nonfinite_kernel(const void *y, int y_bf16, int64_t count, int32_t *status) {
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
        const float v = y_bf16 ? bf16_to_f32(reinterpret_cast<const uint16_t *>(y)[i]) : reinterpret_cast<const float *>(y)[i];
        bad |= !(fabsf(v) <= 3.402823466e38f);
    }
    if (__any(bad) && (threadIdx.x & 63) == 0) *status = NNQ_ERR_NON_FINITE;
}

int launch_swiglu(const float *gu, int64_t m, int64_t inter, float *h, int32_t *status, void *stream,
                  int interleaved8) {
    const int64_t n = m * inter;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, gu, m,
                       inter, h, status, interleaved8);
    return (int)hipGetLastError();
}

int launch_nonfinite_check(const void *y, int y_bf16, int64_t count, int32_t *status, void *stream) {
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 1024);
    hipLaunchKernelGGL(nonfinite_kernel, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0,
                       (hipStream_t)stream, y, y_bf16, count, status);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------
// decode (m <= 2): 8 waves with just enough units each to cover K in one pass
// (longer K loops over passes)
// streaming kernel: workgroups = CUs (every one loops over tiles); dynamic LDS holds
// the staged activation of all of K
static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;  // idempotent: concurrent first calls store the same value
    }
    return cus[dev];
}

template <int FMT, int WAVES, int UPW>
static int launch_stream_t(const GemvArgs &a, int64_t units, int cus, void *stream) {
    constexpr int GRAN = Fmt<FMT>::kSumGran;
    const int64_t kc = units * 256;
    const size_t lds = (size_t)a.m * kc * 4 + (size_t)a.m * (kc / GRAN) * 4 + (size_t)a.m * (kc / 32) * 4;
    const int64_t grid = a.ntile < cus ? a.ntile : cus;
    if (a.argmax_count) *a.argmax_count = grid;
    hipLaunchKernelGGL((gemv_stream_kernel<FMT, WAVES, UPW>), dim3((unsigned)grid), dim3(WAVES * 64), lds,
                       (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

template <int WAVES, int UPW, int XM>
static int launch_q80_decode_x(const GemvArgs &a, void *stream) {
    if (a.m == 1)
        hipLaunchKernelGGL((gemv_q80_decode_kernel<WAVES, UPW, XM, 1>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a.qs, a.hdr, a.x, (int)(a.nblk / 8), (int)a.k, (int)a.m, a);
    else
        hipLaunchKernelGGL((gemv_q80_decode_kernel<WAVES, UPW, XM, 2>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a.qs, a.hdr, a.x, (int)(a.nblk / 8), (int)a.k, (int)a.m, a);
    return (int)hipGetLastError();
}
template <int WAVES, int UPW>
static int launch_q80_decode_t(const GemvArgs &a, void *stream) {
    if (a.x_swiglu) return launch_q80_decode_x<WAVES, UPW, 2>(a, stream);
    return a.x_bf16 ? launch_q80_decode_x<WAVES, UPW, 1>(a, stream) : launch_q80_decode_x<WAVES, UPW, 0>(a, stream);
}
template <int WAVES, int MT>
static int launch_q80_batch_t(const GemvArgs &a, void *stream) {
    if (a.x_swiglu)
        hipLaunchKernelGGL((gemv_q80_batch_kernel<WAVES, 2, MT>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    else if (a.x_bf16)
        hipLaunchKernelGGL((gemv_q80_batch_kernel<WAVES, 1, MT>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL((gemv_q80_batch_kernel<WAVES, 0, MT>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    return (int)hipGetLastError();
}
// Q8_0 batches of 3-8 tokens: 4 or 8 token rows, waves of one unit per pass: 16 when
// the grid has at most two tiles per CU and K is over 8 units, else 8 (4 for K of up
// to 4 units).  4096x4096, 8 tokens: 7.9 us (12.5 in the block GEMV form).
static int launch_q80_batch(const GemvArgs &a, int64_t units, void *stream) {
    const bool w16 = a.ntile <= 512 && units > 8;
    if (a.m <= 4)
        return units <= 4 ? launch_q80_batch_t<4, 4>(a, stream)
                          : (w16 ? launch_q80_batch_t<16, 4>(a, stream) : launch_q80_batch_t<8, 4>(a, stream));
    return units <= 4 ? launch_q80_batch_t<4, 8>(a, stream)
                      : (w16 ? launch_q80_batch_t<16, 8>(a, stream) : launch_q80_batch_t<8, 8>(a, stream));
}

// Q8_0 decode shapes: one wave per unit up to 16 units, then 16 waves of up to
// three units (longer K loops over passes).
static int launch_q80_decode(const GemvArgs &a, int64_t units, void *stream) {
    if (units <= 4) return launch_q80_decode_t<4, 1>(a, stream);
    if (units <= 8) return launch_q80_decode_t<8, 1>(a, stream);
    if (units <= 16) return launch_q80_decode_t<16, 1>(a, stream);
    if (units <= 32) return launch_q80_decode_t<16, 2>(a, stream);
    return launch_q80_decode_t<16, 3>(a, stream);
}

template <int WAVES, int UPW, int XM>
static int launch_q6k_decode_x(const GemvArgs &a, void *stream) {
    if (a.m == 1)
        hipLaunchKernelGGL((gemv_q6k_decode_kernel<WAVES, UPW, XM, 1>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL((gemv_q6k_decode_kernel<WAVES, UPW, XM, 2>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    return (int)hipGetLastError();
}
template <int WAVES, int UPW>
static int launch_q6k_decode_t(const GemvArgs &a, void *stream) {
    if (a.x_swiglu) return launch_q6k_decode_x<WAVES, UPW, 2>(a, stream);
    return a.x_bf16 ? launch_q6k_decode_x<WAVES, UPW, 1>(a, stream) : launch_q6k_decode_x<WAVES, UPW, 0>(a, stream);
}
// Q6_K decode shapes: as Q8_0's, with 8 waves of two units for K of 9-16 units when the
// grid has more than two tiles per CU
static int launch_q6k_decode(const GemvArgs &a, int64_t units, void *stream) {
    if (units <= 4) return launch_q6k_decode_t<4, 1>(a, stream);
    if (units <= 8) return launch_q6k_decode_t<8, 1>(a, stream);
    if (units <= 16) return a.ntile > 512 ? launch_q6k_decode_t<8, 2>(a, stream) : launch_q6k_decode_t<16, 1>(a, stream);
    if (units <= 32) return launch_q6k_decode_t<16, 2>(a, stream);
    return launch_q6k_decode_t<16, 3>(a, stream);
}

template <int WAVES>
static int launch_q6k_batch_t(const GemvArgs &a, void *stream) {
    if (a.x_swiglu)
        hipLaunchKernelGGL((gemv_q6k_batch_kernel<WAVES, 2>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    else if (a.x_bf16)
        hipLaunchKernelGGL((gemv_q6k_batch_kernel<WAVES, 1>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL((gemv_q6k_batch_kernel<WAVES, 0>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                           (hipStream_t)stream, a);
    return (int)hipGetLastError();
}
// Q6_K batches of 3-4 tokens: waves of one unit per pass, as the Q8_0 batched kernel
static int launch_q6k_batch(const GemvArgs &a, int64_t units, void *stream) {
    if (units <= 4) return launch_q6k_batch_t<4>(a, stream);
    return a.ntile <= 512 && units > 8 ? launch_q6k_batch_t<16>(a, stream) : launch_q6k_batch_t<8>(a, stream);
}

template <int FMT>
static int launch_wave(const GemvArgs &a, int64_t units, void *stream) {
    // many tiles per CU (the LM head): loop over tiles with the activation staged once
    // per workgroup and the next tile's weights in flight during the current one's math
    if (!a.x_swiglu) {
        const int cus = device_cus();
        if (a.ntile >= 4 * (int64_t)cus && a.m * units * 256 <= 8192 && units <= 16) {
            if constexpr (FMT == FQ6K) {
                const int64_t kc = units * 256;
                const size_t lds = (size_t)a.m * kc * 4 + (size_t)a.m * (kc / 16) * 4 + (size_t)a.m * (kc / 32) * 4;
                const int64_t grid = a.ntile < cus ? a.ntile : cus;
                if (a.argmax_count) *a.argmax_count = grid;
                if (a.m == 1)
                    hipLaunchKernelGGL((gemv_q6k_stream_kernel<1>), dim3((unsigned)grid), dim3(1024), lds,
                                       (hipStream_t)stream, a);
                else
                    hipLaunchKernelGGL((gemv_q6k_stream_kernel<2>), dim3((unsigned)grid), dim3(1024), lds,
                                       (hipStream_t)stream, a);
                return (int)hipGetLastError();
            } else {
                return launch_stream_t<FMT, 16, 1>(a, units, cus, stream);
            }
        }
    }
    static_assert(FMT == FQ80 || FMT == FQ6K, "Q4_K has its own decode launcher");
    if constexpr (FMT == FQ80)
        return launch_q80_decode(a, units, stream);
    else
        return launch_q6k_decode(a, units, stream);
}

template <int WAVES, int UPW, int XM, int MT>
static int launch_q4k_decode_k(const GemvArgs &a, void *stream) {
    hipLaunchKernelGGL((gemv_q4k_decode_kernel<WAVES, UPW, XM, MT>), dim3((unsigned)a.ntile), dim3(WAVES * 64), 0,
                       (hipStream_t)stream, a.qs, a.hdr, a.x, (int)a.nblk, (int)a.m, a);
    return (int)hipGetLastError();
}
template <int WAVES, int UPW, int XM>
static int launch_q4k_decode_x(const GemvArgs &a, void *stream) {
    return a.m == 1 ? launch_q4k_decode_k<WAVES, UPW, XM, 1>(a, stream) : launch_q4k_decode_k<WAVES, UPW, XM, 2>(a, stream);
}
template <int WAVES, int UPW>
static int launch_q4k_decode_t(const GemvArgs &a, void *stream) {
    if (a.x_swiglu) return launch_q4k_decode_x<WAVES, UPW, 2>(a, stream);
    return a.x_bf16 ? launch_q4k_decode_x<WAVES, UPW, 1>(a, stream) : launch_q4k_decode_x<WAVES, UPW, 0>(a, stream);
}

// Q4_K decode shapes, from sweeps on MI355X: K of up to 16 units takes 8 waves of
// up to 2 units, longer K 16 waves of up to 4 units (then passes); one tile per
// workgroup (two tiles per workgroup, sharing the staged activation, measured slower).
static int device_cus();

// batches of 3-4 tokens: four token rows (two MFMA sets over the same B operands), 8
// waves of up to 3 units or 16 of 2 (the staging buffers of four tokens fill LDS sooner):
// 4 tokens at 4096x12288 in 11.4 us (two passes of two: 15.0)
template <int WAVES, int UPW>
static int launch_q4k_batch_t(const GemvArgs &a, void *stream) {
    return a.x_bf16 ? launch_q4k_decode_k<WAVES, UPW, 1, 4>(a, stream) : launch_q4k_decode_k<WAVES, UPW, 0, 4>(a, stream);
}

static int launch_q4k_decode(const GemvArgs &a, void *stream) {
    const int64_t units = a.nblk;
    if (a.m > 2) {
        if (a.x_swiglu || a.swiglu_out) return (int)hipErrorInvalidValue;
        if (units <= 4) return launch_q4k_batch_t<4, 1>(a, stream);
        if (units <= 8) return launch_q4k_batch_t<8, 1>(a, stream);
        if (units <= 16) return launch_q4k_batch_t<8, 2>(a, stream);
        return a.ntile <= 512 ? launch_q4k_batch_t<16, 2>(a, stream) : launch_q4k_batch_t<8, 3>(a, stream);
    }
    // many tiles per CU and K <= 16 units: one workgroup per CU loops over tiles
    if (!a.x_swiglu && units <= 16) {
        const int cus = device_cus();
        if (a.ntile >= 4 * (int64_t)cus) {
            const dim3 grid((unsigned)(a.ntile < cus ? a.ntile : cus));
            if (a.argmax_count) *a.argmax_count = grid.x;
            if (a.m == 1) {
                if (a.x_bf16)
                    hipLaunchKernelGGL((gemv_q4k_stream_kernel<1, true>), grid, dim3(1024), 0, (hipStream_t)stream, a);
                else
                    hipLaunchKernelGGL((gemv_q4k_stream_kernel<1, false>), grid, dim3(1024), 0, (hipStream_t)stream, a);
            } else {
                if (a.x_bf16)
                    hipLaunchKernelGGL((gemv_q4k_stream_kernel<2, true>), grid, dim3(1024), 0, (hipStream_t)stream, a);
                else
                    hipLaunchKernelGGL((gemv_q4k_stream_kernel<2, false>), grid, dim3(1024), 0, (hipStream_t)stream, a);
            }
            return (int)hipGetLastError();
        }
    }
    if (units <= 4) return launch_q4k_decode_t<4, 1>(a, stream);
    if (units <= 8) return launch_q4k_decode_t<8, 1>(a, stream);
    if (units <= 16) return launch_q4k_decode_t<8, 2>(a, stream);
    const int64_t need = (units + 15) / 16;
    if (need <= 2) return launch_q4k_decode_t<16, 2>(a, stream);
    if (need <= 3) return launch_q4k_decode_t<16, 3>(a, stream);
    return launch_q4k_decode_t<16, 4>(a, stream);
}

// tokens per launch: Q4_K and Q6_K up to 4, Q8_0 up to 8 (callers run passes)
int launch_gemv(int fmt, const GemvArgs &a, void *stream) {
    const int mmax = fmt == FQ80 ? 8 : 4;
    if (a.m < 1 || a.m > mmax) return (int)hipErrorInvalidValue;
    const int64_t units = fmt == FQ80 ? a.nblk / 8 : a.nblk;
    switch (fmt) {
    case FQ4K: return launch_q4k_decode(a, stream);
    case FQ80: return a.m <= 2 ? launch_wave<FQ80>(a, units, stream) : launch_q80_batch(a, units, stream);
    case FQ6K: return a.m <= 2 ? launch_wave<FQ6K>(a, units, stream) : launch_q6k_batch(a, units, stream);
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
