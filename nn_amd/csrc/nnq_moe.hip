// GPT-OSS MXFP4 mixture-of-experts layer on gfx950 (QuantizedDecoderLayer::moe_forward /
// expert_forward, crates/nn-gptoss/src/quantized_model.rs:99-194).
//
// Pipeline (all on the device, no host synchronisation):
//   route    softmax over the router logits, first-index top-k by total order,
//            renormalisation (crates/nn-core/src/dyn_tensor/ops_ext/sorting.rs:22-104)
//   permute  per-expert counts, offsets and a stable (token, slot) order of the
//            assignments: expert e's rows are its tokens in ascending order, as the
//            host grouping of moe_forward (:157-169) builds them; a launch of its own
//            only for batches over 1024 tokens, else done by gate_up per expert
//   gate_up  grouped GEMM over experts: x rows of the expert x W_gu[e] (+ bias), with
//            the SwiGLU epilogue clamp(silu(gate), -limit, limit) * up fused in
//   down     grouped GEMM over experts: h x W_down[e] (+ bias)
//   combine  y[t] = sum of w * y_e[t] over the token's experts in ascending expert
//            order, the order of moe_forward's index_add (:171-189)
//
// Weights.  MXFP4 blocks run along the output dimension (F5): row k of an expert
// matrix has one E8M0 scale per 32 output columns, and the byte that holds columns
// 2c (high nibble) and 2c + 1 (low nibble) shares one scale.  One
// v_cvt_scalef32_pk_bf16_fp4 turns such a byte into the two bf16 values times the
// row's scale, exactly (a 2-bit significand times a power of two); two v_perm_b32
// then regroup the pairs of consecutive rows into the MFMA B operand of the even and
// the odd column.  A wave owns one 32-column block: per 32 rows it loads 8 code bytes
// and 8 scale bytes per lane and feeds two 16x16x32 bf16 MFMAs per 16 token rows.
// Activations: bf16 input is used as is (exact); f32 input and the SwiGLU output h
// are carried as bf16 hi + lo pairs (two MFMAs, ~2^-17 relative).
#include <algorithm>
#include <type_traits>

#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

namespace {

inline size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

struct MoeScratch {
    uint32_t *ti;        // [T][k] expert of each slot
    float *tw;           // [T][k] renormalised weight of each slot
    int32_t *off;        // [E + 1] first sorted row of each expert
    int32_t *stok;       // [T * k] token of each sorted row
    int32_t *pos;        // [T][k] sorted row of each slot
    uint16_t *xb;        // [2][T][H] bf16 hi / lo of an f32 input
    uint16_t *hb;        // [2][T * k][I] bf16 hi / lo of the SwiGLU output
    float *yb;           // [T * k][H] expert outputs (+ bias) per sorted row
};

MoeScratch carve(void *base, int64_t T, int64_t E, int64_t H, int64_t I, int k, int x_bf16) {
    uint8_t *b = reinterpret_cast<uint8_t *>(base);
    MoeScratch s;
    const size_t A = (size_t)T * k;
    s.ti = reinterpret_cast<uint32_t *>(b);
    b += al256(A * 4);
    s.tw = reinterpret_cast<float *>(b);
    b += al256(A * 4);
    s.off = reinterpret_cast<int32_t *>(b);
    b += al256((size_t)(E + 1) * 4);
    s.stok = reinterpret_cast<int32_t *>(b);
    b += al256(A * 4);
    s.pos = reinterpret_cast<int32_t *>(b);
    b += al256(A * 4);
    s.xb = reinterpret_cast<uint16_t *>(b);
    b += x_bf16 ? 0 : al256((size_t)2 * T * H * 2);
    s.hb = reinterpret_cast<uint16_t *>(b);
    b += al256((size_t)2 * A * I * 2);
    s.yb = reinterpret_cast<float *>(b);
    return s;
}

// f32::total_cmp key (crates/nn-core/src/dyn_tensor/ops_ext/sorting.rs:63-72)
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t b = __float_as_int(f);
    return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

__device__ __forceinline__ uint16_t bf16_rne(float f) { return (uint16_t)f32_to_bf16_bits(f); }

// The byte's two bf16 values (low nibble first) times the scale whose E8M0 exponent
// sits at bits 23-30 of `scale_bits` (the instruction reads only that field).
template <int BYTE>
__device__ __forceinline__ uint32_t fp4_pair(uint32_t codes, uint32_t scale_bits) {
    return __builtin_bit_cast(uint32_t,
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, __uint_as_float(scale_bits), BYTE));
}

// Row i = 0..7 of this lane's 8 rows: code byte i, scale byte i moved to bits 23-30.
// Device scale bytes mean 2^(e - 127) for every e: GPT-OSS's byte 0 (2^-126,
// crates/nn-gptoss/src/quantize.rs:84-90) is stored as byte 1 at upload, and the nn-core
// OCP byte 0 (2^-127, crates/nn-core/src/layers/quantized/mxfp4.rs:177-186) stays 0.
__device__ __forceinline__ void fp4_rows(u32x2 codes, u32x2 sc, uint32_t r[8]) {
    r[0] = fp4_pair<0>(codes[0], sc[0] << 23);
    r[1] = fp4_pair<1>(codes[0], sc[0] << 15);
    r[2] = fp4_pair<2>(codes[0], sc[0] << 7);
    r[3] = fp4_pair<3>(codes[0], sc[0] >> 1);
    r[4] = fp4_pair<0>(codes[1], sc[1] << 23);
    r[5] = fp4_pair<1>(codes[1], sc[1] << 15);
    r[6] = fp4_pair<2>(codes[1], sc[1] << 7);
    r[7] = fp4_pair<3>(codes[1], sc[1] >> 1);
}

// B operands of the 16x16x32 MFMA for the even (column 2c) and odd (2c + 1) columns.
__device__ __forceinline__ void fp4_b_operands(const uint8_t *codes, const uint8_t *scales, int lane, u32x4 &be,
                                               u32x4 &bo) {
    const u32x2 c = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(codes + 8 * lane));
    const u32x2 s = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(scales + 8 * (lane >> 4)));
    uint32_t r[8];
    fp4_rows(c, s, r);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        bo[j] = __builtin_amdgcn_perm(r[2 * j + 1], r[2 * j], 0x05040100u);  // low halves: column 2c + 1
        be[j] = __builtin_amdgcn_perm(r[2 * j + 1], r[2 * j], 0x07060302u);  // high halves: column 2c
    }
}

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

}  // namespace

// ---------------------------------------------------------------------------------
// routing: one wave per token, lane c holds logits c, c + 64, ... (E <= 256; more: moe_route_any_kernel)
// ---------------------------------------------------------------------------------
// Wave-wide reductions without LDS round trips: DPP steps inside each 16-lane row
// (quad xor 1, xor 2, half-row mirror, row mirror), then the row swaps.  Every lane
// ends with the result.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}
__device__ __forceinline__ uint64_t swap_rows_max(uint64_t v, bool pair32) {
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    const auto l = pair32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                          : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = pair32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                          : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return max_u64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_u64(v, dpp_u64<0xB1>(v));
    v = max_u64(v, dpp_u64<0x4E>(v));
    v = max_u64(v, dpp_u64<0x141>(v));
    v = max_u64(v, dpp_u64<0x140>(v));
    v = swap_rows_max(v, false);
    return swap_rows_max(v, true);
}
// fmaxf over the wave (a NaN lane is ignored unless every lane is NaN, in any order)
__device__ __forceinline__ float wave_max_f32(float x) {
    x = fmaxf(x, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(x))));
    x = fmaxf(x, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(x))));
    x = fmaxf(x, __uint_as_float(dpp_u32<0x141>(__float_as_uint(x))));
    x = fmaxf(x, __uint_as_float(dpp_u32<0x140>(__float_as_uint(x))));
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += (int)dpp_u32<0xB1>((uint32_t)v);
    v += (int)dpp_u32<0x4E>((uint32_t)v);
    v += (int)dpp_u32<0x141>((uint32_t)v);
    v += (int)dpp_u32<0x140>((uint32_t)v);
    const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = (int)(a[0] + a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return (int)(b[0] + b[1]);
}

// `logits` holds nsplit slabs [T][E] whose sum in slab order, plus `bias` when given,
// are the logits (the router's K parts; nsplit = 1 and no bias: logits given)
__global__ __launch_bounds__(256) void moe_route_kernel(const float *logits, int nsplit, const float *bias, int64_t T,
                                                        int E, int k, uint32_t *ti, float *tw, uint32_t *ti_out,
                                                        float *tw_out) {
    __shared__ __attribute__((aligned(16))) float ex[4][256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + wv;
    if (t >= T) return;  // wave-uniform; no barrier below
    float v[4];
    float mx = -INFINITY;
    int ninf = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = lane + 64 * j;
        if (c < E) {
            float lv = logits[t * E + c];
            for (int sp = 1; sp < nsplit; sp++) lv += logits[((int64_t)sp * T + t) * E + c];
            if (bias) lv += bias[c];
            v[j] = lv;
        } else {
            v[j] = -INFINITY;
        }
        mx = fmaxf(mx, v[j]);
        ninf += (c < E && v[j] == INFINITY);
    }
    mx = wave_max_f32(mx);
    ninf = wave_sum_i32(ninf);
    // probs = softmax(logits) (DynTensor::softmax, crates/nn-core/src/dyn_tensor/softmax.rs:30-60,
    // called at crates/nn-gptoss/src/quantized_model.rs:140): exp(x - max) / sum, with the sum
    // accumulated in index order
    float p[4];
    if (mx == -INFINITY || mx == INFINITY) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            p[j] = (mx == INFINITY && v[j] == INFINITY) ? 1.0f / (float)ninf : 0.0f;
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = lane + 64 * j;
            const float e = expf(v[j] - mx);
            if (c < E) ex[wv][c] = e;
            p[j] = e;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // the index-order sum, the same in every lane: 16-byte broadcast reads (ex rows
        // are 16-byte aligned and 256 long), additions one after another
        float sum = -0.0f;
        for (int c = 0; c < E; c += 4) {
            const floatx4 q = *reinterpret_cast<const floatx4 *>(&ex[wv][c]);
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (c + j < E) sum = sum + q[j];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) p[j] = p[j] / sum;
    }
    // top-k: descending by total order, ties to the lowest index (key = orderable value, ~index)
    bool taken[4] = {false, false, false, false};
    if (k > 8) {
        // any k (up to E): each selection is written as it is made, its probability kept
        // in the wave's LDS row (the softmax sum has been read from it already), and the
        // weights normalised by the sum of the selected values in selection order
        float ssum = -0.0f;
        for (int s = 0; s < k; s++) {
            uint64_t best = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = lane + 64 * j;
                if (c < E && !taken[j]) {
                    const uint32_t o = (uint32_t)total_key(p[j]) ^ 0x80000000u;
                    const uint64_t key = ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)c);
                    best = key > best ? key : best;
                }
            }
            best = wave_max_u64(best);
            const uint32_t c = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu);
            float pv = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (lane + 64 * j == (int)c) {
                    taken[j] = true;
                    pv = p[j];
                }
            }
            pv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), __builtin_amdgcn_readfirstlane((int)(c & 63))));
            ssum = ssum + pv;
            if (lane == 0) {
                ex[wv][s] = pv;
                ti[t * k + s] = c;
                if (ti_out) ti_out[t * k + s] = c;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int s = lane; s < k; s += 64) {
            const float w = ex[wv][s] / ssum;
            tw[t * k + s] = w;
            if (tw_out) tw_out[t * k + s] = w;
        }
        return;
    }
    uint32_t idx[8];
    float val[8];
    for (int s = 0; s < k; s++) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = lane + 64 * j;
            if (c < E && !taken[j]) {
                const uint32_t o = (uint32_t)total_key(p[j]) ^ 0x80000000u;
                const uint64_t key = ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)c);
                best = key > best ? key : best;
            }
        }
        best = wave_max_u64(best);
        const uint32_t c = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu);
        float pv = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (lane + 64 * j == (int)c) {
                taken[j] = true;
                pv = p[j];
            }
        }
        // broadcast the chosen probability from its lane
        pv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), __builtin_amdgcn_readfirstlane((int)(c & 63))));
        idx[s] = c;
        val[s] = pv;
    }
    float ssum = -0.0f;
    for (int s = 0; s < k; s++) ssum = ssum + val[s];
    if (lane < k) {
        uint32_t ci = 0;
        float cv = 0.0f;
        for (int s = 0; s < k; s++)
            if (s == lane) {
                ci = idx[s];
                cv = val[s];
            }
        const float w = cv / ssum;
        ti[t * k + lane] = ci;
        tw[t * k + lane] = w;
        if (ti_out) ti_out[t * k + lane] = ci;
        if (tw_out) tw_out[t * k + lane] = w;
    }
}

// Routing for E > 256 experts: the same computation as moe_route_kernel with the
// token's values in LDS (one row of E floats per wave, dynamic shared memory); the
// selection rounds mark a chosen expert by key 0 (every probability key is above it).
__global__ __launch_bounds__(256) void moe_route_any_kernel(const float *logits, int nsplit, const float *bias,
                                                            int64_t T, int E, int k, uint32_t *ti, float *tw,
                                                            uint32_t *ti_out, float *tw_out) {
    extern __shared__ __attribute__((aligned(16))) float rowbuf[];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + wv;
    if (t >= T) return;  // wave-uniform; no barrier below
    // per wave: E values (then keys), and for k > 8 the k selected values
    float *v = rowbuf + (size_t)wv * (E + (k > 8 ? k : 0));
    uint32_t *key = reinterpret_cast<uint32_t *>(v);
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    float mx = -INFINITY;
    int ninf = 0;
    for (int c = lane; c < E; c += 64) {
        float lv = logits[t * E + c];
        for (int sp = 1; sp < nsplit; sp++) lv += logits[((int64_t)sp * T + t) * E + c];
        if (bias) lv += bias[c];
        v[c] = lv;
        mx = fmaxf(mx, lv);
        ninf += lv == INFINITY;
    }
    mx = wave_max_f32(mx);
    ninf = wave_sum_i32(ninf);
    // probabilities (softmax with the sum in index order, as moe_route_kernel)
    if (mx == -INFINITY || mx == INFINITY) {
        for (int c = lane; c < E; c += 64) v[c] = (mx == INFINITY && v[c] == INFINITY) ? 1.0f / (float)ninf : 0.0f;
        wave_sync();
    } else {
        for (int c = lane; c < E; c += 64) v[c] = expf(v[c] - mx);
        wave_sync();
        float sum = -0.0f;
        for (int c = 0; c < E; c++) sum = sum + v[c];
        wave_sync();
        for (int c = lane; c < E; c += 64) v[c] = v[c] / sum;
        wave_sync();
    }
    // top-k: descending by total order, ties to the lowest index; the probability keys
    // replace the values in LDS (a chosen expert's key becomes 0)
    uint32_t idx[8];
    float val[8];
    float ssum = -0.0f;
    for (int c = lane; c < E; c += 64) key[c] = (uint32_t)total_key(v[c]) ^ 0x80000000u;
    wave_sync();
    for (int s = 0; s < k; s++) {
        uint64_t best = 0;
        for (int c = lane; c < E; c += 64) {
            const uint64_t kk = ((uint64_t)key[c] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)c);
            if (key[c] != 0u) best = kk > best ? kk : best;
        }
        best = wave_max_u64(best);
        const uint32_t c = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu);
        const uint32_t o = (uint32_t)(best >> 32) ^ 0x80000000u;  // back to the total-order key
        // the key -> float inverse of total_key
        const int32_t b = (int32_t)o;
        const float pv = __int_as_float(b ^ (int32_t)((uint32_t)(b >> 31) >> 1));
        ssum = ssum + pv;  // the selected values summed in selection order
        if (k > 8) {
            // any k: written as selected, the values kept after the keys
            if (lane == 0) {
                v[E + s] = pv;
                ti[t * k + s] = c;
                if (ti_out) ti_out[t * k + s] = c;
            }
        } else {
            idx[s] = c;
            val[s] = pv;
        }
        wave_sync();
        if (lane == 0) key[c] = 0u;
        wave_sync();
    }
    if (k > 8) {
        for (int s = lane; s < k; s += 64) {
            const float w = v[E + s] / ssum;
            tw[t * k + s] = w;
            if (tw_out) tw_out[t * k + s] = w;
        }
        return;
    }
    if (lane < k) {
        uint32_t ci = 0;
        float cv = 0.0f;
        for (int s = 0; s < k; s++)
            if (s == lane) {
                ci = idx[s];
                cv = val[s];
            }
        const float w = cv / ssum;
        ti[t * k + lane] = ci;
        tw[t * k + lane] = w;
        if (ti_out) ti_out[t * k + lane] = ci;
        if (tw_out) tw_out[t * k + lane] = w;
    }
}

// One workgroup of 1024 threads, one token per thread per chunk of 1024 tokens.  For
// each expert a ballot gives every token its rank among the wave's tokens that chose
// the expert; per-wave counts in LDS turn that into the rank over all earlier tokens.
// Expert e's rows are then its tokens in ascending order (stable by token, the order
// moe_forward's grouping loop builds, crates/nn-gptoss/src/quantized_model.rs:157-169).
// Experts go in groups of 256 (the per-wave count table); the running per-expert
// totals live in dynamic shared memory (E ints).
template <int k>
__global__ __launch_bounds__(1024) void moe_permute_kernel(const uint32_t *ti, int64_t T, int E, int32_t *off,
                                                           int32_t *stok, int32_t *pos) {
    __shared__ int32_t wcnt[16][256];
    extern __shared__ int32_t base[];  // [E]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int e = tid; e < E; e += 1024) base[e] = 0;
    __syncthreads();
    // with one chunk (T <= 1024) each thread keeps its token's experts and ranks in
    // registers for the final scatter; longer batches pass the ranks through pos
    const bool one_chunk = T <= 1024;
    uint32_t ex[k];
    int32_t myrank[k];
    for (int64_t t0 = 0; t0 < T; t0 += 1024) {
        const int64_t t = t0 + tid;
#pragma unroll
        for (int s = 0; s < k; s++) ex[s] = t < T ? ti[t * k + s] : 0xFFFFFFFFu;
        for (int g0 = 0; g0 < E; g0 += 256) {
            const int ge = min(256, E - g0);
            int32_t rk[k];
#pragma unroll
            for (int s = 0; s < k; s++) rk[s] = 0;
            // waves past the batch only publish zero counts (a short batch leaves most of
            // the 16 waves idle: 256 tokens use 4)
            const bool live = t0 + (int64_t)wv * 64 < T;  // wave-uniform
            for (int e = 0; e < ge; e++) {
                if (!live) {
                    if (lane == 0) wcnt[wv][e] = 0;
                    continue;
                }
                const uint32_t ee = (uint32_t)(g0 + e);
                bool hit = false;
#pragma unroll
                for (int s = 0; s < k; s++) hit |= ex[s] == ee;
                const uint64_t m = __ballot(hit);
                const int32_t r = __popcll(m & lt);
#pragma unroll
                for (int s = 0; s < k; s++)
                    if (ex[s] == ee) rk[s] = r;
                if (lane == 0) wcnt[wv][e] = __popcll(m);
            }
            __syncthreads();
            // per expert (one per thread): wcnt[w][e] becomes the count of earlier tokens,
            // base plus the waves before w (the 16 loads independent of each other)
            for (int e = tid; e < ge; e += 1024) {
                int32_t c[16];
#pragma unroll
                for (int w = 0; w < 16; w++) c[w] = wcnt[w][e];
                int32_t run = base[g0 + e];
#pragma unroll
                for (int w = 0; w < 16; w++) {
                    wcnt[w][e] = run;
                    run += c[w];
                }
                base[g0 + e] = run;
            }
            __syncthreads();
            if (t < T)
#pragma unroll
                for (int s = 0; s < k; s++)
                    if (ex[s] >= (uint32_t)g0 && ex[s] < (uint32_t)(g0 + ge)) {
                        const int32_t r = wcnt[wv][ex[s] - g0] + rk[s];  // rank within the expert; offset below
                        if (one_chunk)
                            myrank[s] = r;
                        else
                            pos[t * k + s] = r;
                    }
            __syncthreads();  // wcnt is rewritten by the next group / chunk
        }
    }
    if (tid < 64) {
        // exclusive scan of the expert counts, 256 at a time: lane l holds experts
        // c0 + 4l .. c0 + 4l + 3, the carry is the total of the earlier groups
        int32_t carry = 0;
        for (int c0 = 0; c0 < E; c0 += 256) {
            int32_t c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c0 + 4 * tid + j;
                c[j] = e < E ? base[e] : 0;
                sum += c[j];
            }
            int32_t before = sum;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int32_t v = __shfl_up(before, o, 64);
                if (tid >= o) before += v;
            }
            const int32_t total = __shfl(before, 63, 64);
            before += carry - sum;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c0 + 4 * tid + j;
                if (e < E) {
                    base[e] = before;
                    off[e] = before;
                }
                before += c[j];
            }
            carry += total;
        }
        if (tid == 0) off[E] = carry;  // the total
    }
    __syncthreads();
    if (one_chunk) {
        if (tid < T)
#pragma unroll
            for (int s = 0; s < k; s++) {
                const int32_t p = myrank[s] + base[ex[s]];
                pos[tid * k + s] = p;
                stok[p] = tid;
            }
        return;
    }
    for (int64_t i = tid; i < T * k; i += 1024) {
        const int32_t p = pos[i] + base[ti[i]];
        pos[i] = p;
        stok[p] = (int32_t)(i / k);
    }
}

// moe_permute_kernel for any k (k > 8): the token's experts are read from ti inside the
// expert loop instead of registers, and the ranks go through pos.
__global__ __launch_bounds__(1024) void moe_permute_any_kernel(const uint32_t *ti, int64_t T, int E, int k,
                                                               int32_t *off, int32_t *stok, int32_t *pos) {
    __shared__ int32_t wcnt[16][256];
    extern __shared__ int32_t base[];  // [E]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int e = tid; e < E; e += 1024) base[e] = 0;
    __syncthreads();
    for (int64_t t0 = 0; t0 < T; t0 += 1024) {
        const int64_t t = t0 + tid;
        for (int g0 = 0; g0 < E; g0 += 256) {
            const int ge = min(256, E - g0);
            const bool live = t0 + (int64_t)wv * 64 < T;  // wave-uniform
            for (int e = 0; e < ge; e++) {
                if (!live) {
                    if (lane == 0) wcnt[wv][e] = 0;
                    continue;
                }
                const uint32_t ee = (uint32_t)(g0 + e);
                int sh = -1;  // the token routes to an expert at most once
                if (t < T)
                    for (int s = 0; s < k; s++)
                        if (ti[t * k + s] == ee) sh = s;
                const uint64_t m = __ballot(sh >= 0);
                if (sh >= 0) pos[t * k + sh] = __popcll(m & lt);  // rank within the wave
                if (lane == 0) wcnt[wv][e] = __popcll(m);
            }
            __syncthreads();
            for (int e = tid; e < ge; e += 1024) {
                int32_t c[16];
#pragma unroll
                for (int w = 0; w < 16; w++) c[w] = wcnt[w][e];
                int32_t run = base[g0 + e];
#pragma unroll
                for (int w = 0; w < 16; w++) {
                    wcnt[w][e] = run;
                    run += c[w];
                }
                base[g0 + e] = run;
            }
            __syncthreads();
            if (t < T)
                for (int s = 0; s < k; s++) {
                    const uint32_t ex = ti[t * k + s];
                    if (ex >= (uint32_t)g0 && ex < (uint32_t)(g0 + ge)) pos[t * k + s] += wcnt[wv][ex - g0];
                }
            __syncthreads();
        }
    }
    if (tid < 64) {
        int32_t carry = 0;
        for (int c0 = 0; c0 < E; c0 += 256) {
            int32_t c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c0 + 4 * tid + j;
                c[j] = e < E ? base[e] : 0;
                sum += c[j];
            }
            int32_t before = sum;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int32_t v = __shfl_up(before, o, 64);
                if (tid >= o) before += v;
            }
            const int32_t total = __shfl(before, 63, 64);
            before += carry - sum;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c0 + 4 * tid + j;
                if (e < E) {
                    base[e] = before;
                    off[e] = before;
                }
                before += c[j];
            }
            carry += total;
        }
        if (tid == 0) off[E] = carry;
    }
    __syncthreads();
    for (int64_t i = tid; i < T * k; i += 1024) {
        const int32_t p = pos[i] + base[ti[i]];
        pos[i] = p;
        stok[p] = (int32_t)(i / k);
    }
}

// ---------------------------------------------------------------------------------
// router Linear: logits[t, e] = x[t, :] . W[e, :] + b[e] (Linear::forward, x @ W^T + bias,
// crates/nn-core/src/layers/core_layers.rs:118-140, as moe_forward calls it at
// crates/nn-gptoss/src/quantized_model.rs:138), f32 products and sums on the
// 16x16x4 f32 MFMA.  Workgroup (token tile, expert tile, K part z) = 16 tokens x 16
// experts over K part z of KS; its 4 waves take quarters of the part and are summed
// in wave order; a part's sum goes to slab z of `out` (KS > 1, the routing kernel
// adds the slabs in order and the bias) or, with the bias, straight to the logits
// (KS = 1).  Lane 16g + r loads 4 consecutive k of token r and of expert r, and MFMA
// j takes element j, so every k meets its own pair once.  Block (0, 0, 0) clears the
// call's status (set later by the output check).
// ---------------------------------------------------------------------------------
constexpr int kRouterBatch = 4;  // 16-k chunks whose loads a wave issues together

template <bool XB>
__global__ __launch_bounds__(256) void router_logits_kernel(const void *x, int64_t T, int64_t H, const float *W,
                                                            const float *bias, int E, float *out, int32_t *status) {
    __shared__ floatx4 red[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t t0 = (int64_t)blockIdx.x * 16;
    const int e0 = (int)blockIdx.y * 16, KS = (int)gridDim.z, z = (int)blockIdx.z;
    if (status && blockIdx.x == 0 && blockIdx.y == 0 && z == 0 && threadIdx.x == 0) *status = NNQ_OK;
    const int64_t trow = min(t0 + r, T - 1);
    const int erow = min(e0 + r, E - 1);
    const int nch = (int)(H / 16);
    const int p0 = z * nch / KS, p1 = (z + 1) * nch / KS;  // this part's chunks
    const int c0 = p0 + wv * (p1 - p0) / 4, c1 = p0 + (wv + 1) * (p1 - p0) / 4;
    const float *wp = W + (int64_t)erow * H + 4 * g;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int cb = c0; cb < c1; cb += kRouterBatch) {
        float xv[kRouterBatch][4];
        floatx4 wv4[kRouterBatch];
#pragma unroll
        for (int u = 0; u < kRouterBatch; u++) {
            const int c = min(cb + u, c1 - 1);  // past the wave's range: a repeat, not used
            if (XB) {
                const u32x2 b2 = *reinterpret_cast<const u32x2 *>(reinterpret_cast<const uint16_t *>(x) + trow * H +
                                                                  (int64_t)c * 16 + 4 * g);
                xv[u][0] = __uint_as_float(b2[0] << 16);
                xv[u][1] = __uint_as_float(b2[0] & 0xFFFF0000u);
                xv[u][2] = __uint_as_float(b2[1] << 16);
                xv[u][3] = __uint_as_float(b2[1] & 0xFFFF0000u);
            } else {
                const floatx4 f = *reinterpret_cast<const floatx4 *>(reinterpret_cast<const float *>(x) + trow * H +
                                                                     (int64_t)c * 16 + 4 * g);
                xv[u][0] = f[0], xv[u][1] = f[1], xv[u][2] = f[2], xv[u][3] = f[3];
            }
            wv4[u] = *reinterpret_cast<const floatx4 *>(wp + (int64_t)c * 16);
        }
#pragma unroll
        for (int u = 0; u < kRouterBatch; u++) {
            if (cb + u >= c1) break;  // wave-uniform
#pragma unroll
            for (int j = 0; j < 4; j++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[u][j], wv4[u][j], acc, 0, 0, 0);
        }
    }
    red[wv][lane] = acc;
    __syncthreads();
    if (wv == 0) {
        floatx4 sum = red[0][lane];
#pragma unroll
        for (int w = 1; w < 4; w++) sum += red[w][lane];
        // lane 16g + r holds D[4g + i][r]: token t0 + 4g + i, expert e0 + r
        const int e = e0 + r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t t = t0 + 4 * g + i;
            if (t < T && e < E) {
                if (KS == 1)
                    out[t * E + e] = sum[i] + (bias ? bias[e] : 0.0f);
                else
                    out[((int64_t)z * T + t) * E + e] = sum[i];
            }
        }
    }
}

// K parts of the router: enough workgroups to spread the loads, at most 4 batches per wave
inline int router_parts(int64_t T, int64_t H, int E) {
    const int64_t tiles = ((T + 15) / 16) * ((E + 15) / 16), nch = H / 16;
    int64_t ks = std::max<int64_t>((256 + tiles - 1) / tiles, (nch + 4 * 4 * kRouterBatch - 1) / (4 * 4 * kRouterBatch));
    return (int)std::min<int64_t>(std::min<int64_t>(ks, nch), 64);
}

// f32 activations -> bf16 hi / lo planes
__global__ __launch_bounds__(256) void moe_split_kernel(const float *x, int64_t n, uint16_t *xb) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    const uint16_t h = bf16_rne(v);
    xb[i] = h;
    xb[n + i] = bf16_rne(v - bf16_to_f32(h));
}

// ---------------------------------------------------------------------------------
// expert GEMMs (grouped over experts)
// ---------------------------------------------------------------------------------
struct MoeRun {
    const uint16_t *xa[2];  // activation planes (bf16), rows of H
    int64_t A;              // assignments (T * k): rows of the sorted buffers
    float limit;
    // gate_up finds its expert's rows itself (no permute launch) when perm is set:
    // ti[T][k] the routed experts; the expert's group-0 workgroup writes off and pos
    const uint32_t *ti;
    int64_t T;
    int k;
    int perm;
};

// batches up to this many tokens skip the permute launch (the expert's token list, one
// int per token, sits in LDS)
constexpr int kMoeInPermT = 1024;
constexpr size_t kMoePermLds = (size_t)kMoeInPermT * 4 + 64 * 4;

// Column streams.  gate_up: stream s = the pair of 32-column blocks (gate s, up I/32 + s),
// both owned by one wave, so the SwiGLU epilogue needs no exchange; down: stream s =
// block s.  Workgroup (expert, group g) takes streams [g S / G, (g + 1) S / G), one per
// wave (rounds when a group has more streams than waves); every wave streams its
// blocks' weight codes over all of K, PF chunks ahead in registers.
// The expert's token rows (up to 64 per pass, P bf16 planes) are shared through an LDS
// ring of NBUF chunks of CKB k-blocks (32 rows of K each), copied NBUF - 1 chunks ahead
// with global_load_lds (one barrier per chunk).  With CKB = 3 a chunk's copies are
// exactly one 16-byte granule per thread and plane, so no copy is wasted.
// Scales (SL): each wave stages the E8M0 scales of its blocks for all of K in its own
// LDS area at the start of a round (1 KB per load instruction) and reads the 8 bytes
// of its rows per k-block from there, so the per-k-block loads are the codes alone.
constexpr int kMoeWaves = 12;
constexpr int kMoeGroups = 8;  // groups per expert (E = 32: one workgroup per CU)
constexpr size_t kMoeLdsMax = 160 * 1024;

template <int P, int CKB>
struct MoeK {
    static constexpr int NTH = kMoeWaves * 64;
    static constexpr int NBUF = CKB == 3 ? 3 : 4;  // LDS ring depth (chunks)
    static constexpr int PF = NBUF - 1;            // weight prefetch distance (chunks)
    static constexpr int ROWG = CKB * 4;           // 16-byte granules per row and chunk
    static constexpr int ACH = P * 64 * ROWG;      // granules per chunk
    static constexpr int LPA = (ACH + NTH - 1) / NTH;  // copy instructions per thread and chunk
    static constexpr int BUF = LPA * NTH * 16;
    static constexpr size_t RING = (size_t)NBUF * BUF;
    static_assert(CKB == 1 || CKB == 3, "chunk widths");
};

// k-blocks of scales staged per block: K / 32 rounded up to whole 1 KB loads
__host__ __device__ constexpr int64_t moe_kbp(int64_t KB) { return (KB + 31) / 32 * 32; }

template <int P, bool GU, int CKB, bool SL>
constexpr size_t moe_lds(int64_t KB) {
    return MoeK<P, CKB>::RING + (SL ? (size_t)kMoeWaves * (GU ? 2 : 1) * moe_kbp(KB) * 32 : 0) + (GU ? kMoePermLds : 0);
}

// slot of the 16-byte granule kc of row r among the row's granules of a chunk: rows r
// and r + 2 .. r + 6 land in different banks; the xor stays inside aligned groups of 4
__device__ __forceinline__ int moe_slot(int kc, int r) { return kc ^ ((r >> 1) & 3); }

// One 16-byte-per-lane copy from a buffer resource straight into LDS (the wave's 64
// granules land contiguously at `lds`); an offset past the resource's range copies zeros.
// (The host pass has no such builtin and would drop the kernels' launch stubs.)
__device__ inline void moe_copy16_lds(__amdgpu_buffer_rsrc_t r, unsigned char *lds, uint32_t voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voff, soff, 0, 0);
#endif
}

__host__ __device__ constexpr int moe_streams(bool gu, int64_t H, int64_t I) { return (int)(gu ? I / 32 : H / 32); }

template <int P, bool GU, int CKB, bool SL>
__global__ __launch_bounds__(kMoeWaves * 64) void moe_stream_kernel(MoeDev d, MoeScratch sc, MoeRun run) {
    using C = MoeK<P, CKB>;
    constexpr int NBW = GU ? 2 : 1, NTH = C::NTH, LPA = C::LPA, NBUF = C::NBUF, PF = C::PF;
    constexpr int WPS = CKB * NBW * (SL ? 1 : 2);  // weight loads per thread and chunk
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int64_t H = d.H, I = d.I;
    const int64_t K = GU ? H : I, KB = K / 32, NB = GU ? 2 * I / 32 : H / 32;
    const int KBP = (int)moe_kbp(KB);
    const int S = moe_streams(GU, H, I);
    // Workgroup ids go round-robin over the 8 XCDs; when the count allows, XCD x gets a
    // contiguous run of (expert, group) items, i.e. whole experts, so an expert's
    // activation rows are read into one XCD's L2 only.
    const int nwg = (int)gridDim.x, bid = (int)blockIdx.x;
    const int item = (nwg % 8 == 0) ? (bid % 8) * (nwg / 8) + bid / 8 : bid;
    const int64_t e = item / kMoeGroups, g = item % kMoeGroups;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the expert's tokens in ascending order (in-kernel permutation only)
    int32_t *tok_s = reinterpret_cast<int32_t *>(smem + C::RING + (SL ? (size_t)kMoeWaves * NBW * KBP * 32 : 0));
    int32_t r0, ne;
    if (GU && run.perm) {
        // moe_permute_kernel's result for this expert: r0 = the assignments to lower
        // experts, the rows = its tokens in ascending order (a token routes to an expert
        // at most once), counted per wave and ordered by lane rank
        int32_t *wc = tok_s + kMoeInPermT;  // [2][kMoeWaves]
        const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
        int below = 0;
        ne = 0;
        for (int64_t t0 = 0; t0 < run.T; t0 += NTH) {
            const int64_t t = t0 + tid;
            bool hit = false;
            if (t < run.T)
                for (int q = 0; q < run.k; q++) {
                    const uint32_t x = run.ti[t * run.k + q];
                    below += x < (uint32_t)e ? 1 : 0;
                    hit |= x == (uint32_t)e;
                }
            const uint64_t m = __ballot(hit);
            if (lane == 0) wc[wv] = __popcll(m);
            __syncthreads();
            int before = ne, total = 0;
            for (int w = 0; w < kMoeWaves; w++) {
                const int c = wc[w];
                before += w < wv ? c : 0;
                total += c;
            }
            if (hit) tok_s[before + __popcll(m & lt)] = (int32_t)t;
            ne += total;
            __syncthreads();  // wc is rewritten by the next chunk
        }
        below = wave_sum_i32(below);
        if (lane == 0) wc[kMoeWaves + wv] = below;
        __syncthreads();  // also publishes tok_s
        r0 = 0;
        for (int w = 0; w < kMoeWaves; w++) r0 += wc[kMoeWaves + w];
        // the same in every lane: scalar registers for the epilogue's uniform addressing
        r0 = __builtin_amdgcn_readfirstlane(r0);
        ne = __builtin_amdgcn_readfirstlane(ne);
        if (g == 0) {
            // for the down and combine launches: the expert's first row, the total, and
            // each assignment's row
            if (tid == 0) {
                sc.off[e] = r0;
                if (e == d.E - 1) sc.off[d.E] = (int32_t)run.A;
            }
            for (int i = tid; i < ne; i += NTH) {
                const int64_t t = tok_s[i];
                for (int q = 0; q < run.k; q++)
                    if (run.ti[t * run.k + q] == (uint32_t)e) sc.pos[t * run.k + q] = r0 + i;
            }
        }
    } else {
        r0 = sc.off[e];
        ne = sc.off[e + 1] - r0;
    }
    if (ne == 0) return;  // workgroup-uniform
    const int p = lane >> 4, l16 = lane & 15;
    const int s_lo = (int)(g * S / kMoeGroups), s_hi = (int)((g + 1) * S / kMoeGroups);
    const int nch = (int)(KB / CKB);  // K / 32 is a multiple of CKB (the host picks CKB)
    unsigned char *scl = smem + C::RING + (size_t)wv * NBW * KBP * 32;  // this wave's scales (SL)

    for (int32_t m0 = 0; m0 < ne; m0 += 64) {
        const int mtn = (ne - m0) >= 64 ? 4 : (ne - m0 + 15) / 16;  // live row tiles
        // copy sources of this pass: granule c -> (plane, row, slot); chunk ch at + ch * CKB * 32 k.
        // A 32-bit byte offset per lane from one uniform base (the planes of an activation
        // are one buffer: x hi / lo at xa[0] and xa[0] + T H, h hi / lo at hb and hb + A I;
        // the host keeps them under 4 GB), so a copy address costs one VGPR, not two
        const unsigned char *abase = reinterpret_cast<const unsigned char *>(GU ? run.xa[0] : sc.hb);
        const int64_t pstride = GU ? (run.xa[1] ? run.xa[1] - run.xa[0] : 0) : run.A * I;  // elements per plane
        // the copies go through a buffer resource over the activation's planes: a granule of a
        // row tile with no live rows gets an offset past the range, so its copy instruction is
        // still issued (every wave issues the same batches: the vmcnt waits below count them)
        // but reads nothing and writes zeros that no MFMA reads
        // (the planes span at most 2^31 bytes under the size limits and token chunking, so
        // live offsets stay below the record count and 2^31 plus the chunk's scalar offset
        // is past it without wrapping)
        const int64_t abytes = 2 * ((int64_t)(P - 1) * pstride + (GU ? run.T * H : run.A * I));
        const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<unsigned char *>(abase), 0, (int)(uint32_t)min(abytes, (int64_t)0x80000000), 0x00020000);
        uint32_t aoff[LPA];
#pragma unroll
        for (int j = 0; j < LPA; j++) {
            const int c = min(j * NTH + tid, C::ACH - 1);
            const int pl = c / (64 * C::ROWG), rem = c % (64 * C::ROWG);
            const int r = rem / C::ROWG, slot = rem % C::ROWG;
            const int kc = moe_slot(slot, r);  // the row's 16-byte granule held at this slot
            const int32_t rr = r0 + m0 + min(r, ne - m0 - 1);  // rows past the expert repeat its last row
            const int64_t tok = GU ? (run.perm ? tok_s[rr - r0] : sc.stok[rr]) : 0;
            aoff[j] = r < 16 * mtn ? (uint32_t)(2 * ((int64_t)pl * pstride + (GU ? tok * H : (int64_t)rr * I) + 8 * kc))
                                   : 0x80000000u;
        }
        auto issue = [&](int ch) {
            const int cv = min(ch, nch - 1);  // past the end: re-copy the last chunk
            unsigned char *buf = smem + (size_t)(ch % NBUF) * C::BUF;
#pragma unroll
            for (int j = 0; j < LPA; j++)
                moe_copy16_lds(ars, buf + (size_t)(j * NTH + wv * 64) * 16, aoff[j], cv * CKB * 64);
        };
        const int nround = (s_hi - s_lo + kMoeWaves - 1) / kMoeWaves;
        for (int rd = 0; rd < nround; rd++) {
            const int st = s_lo + rd * kMoeWaves + wv;
            const bool active = st < s_hi;  // idle waves still copy and join the barriers
            // buffer resources on the wave's blocks (scalar registers, range-checked): a
            // per-lane offset plus a scalar per-k-block offset, no per-load address VALU
            __amdgpu_buffer_rsrc_t rq[NBW], rs[NBW];
            int64_t nbv[NBW];
#pragma unroll
            for (int b = 0; b < NBW; b++) {
                nbv[b] = active ? (GU ? (b == 0 ? st : I / 32 + st) : st) : 0;
                rq[b] = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint8_t *>((GU ? d.gu_q : d.dn_q) + (e * NB + nbv[b]) * KB * 512), 0, (int)(KB * 512),
                    0x00020000);
                rs[b] = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint8_t *>((GU ? d.gu_s : d.dn_s) + (e * NB + nbv[b]) * KB * 32), 0, (int)(KB * 32),
                    0x00020000);
            }
            const int qo = 8 * lane, so = 8 * p;
            // weight ring in registers: slot (ch % (PF + 1)) holds chunk ch
            u32x2 wq[PF + 1][CKB][NBW], ws[SL ? 1 : PF + 1][CKB][NBW];
            auto wload = [&](int ch, int slot) {
                const int cv = min(ch, nch - 1);
#pragma unroll
                for (int j = 0; j < CKB; j++)
#pragma unroll
                    for (int b = 0; b < NBW; b++) {
                        const int kb = cv * CKB + j;
                        // cache policy 2: non-temporal (every weight byte is read once per call)
                        wq[slot][j][b] =
                            __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rq[b], qo, kb * 512, 2));
                        if constexpr (!SL)
                            ws[slot][j][b] =
                                __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs[b], so, kb * 32, 2));
                    }
            };
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __syncthreads();  // the previous round / pass has finished reading the ring
            if constexpr (SL) {
                // this wave's scales for all of K: 1 KB per load (the last one clamped inside
                // the block's KB * 32 bytes); complete before the first chunk's wait
#pragma unroll
                for (int b = 0; b < NBW; b++)
                    for (int i = 0; i < KBP / 32; i++) {
                        const int64_t off = min((int64_t)i * 1024 + 16 * lane, KB * 32 - 16);
                        __builtin_amdgcn_global_load_lds(
                            (const __attribute__((address_space(1))) void *)((GU ? d.gu_s : d.dn_s) +
                                                                             (e * NB + nbv[b]) * KB * 32 + off),
                            (__attribute__((address_space(3))) void *)(scl + (size_t)b * KBP * 32 + (size_t)i * 1024),
                            16, 0, 0);
                    }
            }
            // Every step issues the same batch on every wave: the weights of chunk t + PF
            // (clamped into range; idle waves load block 0), then the copies of chunk
            // t + NBUF - 1.  The prologue runs steps t = 1 - NBUF .. -1 the same way, so
            // before chunk ch is read exactly NBUF - 2 batches follow its copies.
            auto step = [&](int t, int wslot) {
                wload(max(t + PF, 0), wslot);
                issue(t + NBUF - 1);
            };
#pragma unroll
            for (int t = 1 - NBUF; t < 0; t++) step(t, ((t + PF) % (PF + 1) + (PF + 1)) % (PF + 1));
            // lane holds rows 4p + i of each tile; acc[.][.][0]: column 2 * l16 of the block,
            // [1]: 2 * l16 + 1
            auto epilogue = [&](auto &acc) {
                constexpr int MTN = (int)std::extent<std::remove_reference_t<decltype(acc)>, 1>::value;
                // the bases, the row range and the row lengths pass through an empty asm
                // here, so the row offsets and row masks below are formed after the K loop
                // (hoisted above it, they were 16 live 64-bit offsets and 16 masks per lane
                // across the loop, i.e. register spills)
                uint16_t *hbp = sc.hb;
                float *ybp = sc.yb;
                const float *gub = d.gu_b, *dnb = d.dn_b;
                int64_t Ie = I, He = H;
                int32_t r0e = r0, nee = ne, m0e = m0;
                asm volatile("" : "+s"(hbp), "+s"(ybp), "+s"(gub), "+s"(dnb), "+s"(Ie), "+s"(He), "+s"(r0e), "+s"(nee),
                             "+s"(m0e));
                if (GU) {
                    const int64_t col0 = (int64_t)st * 32;
#pragma unroll
                    for (int mt = 0; mt < MTN; mt++) {
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int32_t r = m0e + mt * 16 + 4 * p + i;
                            if (r >= nee) continue;
                            uint32_t hh = 0, hl = 0;
#pragma unroll
                            for (int o = 0; o < 2; o++) {
                                const int64_t c = col0 + 2 * l16 + o;
                                const float gt = acc[0][mt][o][i] + gub[e * 2 * Ie + c];
                                const float up = acc[1][mt][o][i] + gub[e * 2 * Ie + Ie + c];
                                // silu (crates/nn-core/src/dyn_tensor/ops/math.rs:140), clamped to +-limit
                                float sg = gt / (1.0f + expf(-gt));
                                sg = sg < -run.limit ? -run.limit : (sg > run.limit ? run.limit : sg);
                                const float h = sg * up;
                                const uint32_t bh = bf16_rne(h);
                                hh |= bh << (16 * o);
                                hl |= (uint32_t)bf16_rne(h - bf16_to_f32(bh)) << (16 * o);
                            }
                            const int64_t o2 = (int64_t)(r0e + r) * Ie + col0 + 2 * l16;
                            *reinterpret_cast<uint32_t *>(hbp + o2) = hh;
                            *reinterpret_cast<uint32_t *>(hbp + run.A * Ie + o2) = hl;
                        }
                    }
                } else {
                    const int64_t col0 = (int64_t)st * 32 + 2 * l16;
                    const float b0 = dnb[e * He + col0], b1 = dnb[e * He + col0 + 1];
#pragma unroll
                    for (int mt = 0; mt < MTN; mt++) {
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int32_t r = m0e + mt * 16 + 4 * p + i;
                            if (r >= nee) continue;
                            *reinterpret_cast<float2 *>(ybp + (int64_t)(r0e + r) * He + col0) =
                                float2{acc[0][mt][0][i] + b0, acc[0][mt][1][i] + b1};
                        }
                    }
                }
            };
            // MTN: live 16-row tiles of this pass (a constant per instantiation); the
            // accumulators and the epilogue are sized by it, so the passes over fewer rows
            // hold fewer registers
            auto pass = [&](auto mtn_c) {
                constexpr int MTN = decltype(mtn_c)::value;
                floatx4 acc[NBW][MTN][2];
#pragma unroll
                for (int b = 0; b < NBW; b++)
#pragma unroll
                    for (int mt = 0; mt < MTN; mt++) acc[b][mt][0] = acc[b][mt][1] = zero4();
                auto body = [&](int ch, int slot) {
                    wait_vmcnt<(NBUF - 2) * (LPA + WPS)>();  // this thread's copies of chunk ch
                    __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0): this wave's reads of chunk ch - 1
                    __builtin_amdgcn_s_barrier();            // everyone's copies of chunk ch have landed
                    __builtin_amdgcn_sched_barrier(0);
                    step(ch, (slot + PF) % (PF + 1));
                    if (!active) return;
                    const unsigned char *buf = smem + (size_t)(ch % NBUF) * C::BUF;
#pragma unroll
                    for (int j = 0; j < CKB; j++) {
                        u32x4 a[MTN][P];
#pragma unroll
                        for (int mt = 0; mt < MTN; mt++)
#pragma unroll
                            for (int pl = 0; pl < P; pl++) {
                                const int rr = mt * 16 + l16, kc = 4 * j + p;
                                a[mt][pl] = *reinterpret_cast<const u32x4 *>(
                                    buf + (size_t)((pl * 64 + rr) * C::ROWG + moe_slot(kc, rr)) * 16);
                            }
                        u32x4 be[NBW], bo[NBW];
#pragma unroll
                        for (int b = 0; b < NBW; b++) {
                            u32x2 sw;
                            if constexpr (SL)
                                sw = *reinterpret_cast<const u32x2 *>(scl + ((size_t)b * KBP + ch * CKB + j) * 32 + 8 * p);
                            else
                                sw = ws[slot][j][b];
                            uint32_t r[8];
                            fp4_rows(wq[slot][j][b], sw, r);
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                bo[b][q] = __builtin_amdgcn_perm(r[2 * q + 1], r[2 * q], 0x05040100u);  // column 2c + 1
                                be[b][q] = __builtin_amdgcn_perm(r[2 * q + 1], r[2 * q], 0x07060302u);  // column 2c
                            }
                        }
#pragma unroll
                        for (int mt = 0; mt < MTN; mt++)
#pragma unroll
                            for (int pl = 0; pl < P; pl++)
#pragma unroll
                                for (int b = 0; b < NBW; b++) {
                                    acc[b][mt][0] = mfma16x16x32_bf16(a[mt][pl], be[b], acc[b][mt][0]);
                                    acc[b][mt][1] = mfma16x16x32_bf16(a[mt][pl], bo[b], acc[b][mt][1]);
                                }
                    }
                };
                // full groups of PF + 1 chunks (slot = position in the group), then the rest
                const int nfull = nch - nch % (PF + 1);
                for (int c0 = 0; c0 < nfull; c0 += PF + 1) {
#pragma unroll
                    for (int u = 0; u < PF + 1; u++) body(c0 + u, u);
                }
#pragma unroll
                for (int u = 0; u < PF; u++)
                    if (nfull + u < nch) body(nfull + u, u);
                __builtin_amdgcn_s_waitcnt(0);  // trailing copies and weight loads (unused)
                if (!active) return;
                epilogue(acc);
            };
            switch (mtn) {
            case 1: pass(std::integral_constant<int, 1>{}); break;
            case 2: pass(std::integral_constant<int, 2>{}); break;
            case 3: pass(std::integral_constant<int, 3>{}); break;
            default: pass(std::integral_constant<int, 4>{}); break;
            }
        }
    }
}

// y[t] = ((0 + w_a * y_a) + w_b * y_b) + ... over the token's experts a < b < ...
// A NaN or infinite output sets *status (when given) to NNQ_ERR_NON_FINITE, the
// check_output_finite of moe_forward (crates/nn-core/src/layers/nan_check.rs:113-140).
template <int k, bool V4>
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeScratch sc, int64_t H, float *y, int32_t *status) {
    const int64_t t = blockIdx.x;
    uint32_t ex[k];
    int32_t ps[k];
    float ws[k];
#pragma unroll
    for (int s = 0; s < k; s++) {
        ex[s] = sc.ti[t * k + s];
        ps[s] = sc.pos[t * k + s];
        ws[s] = sc.tw[t * k + s];
    }
#pragma unroll
    for (int s = 0; s + 1 < k; s++)  // sort by expert (the k experts are distinct): bubble network
#pragma unroll
        for (int q = 0; q + 1 < k - s; q++) {
            const bool sw = ex[q] > ex[q + 1];
            const uint32_t e0 = ex[q], e1 = ex[q + 1];
            const int32_t p0 = ps[q], p1 = ps[q + 1];
            const float w0 = ws[q], w1 = ws[q + 1];
            ex[q] = sw ? e1 : e0;
            ex[q + 1] = sw ? e0 : e1;
            ps[q] = sw ? p1 : p0;
            ps[q + 1] = sw ? p0 : p1;
            ws[q] = sw ? w1 : w0;
            ws[q + 1] = sw ? w0 : w1;
        }
    bool bad = false;
    if (V4) {
        // four consecutive columns per thread (H % 4 == 0, y 16-byte aligned): the same
        // per-element arithmetic on 16-byte loads and stores
        const int64_t H4 = H / 4;
#pragma unroll 3
        for (int64_t c = threadIdx.x; c < H4; c += 256) {
            floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < k; s++) {
                const floatx4 v = *reinterpret_cast<const floatx4 *>(sc.yb + (int64_t)ps[s] * H + 4 * c);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = acc[i] + v[i] * ws[s];
            }
            *reinterpret_cast<floatx4 *>(y + t * H + 4 * c) = acc;
#pragma unroll
            for (int i = 0; i < 4; i++) bad |= !(fabsf(acc[i]) <= 3.402823466e38f);
        }
    } else {
        for (int64_t c = threadIdx.x; c < H; c += 256) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < k; s++) acc = acc + sc.yb[(int64_t)ps[s] * H + c] * ws[s];
            y[t * H + c] = acc;
            bad |= !(fabsf(acc) <= 3.402823466e38f);
        }
    }
    if (status && __any(bad) && (threadIdx.x & 63) == 0) *status = NNQ_ERR_NON_FINITE;
}

// moe_combine_kernel for any k (k > 8): the token's (row, weight) pairs are put in
// ascending expert order in LDS (an entry's place = the count of its smaller experts).
template <bool V4>
__global__ __launch_bounds__(256) void moe_combine_any_kernel(MoeScratch sc, int64_t H, int k, float *y,
                                                              int32_t *status) {
    extern __shared__ __attribute__((aligned(16))) int32_t cs[];  // [k] rows, then [k] weights
    int32_t *ps = cs;
    float *ws = reinterpret_cast<float *>(cs + k);
    const int64_t t = blockIdx.x;
    for (int s = threadIdx.x; s < k; s += 256) {
        const uint32_t e = sc.ti[t * k + s];
        int r = 0;
        for (int q = 0; q < k; q++) r += sc.ti[t * k + q] < e ? 1 : 0;
        ps[r] = sc.pos[t * k + s];
        ws[r] = sc.tw[t * k + s];
    }
    __syncthreads();
    bool bad = false;
    if (V4) {
        const int64_t H4 = H / 4;
        for (int64_t c = threadIdx.x; c < H4; c += 256) {
            floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int s = 0; s < k; s++) {
                const floatx4 v = *reinterpret_cast<const floatx4 *>(sc.yb + (int64_t)ps[s] * H + 4 * c);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = acc[i] + v[i] * ws[s];
            }
            *reinterpret_cast<floatx4 *>(y + t * H + 4 * c) = acc;
#pragma unroll
            for (int i = 0; i < 4; i++) bad |= !(fabsf(acc[i]) <= 3.402823466e38f);
        }
    } else {
        for (int64_t c = threadIdx.x; c < H; c += 256) {
            float acc = 0.0f;
            for (int s = 0; s < k; s++) acc = acc + sc.yb[(int64_t)ps[s] * H + c] * ws[s];
            y[t * H + c] = acc;
            bad |= !(fabsf(acc) <= 3.402823466e38f);
        }
    }
    if (status && __any(bad) && (threadIdx.x & 63) == 0) *status = NNQ_ERR_NON_FINITE;
}

// ---------------------------------------------------------------------------------
// bit-exact decode of one expert (Mxfp4Tensor::dequantize, crates/nn-gptoss/src/quantize.rs:167-188)
// ---------------------------------------------------------------------------------
__constant__ float kFp4Lut[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// FP4_LUT[code] * 2^(E - 127) as f32 bits (the device scale byte E: GPT-OSS's byte 0 is
// stored as 1, see fp4_rows), built with integer arithmetic so that subnormal results
// are exact whatever the f32 denormal mode.  E = 255 scales by +inf (x * inf, 0 * inf =
// NaN), as both reference decoders do.
__device__ __forceinline__ float fp4_decode(uint32_t code, uint32_t sbyte) {
    const uint32_t mag = code & 7u, sign = (code & 8u) << 28;
    if (mag == 0 || sbyte == 255) {  // zeros, and the inf scale (x * inf, 0 * inf = NaN)
        const float s = __uint_as_float(sbyte << 23);
        return kFp4Lut[code] * s;
    }
    // magnitude = m * 2^x with m in {1, 3}: 0.5 = 1*2^-1, 1, 1.5 = 3*2^-1, 2, 3 = 3*2^0, 4, 6 = 3*2^1
    const int m3 = (mag == 3 || mag == 5 || mag == 7);
    const int x = m3 ? (int)(mag >> 1) - 2 : (int)(mag >> 1) - 1;
    const int E = (int)sbyte;
    const int q = x + m3 + E - 127;  // unbiased exponent of the value (m = 3 -> 1.5 * 2^(x + 1))
    uint32_t bits;
    if (q > 127)
        bits = 0x7F800000u;
    else if (q >= -126)
        bits = ((uint32_t)(q + 127) << 23) | (m3 ? 0x400000u : 0u);
    else
        bits = (m3 ? 3u : 1u) << (x + E + 22);  // m * 2^(x + E - 127) as a multiple of 2^-149 (x >= -1)
    return __uint_as_float(bits | sign);
}

// nn-core OCP MXFP4 tensor decode (dequantize_tensor, crates/nn-core/src/layers/quantized/
// mxfp4.rs:226-244, 320-333): 17-byte blocks [shared_exp][16 packed], element 2i in the
// low nibble of byte i, value magnitude * 2^(shared_exp - 127); one thread per byte pair
// of elements, the first n values.
__global__ __launch_bounds__(256) void ocp_dequant_kernel(const uint8_t *blocks, int64_t n, float *out) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;  // element pair 2p, 2p + 1
    const int64_t i = 2 * p;
    if (i >= n) return;
    const uint8_t *blk = blocks + (i / 32) * 17;
    const uint32_t e = blk[0], byte = blk[1 + (i % 32) / 2];
    out[i] = fp4_decode(byte & 15u, e);
    if (i + 1 < n) out[i + 1] = fp4_decode(byte >> 4, e);
}

// one workgroup per (column block, row block) fragment; thread = (row, byte column)
__global__ __launch_bounds__(512) void moe_dequant_kernel(const uint8_t *codes, const uint8_t *scales, int64_t K,
                                                          int64_t N, float *out) {
    const int64_t KB = K / 32;
    const int64_t nb = blockIdx.x / KB, kb = blockIdx.x % KB;
    const int r = threadIdx.x >> 4, c = threadIdx.x & 15;  // row 0..31, byte column 0..15
    const int64_t frag = nb * KB + kb;
    const uint8_t b = codes[frag * 512 + (16 * (r >> 3) + c) * 8 + (r & 7)];
    const uint8_t e = scales[frag * 32 + r];
    float *o = out + (kb * 32 + r) * N + nb * 32 + 2 * c;
    o[0] = fp4_decode(b >> 4, e);
    o[1] = fp4_decode(b & 15, e);
}

// ---------------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------------
size_t moe_scratch_bytes(int64_t T, int64_t E, int64_t H, int64_t I, int k, int x_bf16) {
    const size_t A = (size_t)T * k;
    return al256(A * 4) * 4 + al256((size_t)(E + 1) * 4) + (x_bf16 ? 0 : al256((size_t)2 * T * H * 2)) +
           al256((size_t)2 * A * I * 2) + al256(A * H * 4) + 256;
}

template <int P, bool GU, int CKB, bool SL>
static int launch_stream_t(const MoeDev &d, const MoeScratch &sc, const MoeRun &run, hipStream_t st, size_t lds) {
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&moe_stream_kernel<P, GU, CKB, SL>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMoeLdsMax);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    hipLaunchKernelGGL((moe_stream_kernel<P, GU, CKB, SL>), dim3((unsigned)(d.E * kMoeGroups)), dim3(kMoeWaves * 64),
                       lds, st, d, sc, run);
    return (int)hipGetLastError();
}

// Chunks of 3 k-blocks when K / 32 allows, scales staged in LDS when they fit beside
// the ring (hidden / intermediate up to 5120 for gate_up with bf16 input).  gate_up over
// f32 input (two activation planes) takes chunks of one k-block: with three its weight
// ring and operands exceed the registers of 12 waves (117 spilled; config 5 with f32 x
// 184 against 168 us).
template <int P, bool GU>
static int launch_stream(const MoeDev &d, const MoeScratch &sc, const MoeRun &run, hipStream_t st) {
    const int64_t KB = (GU ? d.H : d.I) / 32;
    if constexpr (!(P == 2 && GU))
        if (KB % 3 == 0 && moe_lds<P, GU, 3, true>(KB) <= kMoeLdsMax)
            return launch_stream_t<P, GU, 3, true>(d, sc, run, st, moe_lds<P, GU, 3, true>(KB));
    if (moe_lds<P, GU, 1, true>(KB) <= kMoeLdsMax)
        return launch_stream_t<P, GU, 1, true>(d, sc, run, st, moe_lds<P, GU, 1, true>(KB));
    return launch_stream_t<P, GU, 1, false>(d, sc, run, st, moe_lds<P, GU, 1, false>(KB));
}

int launch_moe(const MoeDev &d, const void *x, int x_bf16, int64_t T, const float *logits, int nsplit,
               const float *bias, int k, float limit, float *y, uint32_t *topk_idx, float *topk_w, int32_t *status,
               void *scratch, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    int e = 0;
    const MoeScratch sc = carve(scratch, T, d.E, d.H, d.I, k, x_bf16);
    MoeRun run;
    run.A = T * k;
    run.limit = limit;
    run.ti = sc.ti;
    run.T = T;
    run.k = k;
    run.perm = T <= kMoeInPermT ? 1 : 0;
    if (d.E <= 256)
        hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, logits, nsplit, bias, T,
                           (int)d.E, k, sc.ti, sc.tw, topk_idx, topk_w);
    else
        hipLaunchKernelGGL(moe_route_any_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256),
                           (size_t)4 * (d.E + (k > 8 ? k : 0)) * 4, st, logits, nsplit, bias, T, (int)d.E, k, sc.ti,
                           sc.tw, topk_idx, topk_w);
    if (!run.perm) switch (k) {
#define NNQ_PERM(K)                                                                                              \
    case K:                                                                                                      \
        hipLaunchKernelGGL(moe_permute_kernel<K>, dim3(1), dim3(1024), (size_t)d.E * 4, st, sc.ti, T, (int)d.E, sc.off, \
                           sc.stok, sc.pos);                                                                     \
        break;
        NNQ_PERM(1) NNQ_PERM(2) NNQ_PERM(3) NNQ_PERM(4) NNQ_PERM(5) NNQ_PERM(6) NNQ_PERM(7) NNQ_PERM(8)
#undef NNQ_PERM
    default:
        hipLaunchKernelGGL(moe_permute_any_kernel, dim3(1), dim3(1024), (size_t)d.E * 4, st, sc.ti, T, (int)d.E, k,
                           sc.off, sc.stok, sc.pos);
        break;
    }
    if (x_bf16) {
        run.xa[0] = reinterpret_cast<const uint16_t *>(x);
        run.xa[1] = nullptr;
    } else {
        const int64_t n = T * d.H;
        hipLaunchKernelGGL(moe_split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           reinterpret_cast<const float *>(x), n, sc.xb);
        run.xa[0] = sc.xb;
        run.xa[1] = sc.xb + n;
    }
    if (x_bf16)
        e = launch_stream<1, true>(d, sc, run, st);
    else
        e = launch_stream<2, true>(d, sc, run, st);
    if (e) return e;
    e = launch_stream<2, false>(d, sc, run, st);
    if (e) return e;
    const bool v4 = d.H % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    switch (k) {
#define NNQ_COMB(K)                                                                                         \
    case K:                                                                                                 \
        if (v4)                                                                                             \
            hipLaunchKernelGGL((moe_combine_kernel<K, true>), dim3((unsigned)T), dim3(256), 0, st, sc, d.H, y, status); \
        else                                                                                                \
            hipLaunchKernelGGL((moe_combine_kernel<K, false>), dim3((unsigned)T), dim3(256), 0, st, sc, d.H, y, status); \
        break;
        NNQ_COMB(1) NNQ_COMB(2) NNQ_COMB(3) NNQ_COMB(4) NNQ_COMB(5) NNQ_COMB(6) NNQ_COMB(7) NNQ_COMB(8)
#undef NNQ_COMB
    default:
        if (v4)
            hipLaunchKernelGGL((moe_combine_any_kernel<true>), dim3((unsigned)T), dim3(256), (size_t)k * 8, st, sc, d.H,
                               k, y, status);
        else
            hipLaunchKernelGGL((moe_combine_any_kernel<false>), dim3((unsigned)T), dim3(256), (size_t)k * 8, st, sc, d.H,
                               k, y, status);
        break;
    }
    return (int)hipGetLastError();
}

size_t router_partial_bytes(int64_t T, int64_t H, int E) {
    const int ks = router_parts(T, H, E);
    return ks > 1 ? (size_t)ks * T * E * 4 : 0;
}

int launch_router_logits(const void *x, int x_bf16, int64_t T, int64_t H, const float *W, const float *bias, int E,
                         float *partial, int *nsplit, int32_t *status, void *stream) {
    const int ks = router_parts(T, H, E);
    const dim3 grid((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16), (unsigned)ks);
    if (x_bf16)
        hipLaunchKernelGGL(router_logits_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, x, T, H, W, bias, E,
                           partial, status);
    else
        hipLaunchKernelGGL(router_logits_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, x, T, H, W, bias, E,
                           partial, status);
    *nsplit = ks;
    return (int)hipGetLastError();
}

// logits[t, e] = sum of the K-part slabs in order + bias (the standalone router call)
__global__ __launch_bounds__(256) void router_finalize_kernel(const float *partial, int ks, int64_t T, int E,
                                                              const float *bias, float *logits) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= T * E) return;
    float v = partial[i];
    for (int s = 1; s < ks; s++) v += partial[(int64_t)s * T * E + i];
    logits[i] = v + (bias ? bias[i % E] : 0.0f);
}

int launch_router_finalize(const float *partial, int ks, int64_t T, int E, const float *bias, float *logits,
                           void *stream) {
    hipLaunchKernelGGL(router_finalize_kernel, dim3((unsigned)((T * E + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, partial, ks, T, E, bias, logits);
    return (int)hipGetLastError();
}

int launch_moe_dequant(const MoeDev &d, int64_t e, float *gate_up, float *down, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    if (gate_up) {
        const int64_t K = d.H, N = 2 * d.I;
        const size_t per = (size_t)K * N;
        hipLaunchKernelGGL(moe_dequant_kernel, dim3((unsigned)((N / 32) * (K / 32))), dim3(512), 0, st,
                           d.gu_q + e * per / 2, d.gu_s + e * per / 32, K, N, gate_up);
    }
    if (down) {
        const int64_t K = d.I, N = d.H;
        const size_t per = (size_t)K * N;
        hipLaunchKernelGGL(moe_dequant_kernel, dim3((unsigned)((N / 32) * (K / 32))), dim3(512), 0, st,
                           d.dn_q + e * per / 2, d.dn_s + e * per / 32, K, N, down);
    }
    return (int)hipGetLastError();
}

int launch_ocp_dequant(const uint8_t *blocks, int64_t n, float *out, void *stream) {
    if (n <= 0) return 0;
    const int64_t pairs = (n + 1) / 2;
    hipLaunchKernelGGL(ocp_dequant_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       blocks, n, out);
    return (int)hipGetLastError();
}

}  // namespace nnq
