// Token sampling on gfx950: sample_token (crates/nn-gptoss/src/sampling.rs:136-185) over a
// logits vector that stays on the device, e.g. straight out of the LM-head GEMV.
//
// Every logit becomes a 64-bit key: its orderable value (after the penalties and the
// temperature) above its inverted index, so keys are unique, larger keys are larger
// values, and equal values order the lower index first.  NaN keys sit below every
// value and never become candidates.
//
//   sample_local_kernel  one workgroup per 2048 logits: repetition / frequency penalties
//                        (per occurrence of past_tokens, :277-306), temperature
//                        (:193-199), keys; an exact radix select (8 passes of 8 bits)
//                        finds the block's kk-th largest key, and the kk keys at or
//                        above it go to the candidate buffer (unordered)
//   sample_final_kernel  one workgroup: the same radix select over the candidates gives
//                        exactly the top k (apply_top_k, :245-275), sorted by a small
//                        bitonic network; wave 0 then runs the reference's tail with
//                        the exponentials in parallel and every sum in candidate order:
//                        finite candidates in index order, or top-p over the descending
//                        order (:211-238), softmax and the seed's selector walk
//                        (:340-391), and argmax_slice (:394-400) when no candidate is left.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

constexpr int kSampleBlock = 2048;  // logits per local workgroup
constexpr int kSampleMaxCand = 16384;

// total order of f32 as unsigned (NaN handled by the caller)
__device__ __forceinline__ uint32_t ord_f32(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord_f32(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ uint64_t cand_key(float v, uint32_t idx) {
    if (v != v) return 0xFFFFFFFFull - idx;  // below every value (ord(-inf) > 0), above padding 0
    return ((uint64_t)ord_f32(v) << 32) | (0xFFFFFFFFull - idx);
}
__device__ __forceinline__ uint32_t key_idx(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull); }
__device__ __forceinline__ float key_val(uint64_t k) { return unord_f32((uint32_t)(k >> 32)); }
__device__ __forceinline__ bool key_finite(uint64_t k) { return (k >> 32) != 0 && fabsf(key_val(k)) <= 3.402823466e38f; }
// ord(+inf): the largest orderable value
constexpr uint32_t kOrdPosInf = 0xFF800000u;
// a candidate of the tail: finite, or also +inf when top_k is None (sampling.rs:160-164
// keeps every v > -inf there; apply_top_k keeps finite values only)
__device__ __forceinline__ bool key_cand(uint64_t k, bool keep_inf) {
    return key_finite(k) || (keep_inf && (uint32_t)(k >> 32) == kOrdPosInf);
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// inclusive prefix sum over the 64 lanes by DPP: shifts within each 16-lane row, then
// the row totals broadcast into the following rows (row_bcast:15, row_bcast:31)
__device__ __forceinline__ int wave_scan_incl(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
    return v;
}

// The value of lane (lane ^ S) for S a power of two below 64, without LDS: DPP within each
// 16-lane row (quad permutes and mirrors), lane swaps between rows.  Every lane of the
// wave must be active.
template <int S>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    static_assert(S >= 1 && S <= 32 && (S & (S - 1)) == 0, "xor distance");
    const int x = (int)v;
    if constexpr (S == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (S == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (S == 4) {
        // quad_perm [3,2,1,0] (l ^ 3), then row_half_mirror (l ^ 7)
        const int t = __builtin_amdgcn_update_dpp(0, x, 0x1B, 0xF, 0xF, false);
        return (uint32_t)__builtin_amdgcn_update_dpp(0, t, 0x141, 0xF, 0xF, false);
    } else if constexpr (S == 8) {
        // row_half_mirror (l ^ 7), then row_mirror (l ^ 15)
        const int t = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);
        return (uint32_t)__builtin_amdgcn_update_dpp(0, t, 0x140, 0xF, 0xF, false);
    } else if constexpr (S == 16) {
        // the swap leaves this lane's value and its partner's in the pair
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return p[0] ^ p[1] ^ v;
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return p[0] ^ p[1] ^ v;
    }
}
template <int S>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
    return ((uint64_t)lane_xor<S>((uint32_t)(v >> 32)) << 32) | lane_xor<S>((uint32_t)v);
}

// One compare-exchange step of a bitonic network over one key per lane (partner lane ^ S,
// descending where lane & size is 0).
template <int S>
__device__ __forceinline__ uint64_t bitonic_lanes(uint64_t v, int lane, int size) {
    const uint64_t o = lane_xor64<S>(v);
    const bool desc = (lane & size) == 0, lower = (lane & S) == 0;
    return (lower == desc) ? (o > v ? o : v) : (o < v ? o : v);
}

// Descending bitonic sort of one key per lane over the first n lanes (n a power of two up
// to 64; lanes from n on hold keys no larger than any of them, e.g. 0), in registers.
__device__ uint64_t sort_lanes_desc(uint64_t v, int n) {
    const int lane = threadIdx.x & 63;
    if (n >= 2) v = bitonic_lanes<1>(v, lane, 2);
    if (n >= 4) {
        v = bitonic_lanes<2>(v, lane, 4);
        v = bitonic_lanes<1>(v, lane, 4);
    }
    if (n >= 8) {
        v = bitonic_lanes<4>(v, lane, 8);
        v = bitonic_lanes<2>(v, lane, 8);
        v = bitonic_lanes<1>(v, lane, 8);
    }
    if (n >= 16) {
        v = bitonic_lanes<8>(v, lane, 16);
        v = bitonic_lanes<4>(v, lane, 16);
        v = bitonic_lanes<2>(v, lane, 16);
        v = bitonic_lanes<1>(v, lane, 16);
    }
    if (n >= 32) {
        v = bitonic_lanes<16>(v, lane, 32);
        v = bitonic_lanes<8>(v, lane, 32);
        v = bitonic_lanes<4>(v, lane, 32);
        v = bitonic_lanes<2>(v, lane, 32);
        v = bitonic_lanes<1>(v, lane, 32);
    }
    if (n >= 64) {
        v = bitonic_lanes<32>(v, lane, 64);
        v = bitonic_lanes<16>(v, lane, 64);
        v = bitonic_lanes<8>(v, lane, 64);
        v = bitonic_lanes<4>(v, lane, 64);
        v = bitonic_lanes<2>(v, lane, 64);
        v = bitonic_lanes<1>(v, lane, 64);
    }
    return v;
}

// A threshold t with exactly k of the nonzero keys held E per thread at or above it (k <=
// their number, all distinct; zero keys are padding and take no part): passes over 8-bit
// digits, most significant first, until the digit bin that holds the kth largest is
// needed whole (then t is the prefix so far with zeros below) or all 64 bits are fixed
// (then t is the kth largest key).  Each wave counts into its own histogram, so equal
// digits only contend within a wave, and every wave then reads all NW histograms and
// finds the bin itself, so a pass needs one barrier: the histograms are double-buffered
// and each wave clears its own histogram of the other buffer (read by every wave before
// this pass's barrier) for the next pass.  hist holds 2 * NW * 256 ints.  Every thread of
// the workgroup calls it; it returns without a closing barrier (hist may still be read).
template <int E, int NW>
__device__ uint64_t radix_kth(const uint64_t (&e)[E], int k, int *hist) {
    uint64_t prefix = 0, mask = 0;
    int rem = k;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 2 * NW * 256; i += NW * 64) hist[i] = 0;
    __syncthreads();
    int buf = 0;
    for (int shift = 56; shift >= 0; shift -= 8, buf ^= 1) {
        int *H = hist + buf * (NW * 256);
        int *my = H + wv * 256;
#pragma unroll
        for (int r = 0; r < E; r++)
            if (e[r] != 0 && (e[r] & mask) == prefix) atomicAdd(&my[(e[r] >> shift) & 255], 1);
        __syncthreads();
        // lane l: the descending digits 255 - 4l - j (j = 0..3), i.e. the 16 bytes at digit
        // 252 - 4l of every wave's histogram, summed over the waves
        int c[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const int4 h = *reinterpret_cast<const int4 *>(H + w * 256 + 252 - 4 * lane);
            c[0] += h.w;
            c[1] += h.z;
            c[2] += h.y;
            c[3] += h.x;
        }
        int *other = hist + (buf ^ 1) * (NW * 256) + wv * 256;
        reinterpret_cast<int4 *>(other)[lane] = int4{0, 0, 0, 0};
        const int sum = c[0] + c[1] + c[2] + c[3];
        int before = wave_scan_incl(sum) - sum;  // exclusive scan over the lanes
        int hit = -1, hbefore = 0, hcount = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (before < rem && before + c[j] >= rem) {
                hit = j;
                hbefore = before;
                hcount = c[j];
            }
            before += c[j];
        }
        // exactly one lane holds the bin (k does not exceed the keys that take part)
        const uint64_t found = __ballot(hit >= 0);
        if (found == 0) break;  // not reached: callers keep k within the keys that take part
        const int src = (int)__builtin_ctzll(found);
        const int digit = 255 - 4 * src - __builtin_amdgcn_readlane(hit, src);
        const int above = __builtin_amdgcn_readlane(hbefore, src), inbin = __builtin_amdgcn_readlane(hcount, src);
        rem -= above;
        prefix |= (uint64_t)digit << shift;
        mask |= 0xFFull << shift;
        if (inbin == rem) break;  // the whole bin is taken (uniform)
    }
    return prefix;
}

// Appends the keys e[r] >= kth (nonzero) to out at slots taken from the LDS counter *n:
// one counter atomic per wave, the slots within the wave by lane rank.  Every lane of the
// calling wave must be active.
template <int E>
__device__ __forceinline__ void append_selected(const uint64_t (&e)[E], uint64_t kth, int *n, uint64_t *out) {
    uint64_t bal[E];
    int total = 0;
#pragma unroll
    for (int r = 0; r < E; r++) {
        bal[r] = __ballot(e[r] >= kth && e[r] != 0);
        total += __builtin_popcountll(bal[r]);
    }
    if (total == 0) return;  // uniform
    int base = 0;
    if ((threadIdx.x & 63) == 0) base = atomicAdd(n, total);
    base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
    for (int r = 0; r < E; r++) {
        const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal[r] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal[r], 0));
        if ((bal[r] >> (threadIdx.x & 63)) & 1) out[base + below] = e[r];
        base += __builtin_popcountll(bal[r]);
    }
}

// Bitonic sort, descending, of n keys in LDS (n a power of two <= 16384); all threads
// call it.  Up to 64 keys wave 0 sorts them in registers (one per lane, partners by lane
// exchange), up to 128 in LDS with wave-level synchronisation; one barrier at the end
// publishes the result to the other waves.
__device__ void sort_desc_lds(uint64_t *a, int n) {
    if (n <= 64) {
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            const uint64_t v = sort_lanes_desc(lane < n ? a[lane] : 0ull, n);
            if (lane < n) a[lane] = v;
        }
        __syncthreads();
        return;
    }
    const bool small = n <= 128;  // uniform
    if (!small || threadIdx.x < 64) {
        const int nth = small ? 64 : (int)blockDim.x;
        for (int size = 2; size <= n; size <<= 1)
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int i = threadIdx.x; i < n / 2; i += nth) {
                    const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                    const bool desc = (lo & size) == 0;
                    const uint64_t x = a[lo], y = a[hi];
                    if ((x < y) == desc) {
                        a[lo] = y;
                        a[hi] = x;
                    }
                }
                if (small)
                    wave_sync();
                else
                    __syncthreads();
            }
    }
    if (small) __syncthreads();
}

struct SampleParams {
    float temperature, top_p, rep, freq;
    int rep_on, freq_on, use_top_p;
    int keep_inf;  // top_k None: +inf logits are candidates too
    int64_t k;     // candidates kept by top-k (already min(top_k, n); 0: none)
    uint64_t seed;
};

// The keys of the kSampleBlock logits from `base` (E per thread of 256, element r * 256 +
// tid): repetition / frequency penalties per occurrence of past_tokens (counted in LDS
// `cnt`), temperature, orderable key; 0 past n.  Every thread of the workgroup calls it.
template <int E>
__device__ void block_keys(const float *logits, int64_t n, const uint32_t *past, int64_t n_past,
                           const SampleParams &sp, int64_t base, int *cnt, uint64_t (&e)[E]) {
    const int tid = threadIdx.x;
    const bool pen = (sp.rep_on || sp.freq_on) && n_past > 0;
    if (pen) {
        for (int j = tid; j < kSampleBlock; j += 256) cnt[j] = 0;
        __syncthreads();
        for (int64_t i = tid; i < n_past; i += 256) {
            const int64_t t = past[i];
            if (t >= base && t < base + kSampleBlock && t < n) atomicAdd(&cnt[t - base], 1);
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < E; r++) {
        const int j = r * 256 + tid;  // coalesced
        const int64_t i = base + j;
        uint64_t key = 0;  // padding past n: below everything
        if (i < n) {
            float l = logits[i];
            if (pen) {
                const int c = cnt[j];
                if (sp.rep_on)
                    for (int q = 0; q < c; q++) l = l > 0.0f ? l / sp.rep : (l < 0.0f ? l * sp.rep : l);
                if (sp.freq_on)
                    for (int q = 0; q < c; q++) l -= sp.freq;
            }
            if (fabsf(l) <= 3.402823466e38f) l = l / sp.temperature;
            key = cand_key(l, (uint32_t)i);
        }
        e[r] = key;
    }
}

__global__ __launch_bounds__(256) void sample_local_kernel(const float *logits, int64_t n, const uint32_t *past,
                                                           int64_t n_past, SampleParams sp, int kk, uint64_t *cand) {
    __shared__ int cnt[kSampleBlock];
    __shared__ __attribute__((aligned(16))) int hist[2 * 4 * 256];
    __shared__ int nout;
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * kSampleBlock;
    if (tid == 0) nout = 0;
    constexpr int E = kSampleBlock / 256;
    uint64_t e[E];
    block_keys<E>(logits, n, past, n_past, sp, base, cnt, e);
    // the block's real logits may be fewer than kk: keep them all, pad the slots with 0
    const int real = (int)std::min<int64_t>(kSampleBlock, n - base);
    const int kb = std::min(kk, real);
    const uint64_t kth = radix_kth<E, 4>(e, kb, hist);  // (its first barrier orders nout)
    uint64_t *out = cand + (int64_t)blockIdx.x * kk;
    append_selected<E>(e, kth, &nout, out);
    for (int j = kb + tid; j < kk; j += 256) out[j] = 0;
}

// The f32 sum ((0 + p[0]) + p[1]) + ... + p[n - 1] in element order, the same value in
// every lane: 16-byte broadcast reads (p is 16-byte aligned and readable up to the next
// multiple of 4), the additions one after another.
__device__ __forceinline__ float ordered_sum(const float *p, int n) {
    float sum = 0.0f;
    for (int i = 0; i < n; i += 4) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(p + i);
        sum += v[0];
        if (i + 1 < n) sum += v[1];
        if (i + 2 < n) sum += v[2];
        if (i + 3 < n) sum += v[3];
    }
    return sum;
}

// softmax_candidates (sampling.rs:371-391) of val[0..n) into p[0..n), by wave 0:
// exponentials and quotients in parallel, the maximum (order-free) by reduction, the sum
// in candidate order.
__device__ void softmax_wave(const float *val, int n, float *ex, float *p) {
    const int lane = threadIdx.x;
    float mx = -INFINITY;
    for (int i = lane; i < n; i += 64) mx = fmaxf(mx, val[i]);
    mx = wave_max(mx);
    if (!(fabsf(mx) <= 3.402823466e38f)) {
        for (int i = lane; i < n; i += 64) p[i] = 1.0f / (float)n;
        wave_sync();
        return;
    }
    for (int i = lane; i < n; i += 64) ex[i] = expf(val[i] - mx);
    wave_sync();
    const float sum = ordered_sum(ex, n);
    if (!(fabsf(sum) <= 3.402823466e38f) || sum == 0.0f) {
        for (int i = lane; i < n; i += 64) p[i] = 1.0f / (float)n;
    } else {
        for (int i = lane; i < n; i += 64) p[i] = ex[i] / sum;
    }
    wave_sync();
}

// the first i with (cumulative sum of p[0..i] in order) meeting `stop` (n when none);
// every lane walks the same broadcast values
template <class F>
__device__ int walk_wave(const float *p, int n, F stop) {
    float cum = 0.0f;
    for (int i = 0; i < n; i += 4) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(p + i);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (i + j >= n) return n;
            cum += v[j];
            if (stop(cum)) return i + j;
        }
    }
    return n;
}

// ((0 + x_0) + x_1) + ... + x_{n-1} over lanes 0 .. n - 1 (n <= 64) in lane order, the
// same value in every lane: one addition after another, the addends read by readlane.
// x must be 0 in the lanes at or past n and no addend negative (adding +0 to a sum that
// is not negative leaves it unchanged), so whole groups of 16 lanes are added.
__device__ __forceinline__ float ordered_lane_sum(float x, int n) {
    float s = 0.0f;
    for (int j0 = 0; j0 < n; j0 += 16)
#pragma unroll
        for (int j = 0; j < 16; j++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j0 + j));
    return s;
}

// the first lane i < n whose cumulative sum p_0 + ... + p_i (in lane order, p >= 0 and 0
// at or past n) meets `stop`, n when none
template <class F>
__device__ __forceinline__ int walk_lanes(float p, int n, F stop) {
    const int lane = threadIdx.x & 63;
    float cum = 0.0f, mine = 0.0f;
    for (int j0 = 0; j0 < n; j0 += 16)
#pragma unroll
        for (int j = 0; j < 16; j++) {
            cum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j0 + j));
            mine = lane == j0 + j ? cum : mine;
        }
    const uint64_t hit = __ballot(lane < n && stop(mine));
    return hit ? (int)__builtin_ctzll(hit) : n;
}

// softmax_candidates (sampling.rs:371-391) of the lane values v of lanes 0 .. n - 1
// (n <= 64): this lane's probability, 0 at or past n.  The maximum is order-free, the
// sum runs in candidate order.
__device__ __forceinline__ float softmax_lanes(float v, int n) {
    const int lane = threadIdx.x & 63;
    const bool in = lane < n;
    const float mx = wave_max(in ? v : -INFINITY);
    if (!(fabsf(mx) <= 3.402823466e38f)) return in ? 1.0f / (float)n : 0.0f;
    const float ex = in ? expf(v - mx) : 0.0f;
    const float sum = ordered_lane_sum(ex, n);
    if (!(fabsf(sum) <= 3.402823466e38f) || sum == 0.0f) return in ? 1.0f / (float)n : 0.0f;
    return in ? ex / sum : 0.0f;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    return ((uint64_t)(uint32_t)__shfl((int)(v >> 32), src, 64) << 32) | (uint32_t)__shfl((int)v, src, 64);
}

// argmax_slice (sampling.rs:394-400) of the original logits, by one thread: the running
// maximum moves on unless it compares greater (ties and NaN move on)
__device__ void argmax_slice_serial(const float *logits, int64_t n, uint32_t *token) {
    int64_t best = 0;
    float bv = logits[0];
    for (int64_t j = 1; j < n; j++) {
        const float v = logits[j];
        if (!(bv > v)) {
            best = j;
            bv = v;
        }
    }
    *token = (uint32_t)best;
}

// The reference's tail for top-k up to 64, by wave 0 with one candidate per lane: sel[0..k)
// holds the top k keys (unordered).  They are sorted in registers; the candidates then
// sit in lanes 0 .. nc - 1 in the reference's order (descending for top-p, else ascending
// index), and the top-p cut, softmax and selector walk run on lane values.
__device__ void tail_lanes(const float *logits, int64_t n, const uint64_t *sel, int k, const SampleParams &sp,
                           uint32_t *token) {
    const int lane = threadIdx.x & 63;
    const bool keep_inf = sp.keep_inf != 0;
    int Q = 1;
    while (Q < k) Q <<= 1;
    const uint64_t v = sort_lanes_desc(lane < k ? sel[lane] : 0ull, Q);  // ties: lower index first
    uint64_t w;
    int nc;
    if (!sp.use_top_p && k > 1) {
        // without top-p the reference walks the candidates in index order: sort again by
        // (candidate first, ascending index), carrying each one's lane
        uint64_t r = 0;
        if (lane < k && key_cand(v, keep_inf))
            r = 0x8000000000000000ull | ((uint64_t)(0xFFFFFFFFu - key_idx(v)) << 14) | (uint64_t)lane;
        r = sort_lanes_desc(r, Q);
        nc = __builtin_popcountll(__ballot(r >> 63));
        w = shfl_u64(v, (int)(r & 63));
    } else {
        // descending order: +inf keys first, then the finite ones, then -inf and NaN; the
        // candidates move to the front in order (the +inf keys are candidates, and stay in
        // front, only when top_k is None)
        nc = __builtin_popcountll(__ballot(lane < k && key_cand(v, keep_inf)));
        const int a = __builtin_popcountll(__ballot(lane < k && !keep_inf && (uint32_t)(v >> 32) == kOrdPosInf));
        w = shfl_u64(v, std::min(lane + a, 63));
    }
    const float val = key_val(w);  // lanes < nc: the candidates' values and indices
    const int id = (int)key_idx(w);
    float p = 0.0f;  // the final softmax over lanes < nc, once known
    bool have_p = false;
    if (sp.use_top_p && nc > 0) {
        // apply_top_p_candidates: softmax_candidates, then the smallest prefix (descending
        // order) whose cumulative probability reaches top_p.  The softmax of that prefix
        // needs no second pass: its maximum is the same (lane 0 holds the largest value),
        // so are its exponentials, and its sum is the ordered sum's partial sum at the
        // prefix's last lane, kept per lane here.
        const bool in = lane < nc;
        const float mx = wave_max(in ? val : -INFINITY);
        const bool mx_ok = fabsf(mx) <= 3.402823466e38f;
        const float ex = (in && mx_ok) ? expf(val - mx) : 0.0f;
        float sum = 0.0f, upto = 0.0f;
        for (int j0 = 0; j0 < nc; j0 += 16)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), j0 + j));
                upto = lane == j0 + j ? sum : upto;
            }
        const bool uni = !mx_ok || !(fabsf(sum) <= 3.402823466e38f) || sum == 0.0f;
        const float p1 = in ? (uni ? 1.0f / (float)nc : ex / sum) : 0.0f;
        const float tp = sp.top_p;
        const int i = walk_lanes(p1, nc, [tp](float cum) { return cum >= tp; });
        nc = i < nc ? i + 1 : nc;
        const float sum2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(upto), nc - 1));
        const bool uni2 = !mx_ok || !(fabsf(sum2) <= 3.402823466e38f) || sum2 == 0.0f;
        p = lane < nc ? (uni2 ? 1.0f / (float)nc : ex / sum2) : 0.0f;
        have_p = true;
    }
    if (nc == 0) {
        if (lane == 0) argmax_slice_serial(logits, n, token);
        return;
    }
    if (nc == 1) {
        const int pick = __builtin_amdgcn_readlane(id, 0);
        if (lane == 0) *token = (uint32_t)pick;
        return;
    }
    if (!have_p) p = softmax_lanes(val, nc);
    const float selector = (float)(sp.seed % 10000ull) / 10000.0f;
    const int i = walk_lanes(p, nc, [selector](float cum) { return selector < cum; });
    const int pick = __builtin_amdgcn_readlane(id, i < nc ? i : nc - 1);
    if (lane == 0) *token = (uint32_t)pick;
}

template <int NTH>
__global__ __launch_bounds__(NTH) void sample_final_kernel(const float *logits, int64_t n, const uint64_t *cand,
                                                            int ncand, SampleParams sp, float *work,
                                                            uint32_t *token) {
    __shared__ __attribute__((aligned(16))) uint64_t sel[kSampleMaxCand];
    __shared__ int nsel;
    // the select's histograms borrow the top of sel (free until the selected keys go in)
    int *hist = reinterpret_cast<int *>(sel + kSampleMaxCand) - 2 * (NTH / 64) * 256;
    constexpr int E = 16;  // keys per thread: NTH * 16 >= the candidates (host-checked)
    const int tid = threadIdx.x, k = (int)sp.k;
    // the tail's arrays: in the upper half of `sel` when k <= 2048, else global scratch
    const bool in_lds = k <= 2048;
    const int cap = in_lds ? 2048 : kSampleMaxCand;
    float *val = in_lds ? reinterpret_cast<float *>(sel + kSampleMaxCand / 2) : work;
    float *ex = val + cap, *prob = ex + cap;
    uint32_t *idx = reinterpret_cast<uint32_t *>(prob + cap);
    int nc = 0;
    if (k > 0) {
        uint64_t e[E];
#pragma unroll
        for (int r = 0; r < E; r++) {
            const int j = r * NTH + tid;
            e[r] = j < ncand ? cand[j] : 0ull;
        }
        if (tid == 0) nsel = 0;
        const uint64_t kth = radix_kth<E, NTH / 64>(e, k, hist);  // (its first barrier orders nsel)
        __syncthreads();  // every wave is done with hist before sel is written
        int Q = 1;
        while (Q < k) Q <<= 1;
        for (int j = k + tid; j < Q; j += NTH) sel[j] = 0;
        append_selected<E>(e, kth, &nsel, sel);
        __syncthreads();
        if (k <= 64) {
            if (tid < 64) tail_lanes(logits, n, sel, k, sp, token);
            return;
        }
        sort_desc_lds(sel, Q);  // sel[0..k): the top k, descending (ties: lower index first)
        if (!sp.use_top_p && k > 1) {
            // without top-p the reference walks the candidates in index order: re-sort by
            // (candidates first, ascending index), carrying each one's position (< 2^14)
            for (int j = tid; j < k; j += NTH) val[j] = key_val(sel[j]);
            __syncthreads();
            for (int j = tid; j < Q; j += NTH) {
                uint64_t r = 0;
                if (j < k && key_cand(sel[j], sp.keep_inf != 0))
                    r = 0x8000000000000000ull | ((uint64_t)(0xFFFFFFFFu - key_idx(sel[j])) << 14) | (uint64_t)j;
                sel[j] = r;
            }
            __syncthreads();
            sort_desc_lds(sel, Q);
            if (tid < 64) {
                int f = 0;
                for (int j = tid; j < k; j += 64) {
                    const uint64_t r = sel[j];
                    if (r >> 63) {
                        prob[j] = val[r & 0x3FFFull];
                        idx[j] = 0xFFFFFFFFu - (uint32_t)((r >> 14) & 0xFFFFFFFFull);
                        f++;
                    }
                }
                wave_sync();
                for (int j = tid; j < k; j += 64) val[j] = prob[j];
                for (int o = 32; o > 0; o >>= 1) f += __shfl_xor(f, o, 64);
                nc = f;  // the candidates come first
            }
        } else if (tid < 64) {
            // descending order: +inf keys first, then the finite ones, then -inf and NaN;
            // the candidates move to the front in order (the +inf keys are candidates, and
            // stay in front, only when top_k is None)
            int f = 0, a = 0;
            for (int j = tid; j < k; j += 64) {
                const uint64_t s = sel[j];
                f += key_cand(s, sp.keep_inf != 0) ? 1 : 0;
                a += (!sp.keep_inf && (uint32_t)(s >> 32) == kOrdPosInf) ? 1 : 0;
            }
            for (int o = 32; o > 0; o >>= 1) {
                f += __shfl_xor(f, o, 64);
                a += __shfl_xor(a, o, 64);
            }
            for (int j = tid; j < k; j += 64) {
                const uint64_t s = sel[j];
                if (key_cand(s, sp.keep_inf != 0)) {
                    val[j - a] = key_val(s);
                    idx[j - a] = key_idx(s);
                }
            }
            nc = f;
        }
    }
    if (tid >= 64) return;
    wave_sync();
    if (sp.use_top_p && nc > 0) {
        // apply_top_p_candidates: the smallest prefix (descending order) whose cumulative
        // probability reaches top_p
        softmax_wave(val, nc, ex, prob);
        const float tp = sp.top_p;
        const int i = walk_wave(prob, nc, [tp](float cum) { return cum >= tp; });
        nc = i < nc ? i + 1 : nc;
    }
    if (nc == 0) {
        if (tid == 0) argmax_slice_serial(logits, n, token);
        return;
    }
    if (nc == 1) {
        if (tid == 0) *token = idx[0];
        return;
    }
    softmax_wave(val, nc, ex, prob);
    const float selector = (float)(sp.seed % 10000ull) / 10000.0f;
    const int i = walk_wave(prob, nc, [selector](float cum) { return selector < cum; });
    if (tid == 0) *token = i < nc ? idx[i] : idx[nc - 1];
}

// ---------------------------------------------------------------------------------
// Any top-k over any vocabulary (beyond the two-pass capacity): every key, sorted on the
// device.  sample_keys_kernel writes the keys in index order (A) and a copy padded with
// zeros to a power of two P (B); a bitonic network sorts B in descending order (chunks of
// kSortChunk keys in LDS, longer strides in global passes); sample_large_final_kernel
// takes the k-th largest key as the threshold and the candidates either as a prefix of B
// (top-p walks the descending order) or, compacted in index order, from A, and wave 0
// runs the reference's tail over them with every sum in candidate order.
// ---------------------------------------------------------------------------------
constexpr int kSortChunk = 8192;  // keys per LDS bitonic chunk (64 KiB)
constexpr int kStage = 4096;      // values per LDS chunk of the ordered sums

__global__ __launch_bounds__(256) void sample_keys_kernel(const float *logits, int64_t n, const uint32_t *past,
                                                          int64_t n_past, SampleParams sp, int64_t P, uint64_t *A,
                                                          uint64_t *B) {
    __shared__ int cnt[kSampleBlock];
    constexpr int E = kSampleBlock / 256;
    const int64_t base = (int64_t)blockIdx.x * kSampleBlock;
    uint64_t e[E];
    block_keys<E>(logits, n, past, n_past, sp, base, cnt, e);
#pragma unroll
    for (int r = 0; r < E; r++) {
        const int64_t i = base + r * 256 + threadIdx.x;
        if (i < n) A[i] = e[r];
        if (i < P) B[i] = e[r];  // zeros past n
    }
}

// bitonic steps inside chunks of `chunk` keys (a power of two <= kSortChunk): for every
// size in [size_lo, size_hi] (powers of two), the strides below min(size, chunk); the
// direction of a pair follows its global index (descending where index & size == 0)
__global__ __launch_bounds__(1024) void bitonic_lds_kernel(uint64_t *keys, int chunk, int64_t size_lo,
                                                           int64_t size_hi) {
    __shared__ uint64_t a[kSortChunk];
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    for (int j = threadIdx.x; j < chunk; j += 1024) a[j] = keys[c0 + j];
    __syncthreads();
    for (int64_t size = size_lo; size <= size_hi; size <<= 1) {
        for (int stride = (int)std::min<int64_t>(size, chunk) >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < chunk / 2; i += 1024) {
                const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const bool desc = ((c0 + lo) & size) == 0;
                const uint64_t x = a[lo], y = a[hi];
                if ((x < y) == desc) {
                    a[lo] = y;
                    a[hi] = x;
                }
            }
            __syncthreads();
        }
    }
    for (int j = threadIdx.x; j < chunk; j += 1024) keys[c0 + j] = a[j];
}

// one bitonic step with a stride of at least a chunk: one pair per thread
__global__ __launch_bounds__(256) void bitonic_global_kernel(uint64_t *keys, int64_t P, int64_t size, int64_t stride) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P / 2) return;
    const int64_t lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
    const bool desc = (lo & size) == 0;
    const uint64_t x = keys[lo], y = keys[hi];
    if ((x < y) == desc) {
        keys[lo] = y;
        keys[hi] = x;
    }
}

// The f32 sum ((s + p[0]) + p[1]) + ... of a global array in element order, the same in
// every lane of the calling wave: chunks staged in LDS by the wave, then ordered_sum.
__device__ float ordered_sum_g(const float *p, int64_t n, float *stage, float s) {
    const int lane = threadIdx.x & 63;
    for (int64_t c0 = 0; c0 < n; c0 += kStage) {
        const int cn = (int)std::min<int64_t>(kStage, n - c0);
        for (int j = 4 * lane; j < cn; j += 256)
            *reinterpret_cast<floatx4 *>(stage + j) = *reinterpret_cast<const floatx4 *>(p + c0 + j);
        wave_sync();
        for (int i = 0; i < cn; i += 4) {
            const floatx4 v = *reinterpret_cast<const floatx4 *>(stage + i);
            s += v[0];
            if (i + 1 < cn) s += v[1];
            if (i + 2 < cn) s += v[2];
            if (i + 3 < cn) s += v[3];
        }
        wave_sync();
    }
    return s;
}

// within one staged chunk: continue the cumulative sum `cum` over v[0..cn) in order (16-byte
// broadcast reads), returning the first index where it meets `stop`, or -1
template <class F>
__device__ __forceinline__ int walk_chunk(const float *v, int cn, float &cum, F stop) {
    for (int i = 0; i < cn; i += 4) {
        const floatx4 q = *reinterpret_cast<const floatx4 *>(v + i);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (i + j >= cn) return -1;
            cum += q[j];
            if (stop(cum)) return i + j;
        }
    }
    return -1;
}

// the first i with (cumulative sum of p[0..i] in order) meeting `stop` (n when none)
template <class F>
__device__ int64_t walk_g(const float *p, int64_t n, float *stage, F stop) {
    const int lane = threadIdx.x & 63;
    float cum = 0.0f;
    for (int64_t c0 = 0; c0 < n; c0 += kStage) {
        const int cn = (int)std::min<int64_t>(kStage, n - c0);
        for (int j = 4 * lane; j < cn; j += 256)
            *reinterpret_cast<floatx4 *>(stage + j) = *reinterpret_cast<const floatx4 *>(p + c0 + j);
        wave_sync();
        const int hit = walk_chunk(stage, cn, cum, stop);
        wave_sync();
        if (hit >= 0) return c0 + hit;
    }
    return n;
}

// softmax_candidates (sampling.rs:371-391) of val[0..n) into p, by wave 0, global arrays
__device__ void softmax_g(const float *val, int64_t n, float *ex, float *p, float *stage) {
    const int lane = threadIdx.x & 63;
    float mx = -INFINITY;
    for (int64_t i = lane; i < n; i += 64) mx = fmaxf(mx, val[i]);
    mx = wave_max(mx);
    if (!(fabsf(mx) <= 3.402823466e38f)) {
        for (int64_t i = lane; i < n; i += 64) p[i] = 1.0f / (float)n;
        __threadfence_block();
        wave_sync();
        return;
    }
    for (int64_t i = lane; i < n; i += 64) ex[i] = expf(val[i] - mx);
    __threadfence_block();
    wave_sync();
    const float sum = ordered_sum_g(ex, n, stage, 0.0f);
    if (!(fabsf(sum) <= 3.402823466e38f) || sum == 0.0f) {
        for (int64_t i = lane; i < n; i += 64) p[i] = 1.0f / (float)n;
    } else {
        for (int64_t i = lane; i < n; i += 64) p[i] = ex[i] / sum;
    }
    __threadfence_block();
    wave_sync();
}

// work: val | ex | prob (f32) | idx (u32), each n + 4 long from 16-byte aligned starts
__global__ __launch_bounds__(1024) void sample_large_final_kernel(const float *logits, int64_t n, const uint64_t *A,
                                                                 const uint64_t *B, SampleParams sp, float *work,
                                                                 int64_t stride, uint32_t *token) {
    __shared__ float stage[kStage];
    __shared__ int64_t wsum[16][2];
    __shared__ int64_t nc_s;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t k = sp.k;
    float *val = work, *ex = work + stride, *prob = work + 2 * stride;
    uint32_t *idx = reinterpret_cast<uint32_t *>(work + 3 * stride);
    const bool keep_inf = sp.keep_inf != 0;
    if (k > 0) {
        if (sp.use_top_p) {
            // descending order: the candidates are B[a, a + f) (a: the +inf keys in front
            // that are not candidates, only when top_k is Some)
            int64_t f = 0, a = 0;
            for (int64_t j = tid; j < k; j += 1024) {
                const uint64_t s = B[j];
                f += key_cand(s, keep_inf) ? 1 : 0;
                a += (!keep_inf && (uint32_t)(s >> 32) == kOrdPosInf) ? 1 : 0;
            }
            for (int o = 32; o > 0; o >>= 1) {
                f += __shfl_xor(f, o, 64);
                a += __shfl_xor(a, o, 64);
            }
            if (lane == 0) {
                wsum[wv][0] = f;
                wsum[wv][1] = a;
            }
            __syncthreads();
            f = a = 0;
            for (int w = 0; w < 16; w++) {
                f += wsum[w][0];
                a += wsum[w][1];
            }
            for (int64_t j = tid; j < f; j += 1024) {
                const uint64_t s = B[a + j];
                val[j] = key_val(s);
                idx[j] = key_idx(s);
            }
            if (tid == 0) nc_s = f;
        } else {
            // index order: the keys of A at or above the k-th largest, candidates only;
            // thread t compacts its contiguous range, offsets from a block scan
            const uint64_t T = B[k - 1];
            const int64_t per = (n + 1023) / 1024, i0 = tid * per, i1 = std::min<int64_t>(n, i0 + per);
            int64_t c = 0;
            for (int64_t i = i0; i < i1; i++) c += (A[i] >= T && key_cand(A[i], keep_inf)) ? 1 : 0;
            int64_t incl = c;
            for (int o = 1; o < 64; o <<= 1) {
                const int64_t v = __shfl_up(incl, o, 64);
                if (lane >= o) incl += v;
            }
            if (lane == 63) wsum[wv][0] = incl;
            __syncthreads();
            int64_t before = incl - c;
            for (int w = 0; w < wv; w++) before += wsum[w][0];
            for (int64_t i = i0; i < i1; i++) {
                const uint64_t s = A[i];
                if (s >= T && key_cand(s, keep_inf)) {
                    val[before] = key_val(s);
                    idx[before] = (uint32_t)i;
                    before++;
                }
            }
            if (tid == 1023) nc_s = before;
        }
    } else if (tid == 0) {
        nc_s = 0;
    }
    __threadfence_block();
    __syncthreads();
    if (tid >= 64) return;
    int64_t nc = nc_s;
    if (sp.use_top_p && nc > 0) {
        softmax_g(val, nc, ex, prob, stage);
        const float tp = sp.top_p;
        const int64_t i = walk_g(prob, nc, stage, [tp](float cum) { return cum >= tp; });
        nc = i < nc ? i + 1 : nc;
    }
    if (nc == 0) {
        if (tid == 0) argmax_slice_serial(logits, n, token);
        return;
    }
    if (nc == 1) {
        if (tid == 0) *token = idx[0];
        return;
    }
    softmax_g(val, nc, ex, prob, stage);
    const float selector = (float)(sp.seed % 10000ull) / 10000.0f;
    const int64_t i = walk_g(prob, nc, stage, [selector](float cum) { return selector < cum; });
    if (tid == 0) *token = i < nc ? idx[i] : idx[nc - 1];
}

int64_t pow2_at_least(int64_t n) {
    int64_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

struct LargeScratch {
    uint64_t *A, *B;
    float *work;
    int64_t stride, P;
};

LargeScratch large_carve(void *base, int64_t n, size_t *bytes) {
    LargeScratch L;
    L.P = pow2_at_least(std::max<int64_t>(n, 2));
    L.stride = (n + 4 + 63) / 64 * 64;
    uint8_t *b = reinterpret_cast<uint8_t *>(base);
    size_t off = 0;
    L.A = reinterpret_cast<uint64_t *>(b + off);
    off += ((size_t)n * 8 + 255) & ~(size_t)255;
    L.B = reinterpret_cast<uint64_t *>(b + off);
    off += ((size_t)L.P * 8 + 255) & ~(size_t)255;
    L.work = reinterpret_cast<float *>(b + off);
    off += (size_t)L.stride * 16;
    if (bytes) *bytes = off;
    return L;
}

}  // namespace

bool sample_two_pass(int64_t n, int64_t k) {
    const int64_t blocks = (n + kSampleBlock - 1) / kSampleBlock;
    const int64_t kk = std::min<int64_t>(std::max<int64_t>(k, 1), kSampleBlock);
    return blocks * kk <= kSampleMaxCand;
}

size_t sample_scratch_bytes(int64_t n, int64_t k) {
    if (!sample_two_pass(n, k)) {
        size_t b = 0;
        large_carve(nullptr, n, &b);
        return b;
    }
    const int64_t blocks = (n + kSampleBlock - 1) / kSampleBlock;
    const int64_t kk = std::min<int64_t>(std::max<int64_t>(k, 1), kSampleBlock);
    return (((size_t)blocks * kk * 8 + 255) & ~(size_t)255) + (size_t)kSampleMaxCand * 16;
}

bool sample_supported(int64_t n, int64_t k) { return n >= 1 && n <= 0xFFFFFFFFll && k >= 0; }

// ---- fixed device scratch for the allocation-free entry point -----------------------
//
// One array per GPU (each device that loads the library holds its own copy until the
// process ends).  Host code never uses its name as an address: the name is a host-side
// stand-in, so its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and that address is what kernels and
// copies receive.

static __device__ __align__(256) uint8_t scratch[kSampleStaticScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
void *g_static_ptr[kMaxDevices] = {};
}  // namespace

int sample_static_scratch(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_static_mu);
    if (!g_static_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_static_ptr[dev] = p;
    }
    *out = g_static_ptr[dev];
    return (int)hipSuccess;
}

int launch_sample(const float *logits, int64_t n, const uint32_t *past, int64_t n_past, float temperature, int64_t k,
                  int keep_inf, int use_top_p, float top_p, float rep, int rep_on, float freq, int freq_on,
                  uint64_t seed, uint32_t *token, void *scratch, void *stream) {
    SampleParams sp;
    sp.keep_inf = keep_inf;
    sp.temperature = temperature;
    sp.top_p = top_p;
    sp.rep = rep;
    sp.freq = freq;
    sp.rep_on = rep_on;
    sp.freq_on = freq_on;
    sp.use_top_p = use_top_p;
    sp.k = k;
    sp.seed = seed;
    const int64_t blocks = (n + kSampleBlock - 1) / kSampleBlock;
    if (!sample_two_pass(n, k)) {
        hipStream_t st = (hipStream_t)stream;
        const LargeScratch L = large_carve(scratch, n, nullptr);
        hipLaunchKernelGGL(sample_keys_kernel, dim3((unsigned)((L.P + kSampleBlock - 1) / kSampleBlock)), dim3(256), 0,
                           st, logits, n, past, n_past, sp, L.P, L.A, L.B);
        const int chunk = (int)std::min<int64_t>(L.P, kSortChunk);
        hipLaunchKernelGGL(bitonic_lds_kernel, dim3((unsigned)(L.P / chunk)), dim3(1024), 0, st, L.B, chunk, (int64_t)2,
                           (int64_t)chunk);
        for (int64_t size = 2 * (int64_t)chunk; size <= L.P; size <<= 1) {
            for (int64_t stride = size / 2; stride >= chunk; stride >>= 1)
                hipLaunchKernelGGL(bitonic_global_kernel, dim3((unsigned)((L.P / 2 + 255) / 256)), dim3(256), 0, st,
                                   L.B, L.P, size, stride);
            hipLaunchKernelGGL(bitonic_lds_kernel, dim3((unsigned)(L.P / chunk)), dim3(1024), 0, st, L.B, chunk, size,
                               size);
        }
        hipLaunchKernelGGL(sample_large_final_kernel, dim3(1), dim3(1024), 0, st, logits, n, L.A, L.B, sp, L.work,
                           L.stride, token);
        return (int)hipGetLastError();
    }
    const int kk = (int)std::min<int64_t>(std::max<int64_t>(k, 1), kSampleBlock);
    uint64_t *cand = reinterpret_cast<uint64_t *>(scratch);
    float *work = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(scratch) +
                                            (((size_t)blocks * kk * 8 + 255) & ~(size_t)255));
    hipLaunchKernelGGL(sample_local_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, logits, n, past,
                       n_past, sp, kk, cand);
    // up to 4096 candidates (top-k up to 54 over a 151936 vocabulary) four waves hold
    // them, and the select's barriers are cheaper than with sixteen
    const int ncand = (int)(blocks * kk);
    if (ncand <= 256 * 16)
        hipLaunchKernelGGL((sample_final_kernel<256>), dim3(1), dim3(256), 0, (hipStream_t)stream, logits, n, cand,
                           ncand, sp, work, token);
    else
        hipLaunchKernelGGL((sample_final_kernel<1024>), dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, n, cand,
                           ncand, sp, work, token);
    return (int)hipGetLastError();
}

}  // namespace nnq
