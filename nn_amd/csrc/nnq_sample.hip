// Token sampling on gfx950: sample_token (crates/nn-gptoss/src/sampling.rs:136-185) over a
// logits vector that stays on the device, e.g. straight out of the LM-head GEMV.
//
//   sample_local_kernel  one workgroup per 2048 logits: repetition / frequency penalties
//                        (per occurrence in past_tokens, :277-306), temperature (:193-199),
//                        then the block's logits as 64-bit keys (orderable value, inverted
//                        index) sorted descending in LDS (bitonic); the block's best
//                        min(k, 2048) keys go to the candidate buffer
//   sample_final_kernel  one workgroup: the candidates sorted the same way give the top k
//                        (apply_top_k, :245-275; equal values keep the lower index first),
//                        then one thread runs the short sequential tail exactly as the
//                        reference does: finite candidates in index order, top-p over the
//                        descending order (:211-238), softmax and the seed's selector walk
//                        (:340-391), and the argmax_slice fallback (:394-400) when no
//                        candidate is left.
// NaN logits sort below -inf and never become candidates.
#include <algorithm>
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
// descending key order = descending value, then ascending index; NaN and padding at the end
__device__ __forceinline__ uint64_t cand_key(float v, uint32_t idx) {
    if (v != v) return 0xFFFFFFFFull - idx;  // below every real value (ord(-inf) > 0)
    return ((uint64_t)ord_f32(v) << 32) | (0xFFFFFFFFull - idx);
}
__device__ __forceinline__ uint32_t key_idx(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull); }
__device__ __forceinline__ float key_val(uint64_t k) { return unord_f32((uint32_t)(k >> 32)); }

// Bitonic sort, descending, of E * nact 64-bit keys (a power of two) held E per thread in
// registers: thread t < nact owns elements E t .. E t + E - 1 in e[].  Stages whose partner
// is in the same thread (stride < E) run in registers; the others publish the thread's
// keys to `buf` (E * nact entries, element r of thread t at r * nact + t, so that a wave's
// accesses fall in distinct banks), read the partner thread's, and keep the larger or
// smaller of each pair.  Every thread of the workgroup calls it (barriers).
template <int E>
__device__ void bitonic_reg(uint64_t (&e)[E], uint64_t *buf, int nact) {
    const int t = threadIdx.x;
    const bool act = t < nact;
    const int n = E * nact;
    for (int size = 2; size <= n; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= E) {
                if (act)
#pragma unroll
                    for (int r = 0; r < E; r++) buf[r * nact + t] = e[r];
                __syncthreads();
                if (act) {
                    const int pt = t ^ (stride / E);
#pragma unroll
                    for (int r = 0; r < E; r++) {
                        const int j = E * t + r, p = E * pt + r;
                        const uint64_t ep = buf[r * nact + pt];
                        const bool desc = ((j < p ? j : p) & size) == 0, lo = j < p;
                        const uint64_t mx = e[r] > ep ? e[r] : ep, mn = e[r] > ep ? ep : e[r];
                        e[r] = (lo == desc) ? mx : mn;
                    }
                }
                __syncthreads();
            } else if (act) {
#pragma unroll
                for (int r = 0; r < E; r++)
                    if ((r & stride) == 0) {
                        const int p = r | stride;
                        const bool desc = ((E * t + r) & size) == 0;
                        const uint64_t x = e[r], y = e[p];
                        if ((x < y) == desc) {
                            e[r] = y;
                            e[p] = x;
                        }
                    }
            }
        }
}

// keys[0..n) (n a power of two, at most 1024 * 16) sorted descending in place, 1024 threads
__device__ void sort_desc_lds(uint64_t *keys, int n) {
    auto run = [&](auto ec) {
        constexpr int E = decltype(ec)::value;
        const int nact = n / E;
        uint64_t e[E];
        if ((int)threadIdx.x < nact)
#pragma unroll
            for (int r = 0; r < E; r++) e[r] = keys[E * threadIdx.x + r];
        __syncthreads();
        bitonic_reg<E>(e, keys, nact);
        if ((int)threadIdx.x < nact)
#pragma unroll
            for (int r = 0; r < E; r++) keys[E * threadIdx.x + r] = e[r];
        __syncthreads();
    };
    if (n <= 1024) run(std::integral_constant<int, 1>{});
    else if (n <= 2048) run(std::integral_constant<int, 2>{});
    else if (n <= 4096) run(std::integral_constant<int, 4>{});
    else if (n <= 8192) run(std::integral_constant<int, 8>{});
    else run(std::integral_constant<int, 16>{});
}

struct SampleParams {
    float temperature, top_p, rep, freq;
    int rep_on, freq_on, use_top_p;
    int64_t k;  // candidates kept by top-k (already min(top_k, n); 0: none)
    uint64_t seed;
};

__global__ __launch_bounds__(256) void sample_local_kernel(const float *logits, int64_t n, const uint32_t *past,
                                                           int64_t n_past, SampleParams sp, int kk, uint64_t *cand) {
    __shared__ uint64_t keys[kSampleBlock];
    __shared__ int cnt[kSampleBlock];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * kSampleBlock;
    const bool pen = (sp.rep_on || sp.freq_on) && n_past > 0;
    if (pen) {
        for (int j = tid; j < kSampleBlock; j += 256) cnt[j] = 0;
        __syncthreads();
        for (int64_t i = tid; i < n_past; i += 256) {
            const int64_t t = past[i];
            if (t >= base && t < base + kSampleBlock && t < n) atomicAdd(&cnt[t - base], 1);
        }
        __syncthreads();
    }
    // thread t: elements 8t .. 8t + 7 of the block (loaded as two coalesced passes)
    constexpr int E = kSampleBlock / 256;
    uint64_t e[E];
#pragma unroll
    for (int r = 0; r < E; r++) {
        const int j = E * tid + r;
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
    bitonic_reg<E>(e, keys, 256);
#pragma unroll
    for (int r = 0; r < E; r++)
        if (E * tid + r < kk) cand[(int64_t)blockIdx.x * kk + E * tid + r] = e[r];
}

// softmax_candidates (sampling.rs:371-391) over c[0..n) into p[0..n), one thread
__device__ void softmax_seq(const float *v, int n, float *p) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, v[i]);
    if (!(fabsf(mx) <= 3.402823466e38f)) {
        for (int i = 0; i < n; i++) p[i] = 1.0f / (float)n;
        return;
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        p[i] = expf(v[i] - mx);
        sum += p[i];
    }
    if (!(fabsf(sum) <= 3.402823466e38f) || sum == 0.0f) {
        for (int i = 0; i < n; i++) p[i] = 1.0f / (float)n;
        return;
    }
    for (int i = 0; i < n; i++) p[i] = p[i] / sum;
}

__global__ __launch_bounds__(1024) void sample_final_kernel(const float *logits, int64_t n, const uint64_t *cand,
                                                            int ncand, SampleParams sp, float *work,
                                                            uint32_t *token) {
    __shared__ uint64_t keys[kSampleMaxCand];
    // the tail's arrays: in the upper half of `keys` (free once the top k, k <= 2048, sit
    // in keys[0..k)), else in the global scratch
    const bool in_lds = sp.k <= 2048;
    float *val = in_lds ? reinterpret_cast<float *>(keys + kSampleMaxCand / 2) : work;
    float *prob = in_lds ? val + 2048 : work + kSampleMaxCand;
    uint32_t *idx = in_lds ? reinterpret_cast<uint32_t *>(val + 4096) : reinterpret_cast<uint32_t *>(work + 2 * kSampleMaxCand);
    int P = 1;
    while (P < ncand) P <<= 1;
    for (int j = threadIdx.x; j < P; j += 1024) keys[j] = j < ncand ? cand[j] : 0ull;
    __syncthreads();
    sort_desc_lds(keys, P);
    const int k = (int)sp.k;  // keys[0..k) are the top k (k <= ncand)
    if (!sp.use_top_p && k > 1) {
        // Without top-p the reference walks its candidates in index order: re-sort the k
        // by (finite first, ascending index), carrying each one's position (< 2^14) so
        // that its value can be found again in `val`.
        int Q = 1;
        while (Q < k) Q <<= 1;
        for (int j = threadIdx.x; j < k; j += 1024) val[j] = key_val(keys[j]);
        __syncthreads();
        for (int j = threadIdx.x; j < Q; j += 1024) {
            uint64_t r = 0;
            if (j < k) {
                const uint64_t key = keys[j];
                const bool fin = (key >> 32) != 0 && fabsf(val[j]) <= 3.402823466e38f;
                r = fin ? (0x8000000000000000ull | ((uint64_t)(0xFFFFFFFFu - key_idx(key)) << 14) | (uint64_t)j) : 0ull;
            }
            keys[j] = r;
        }
        __syncthreads();
        sort_desc_lds(keys, Q);
    }
    if (threadIdx.x != 0) return;
    // the finite candidates, in the order the reference walks them
    int nc = 0;
    if (!sp.use_top_p && k > 1) {
        for (int j = 0; j < k; j++) {
            const uint64_t r = keys[j];
            if (!(r >> 63)) break;  // the non-finite ones sort last
            const int pos = (int)(r & 0x3FFFull);
            prob[nc] = val[pos];
            idx[nc] = 0xFFFFFFFFu - (uint32_t)((r >> 14) & 0xFFFFFFFFull);
            nc++;
        }
        for (int j = 0; j < nc; j++) val[j] = prob[j];
    } else {
        for (int j = 0; j < k; j++) {
            const uint64_t key = keys[j];
            const float v = key_val(key);
            if ((key >> 32) != 0 && fabsf(v) <= 3.402823466e38f) {
                val[nc] = v;
                idx[nc] = key_idx(key);
                nc++;
            }
        }
        if (sp.use_top_p && nc > 0) {
            // apply_top_p_candidates: descending order (ties by index), the smallest
            // prefix whose cumulative probability reaches top_p
            softmax_seq(val, nc, prob);
            float cum = 0.0f;
            int keep = 0;
            for (int i = 0; i < nc; i++) {
                cum += prob[i];
                keep = i + 1;
                if (cum >= sp.top_p) break;
            }
            nc = keep;
        }
    }
    if (nc == 0) {
        // argmax_slice of the original logits: the running maximum moves on unless it
        // compares greater (ties and NaN move on)
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
        return;
    }
    if (nc == 1) {
        *token = idx[0];
        return;
    }
    softmax_seq(val, nc, prob);
    const float selector = (float)(sp.seed % 10000ull) / 10000.0f;
    float cum = 0.0f;
    uint32_t out = idx[nc - 1];
    for (int i = 0; i < nc; i++) {
        cum += prob[i];
        if (selector < cum) {
            out = idx[i];
            break;
        }
    }
    *token = out;
}

}  // namespace

size_t sample_scratch_bytes(int64_t n, int64_t k) {
    const int64_t blocks = (n + kSampleBlock - 1) / kSampleBlock;
    const int64_t kk = std::min<int64_t>(std::max<int64_t>(k, 1), kSampleBlock);
    return (size_t)blocks * kk * 8 + 256 + (size_t)kSampleMaxCand * 12;
}

bool sample_supported(int64_t n, int64_t k) {
    const int64_t blocks = (n + kSampleBlock - 1) / kSampleBlock;
    const int64_t kk = std::min<int64_t>(std::max<int64_t>(k, 1), kSampleBlock);
    return blocks * kk <= kSampleMaxCand && n <= 0xFFFFFFFFll;
}

int launch_sample(const float *logits, int64_t n, const uint32_t *past, int64_t n_past, float temperature, int64_t k,
                  int use_top_p, float top_p, float rep, int rep_on, float freq, int freq_on, uint64_t seed,
                  uint32_t *token, void *scratch, void *stream) {
    SampleParams sp;
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
    const int kk = (int)std::min<int64_t>(std::max<int64_t>(k, 1), kSampleBlock);
    uint64_t *cand = reinterpret_cast<uint64_t *>(scratch);
    float *work = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(scratch) +
                                            (((size_t)blocks * kk * 8 + 255) & ~(size_t)255));
    hipLaunchKernelGGL(sample_local_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, logits, n, past,
                       n_past, sp, kk, cand);
    hipLaunchKernelGGL(sample_final_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, n, cand,
                       (int)(blocks * kk), sp, work, token);
    return (int)hipGetLastError();
}

}  // namespace nnq
