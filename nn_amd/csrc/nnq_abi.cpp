// C ABI of the nnq library (include/nnq.h): validation, device memory, repack
// upload and kernel dispatch.  Error semantics follow the reference's
// quantized-matmul / tensor errors; messages are kept per thread.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "nnq_internal.h"

using namespace nnq;

struct nnq_weight {
    Layout L;
    uint8_t *dev = nullptr;
    int device = 0;
};

struct nnq_mlp {
    nnq_weight *gu = nullptr;    // [2 * inter, hidden]: gate rows, then up rows (or interleaved8)
    nnq_weight *down = nullptr;  // [hidden, inter]
    int64_t hidden = 0, inter = 0;
    bool interleaved8 = false;   // rows 16j .. 16j + 7 = gate rows 8j .., 16j + 8 .. = up rows 8j ..
};

struct nnq_router {
    float *w = nullptr;     // [E, hidden] f32
    float *b = nullptr;     // [E] f32 or null
    int64_t E = 0, H = 0;
};

struct nnq_moe {
    MoeDev d;
    int device = 0;
    std::vector<void *> allocs;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return fail(NNQ_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    return fail(NNQ_ERR_DISPATCH_FAILED, "%s: %s", what, hipGetErrorString(e));
}

// a workspace whose size does not fit size_t (absurd shapes)
int size_fail() { return fail(NNQ_ERR_OUT_OF_MEMORY, "workspace size overflows"); }

#define HIP_TRY(expr, what)                       \
    do {                                          \
        hipError_t _e = (expr);                   \
        if (_e != hipSuccess) return hip_fail(_e, what); \
    } while (0)

// experts of a MoE layer: the routing kernels keep a token's E probabilities (4 tokens per
// workgroup) and the permutation its E running counts in LDS
constexpr int kMoeMaxExperts = 4096;

size_t block_elems(int fmt) { return fmt == NNQ_FMT_Q8_0 ? 32 : 256; }
size_t block_bytes(int fmt) {
    switch (fmt) {
    case NNQ_FMT_Q8_0: return 34;
    case NNQ_FMT_Q4_K: return 144;
    case NNQ_FMT_Q6_K: return 210;
    }
    return 0;
}

// Workspaces.  Calls on one stream run in order, so they can share one buffer:
//  - eager calls use the stream's workspace (keyed by device and stream).  It grows by a
//    stream-ordered allocation, and the buffer it replaces is freed stream-ordered, after
//    the work already queued on the stream;
//  - calls captured into a HIP graph use a workspace of their capture sequence (keyed by
//    device, stream and capture id), allocated with the capture's ban on allocation calls
//    relaxed for this thread, so the graph holds no allocation nodes.  A graph keeps
//    reading that buffer whenever and on whatever stream it is replayed, so it is never
//    shared with eager calls or other captures, and it is kept until
//    nnq_release_capture_workspaces (the library cannot see when the graph is destroyed).
//    A buffer outgrown within one capture is kept as well, since the calls captured
//    before hold it.
// If the relaxed allocation is refused, the call takes a stream-ordered allocation that
// becomes nodes of the graph (freed by the graph after the call's work).
//
// Stream order alone does not keep two host threads that call on one stream apart: their
// copies and kernels could interleave on the shared buffer, and a call that grows the
// workspace would free the buffer that another thread's call holds but has not yet used.
// So a call holds its stream's lock (recursive: a call may take scratch twice) from its
// first workspace request until its last enqueue.
//
// hipStreamPerThread names a different stream in each host thread, so for that handle the
// thread is part of the key.
struct StreamKey {
    int dev;
    hipStream_t st;
    std::thread::id owner;
    bool operator==(const StreamKey &o) const { return dev == o.dev && st == o.st && owner == o.owner; }
};
struct Workspace {
    StreamKey key;
    unsigned long long capture;  // 0: eager
    void *p;
    size_t n;
};
struct StreamLock {
    StreamKey key;
    std::recursive_mutex mu;
};
struct Retired {
    int dev;
    void *p;
};
std::mutex g_ws_mu;
std::vector<Workspace> g_ws;
std::vector<Retired> g_capture_retired;
std::vector<std::unique_ptr<StreamLock>> g_stream_locks;  // never erased: held locks stay valid

hipError_t stream_key(hipStream_t st, StreamKey *k) {
    k->st = st;
    k->owner = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    return hipGetDevice(&k->dev);
}

std::recursive_mutex &stream_lock(const StreamKey &k) {
    std::lock_guard<std::mutex> g(g_ws_mu);
    for (auto &l : g_stream_locks)
        if (l->key == k) return l->mu;
    g_stream_locks.push_back(std::make_unique<StreamLock>());
    g_stream_locks.back()->key = k;
    return g_stream_locks.back()->mu;
}

hipError_t stream_workspace(const StreamKey &key, size_t n, void **out, bool *owned) {
    const hipStream_t st = key.st;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    hipError_t e = hipStreamGetCaptureInfo(st, &cs, &cid);
    if (e != hipSuccess) return e;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (!capturing) cid = 0;
    std::lock_guard<std::mutex> g(g_ws_mu);
    Workspace *w = nullptr;
    for (auto &x : g_ws)
        if (x.key == key && x.capture == cid) w = &x;
    if (w && w->n >= n) {
        *out = w->p;
        *owned = false;
        return hipSuccess;
    }
    size_t sz = std::max<size_t>(n, (size_t)1 << 20);
    if (w) sz = std::max(sz, 2 * w->n);
    void *p = nullptr;
    if (capturing) {
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        (void)hipThreadExchangeStreamCaptureMode(&mode);
        e = hipMalloc(&p, sz);
        (void)hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            *owned = true;
            return hipMallocAsync(out, n, st);
        }
        if (w) g_capture_retired.push_back(Retired{key.dev, w->p});
    } else {
        e = hipMallocAsync(&p, sz, st);
        if (e != hipSuccess) return e;
        if (w) {
            e = hipFreeAsync(w->p, st);  // after the work queued on st that uses it
            if (e != hipSuccess) {
                (void)hipFreeAsync(p, st);
                return e;
            }
        }
    }
    if (w) {
        w->p = p;
        w->n = sz;
    } else {
        g_ws.push_back(Workspace{key, cid, p, sz});
    }
    *out = p;
    *owned = false;
    return hipSuccess;
}

// frees the eager workspace of `st` on the current device (stream-ordered on st), once no
// call on the stream holds it
hipError_t release_stream_workspace(hipStream_t st) {
    StreamKey key;
    hipError_t e = stream_key(st, &key);
    if (e != hipSuccess) return e;
    std::lock_guard<std::recursive_mutex> call(stream_lock(key));
    std::lock_guard<std::mutex> g(g_ws_mu);
    for (size_t i = 0; i < g_ws.size(); i++)
        if (g_ws[i].key == key && g_ws[i].capture == 0) {
            e = hipFreeAsync(g_ws[i].p, st);
            g_ws.erase(g_ws.begin() + (ptrdiff_t)i);
            return e;
        }
    return hipSuccess;
}

// frees every capture workspace on the current device; the caller guarantees that no
// graph captured with library calls on this device runs or is replayed afterwards
hipError_t release_capture_workspaces() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::vector<void *> victims;
    {
        std::lock_guard<std::mutex> g(g_ws_mu);
        for (size_t i = 0; i < g_ws.size();)
            if (g_ws[i].key.dev == dev && g_ws[i].capture != 0) {
                victims.push_back(g_ws[i].p);
                g_ws.erase(g_ws.begin() + (ptrdiff_t)i);
            } else {
                i++;
            }
        for (size_t i = 0; i < g_capture_retired.size();)
            if (g_capture_retired[i].dev == dev) {
                victims.push_back(g_capture_retired[i].p);
                g_capture_retired.erase(g_capture_retired.begin() + (ptrdiff_t)i);
            } else {
                i++;
            }
    }
    // relaxed for this thread, so that a capture another thread runs is not invalidated
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    hipError_t first = hipSuccess;
    for (void *p : victims) {
        e = hipFree(p);
        if (e != hipSuccess && first == hipSuccess) first = e;
    }
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    return first;
}

// Scratch of one call: the stream's workspace (or, under capture when that is too
// small, a stream-ordered allocation freed after the call's work).  The first alloc takes
// the stream's lock, which the Scratch holds until it is destroyed, i.e. after the call
// has enqueued its work (every entry point declares its Scratch before its launches).
// Calls from several threads on one stream therefore take the workspace one at a time.
struct Scratch {
    void *p = nullptr;
    hipStream_t s = nullptr;
    bool owned = false;
    std::unique_lock<std::recursive_mutex> call;  // released after the destructor's body
    ~Scratch() {
        if (owned && p) (void)hipFreeAsync(p, s);
    }
    hipError_t alloc(size_t n, hipStream_t st) {
        s = st;
        StreamKey key;
        hipError_t e = stream_key(st, &key);
        if (e != hipSuccess) return e;
        if (!call.owns_lock()) call = std::unique_lock<std::recursive_mutex>(stream_lock(key));
        return stream_workspace(key, n ? n : 16, &p, &owned);
    }
};


// The kernels load activations as 16-byte vectors and store outputs as 4-byte words (or
// wider); an input or output at an address that does not allow that (a narrowed view)
// goes through the call's workspace with a device copy.
inline bool misaligned_in(const void *p) { return ((uintptr_t)p & 15) != 0; }
inline bool misaligned_out(const void *p) { return ((uintptr_t)p & 3) != 0; }

template <class F>
void parallel_for(int64_t n, F &&fn) {
    int64_t nt = std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()), std::max<int64_t>(1, n / 64));
    if (nt <= 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> th;
    int64_t per = (n + nt - 1) / nt;
    for (int64_t t = 0; t < nt; t++) {
        int64_t lo = t * per, hi = std::min(n, lo + per);
        if (lo < hi) th.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto &x : th) x.join();
}

}  // namespace

int nnq::set_error(int code, const char *msg) {
    g_err = msg;
    return code;
}

extern "C" {

const char *nnq_last_error(void) { return g_err.c_str(); }

int nnq_release_workspace(void *stream) {
    hipError_t e = release_stream_workspace((hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "release workspace");
    return NNQ_OK;
}

int nnq_release_capture_workspaces(void) {
    hipError_t e = release_capture_workspaces();
    if (e != hipSuccess) return hip_fail(e, "release capture workspaces");
    return NNQ_OK;
}

int nnq_device_count(int *count) {
    if (!count) return fail(NNQ_ERR_INVALID_ARGUMENT, "count is null");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    *count = (e == hipSuccess) ? c : 0;
    return NNQ_OK;
}

int nnq_init(int device) {
    int c = 0;
    if (hipGetDeviceCount(&c) != hipSuccess || c == 0) return fail(NNQ_ERR_NO_DEVICE, "no HIP device");
    if (device < 0 || device >= c) return fail(NNQ_ERR_INVALID_ARGUMENT, "device %d out of range (%d)", device, c);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (!std::strstr(prop.gcnArchName, "gfx950"))
        return fail(NNQ_ERR_UNSUPPORTED, "kernels are built for gfx950, device is %s", prop.gcnArchName);
    // the device address of the fixed scratch of nnq_linear_sample_noalloc, looked up
    // here so that the entry point's calls do no set-up work
    void *p = nullptr;
    HIP_TRY((hipError_t)sample_static_scratch(&p), "hipGetSymbolAddress(scratch)");
    return NNQ_OK;
}

int nnq_weight_create(nnq_format fmt, nnq_layout layout, const uint8_t *bytes, size_t nbytes, int64_t n, int64_t k,
                      nnq_weight **out) {
    if (!out) return fail(NNQ_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (fmt != NNQ_FMT_Q8_0 && fmt != NNQ_FMT_Q4_K && fmt != NNQ_FMT_Q6_K)
        return fail(NNQ_ERR_WRONG_FORMAT, "format %d is not a linear-weight block format", (int)fmt);
    if (n <= 0 || k <= 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "weight shape [%lld, %lld]", (long long)n, (long long)k);
    if ((size_t)k % block_elems(fmt))
        return fail(NNQ_ERR_INVALID_SHAPE, "in_features %lld is not a multiple of the block size %zu", (long long)k,
                    block_elems(fmt));
    size_t expect = (size_t)n * ((size_t)k / block_elems(fmt)) * block_bytes(fmt);
    if (nbytes != expect)
        return fail(NNQ_ERR_DATA_LENGTH, "data length mismatch: expected %zu bytes, got %zu", expect, nbytes);
    if (!bytes) return fail(NNQ_ERR_INVALID_ARGUMENT, "bytes is null");
    Layout L;
    const char *err = nullptr;
    if (!make_layout(fmt, layout, n, k, &L, &err)) return fail(NNQ_ERR_WRONG_FORMAT, "%s", err);
    std::vector<uint8_t> host(L.total());
    // repack tile by tile in parallel (disjoint output ranges)
    switch (fmt) {
    case NNQ_FMT_Q4_K:
    case NNQ_FMT_Q6_K: {
        // each tile's rows map to disjoint destination ranges; run the whole-weight repack
        // on row-tile slices of a sub-layout to parallelise.
        parallel_for(L.ntile, [&](int64_t lo, int64_t hi) {
            Layout S = L;
            S.n = std::min<int64_t>(L.n - lo * kTile, (hi - lo) * kTile);
            S.ntile = hi - lo;
            size_t per_q = L.qs_bytes / L.ntile, per_h = L.hdr_bytes / L.ntile;
            S.qs_bytes = per_q * S.ntile;
            S.hdr_bytes = per_h * S.ntile;
            S.aux_bytes = 0;
            std::vector<uint8_t> tmp(S.total());
            const uint8_t *src = bytes + (size_t)lo * kTile * (k / 256) * block_bytes(fmt);
            if (fmt == NNQ_FMT_Q4_K)
                repack_q4k(src, layout == NNQ_LAYOUT_NN_GGUF, S, tmp.data());
            else
                repack_q6k(src, S, tmp.data());
            std::memcpy(host.data() + per_q * lo, tmp.data(), S.qs_bytes);
            std::memcpy(host.data() + L.qs_bytes + per_h * lo, tmp.data() + S.qs_bytes, S.hdr_bytes);
        });
        if (fmt == NNQ_FMT_Q4_K)
            parallel_for(L.ntile, [&](int64_t lo, int64_t hi) {
                q4k_aux_plane(host.data() + L.qs_bytes, L, host.data() + L.qs_bytes + L.hdr_bytes, lo, hi);
            });
        break;
    }
    case NNQ_FMT_Q8_0:
        repack_q8_0(bytes, L, host.data());
        break;
    }
    nnq_weight *w = new nnq_weight;
    w->L = L;
    hipGetDevice(&w->device);
    hipError_t e = hipMalloc(&w->dev, L.total());
    if (e != hipSuccess) {
        delete w;
        return hip_fail(e, "hipMalloc(weight)");
    }
    e = hipMemcpy(w->dev, host.data(), L.total(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(w->dev);
        delete w;
        return hip_fail(e, "hipMemcpy(weight)");
    }
    *out = w;
    return NNQ_OK;
}

int nnq_weight_destroy(nnq_weight *w) {
    if (!w) return NNQ_OK;
    if (w->dev) hipFree(w->dev);
    delete w;
    return NNQ_OK;
}

int nnq_weight_info(const nnq_weight *w, int *fmt, int *layout, int64_t *n, int64_t *k, size_t *device_bytes) {
    if (!w) return fail(NNQ_ERR_NOT_QUANTIZED, "weight handle is null");
    if (fmt) *fmt = w->L.fmt;
    if (layout) *layout = w->L.layout;
    if (n) *n = w->L.n;
    if (k) *k = w->L.k;
    if (device_bytes) *device_bytes = w->L.total();
    return NNQ_OK;
}

int nnq_dequant(const nnq_weight *w, float *out, void *stream) {
    if (!w) return fail(NNQ_ERR_NOT_QUANTIZED, "weight handle is null");
    if (!out) return fail(NNQ_ERR_INVALID_ARGUMENT, "out is null");
    int e = launch_dequant(w->L.fmt, w->dev, w->dev + w->L.qs_bytes, w->L.n, w->L.k, w->L.ntile, w->L.nblk, out,
                           stream);
    if (e) return hip_fail((hipError_t)e, "dequant launch");
    return NNQ_OK;
}

static int check_linear(const nnq_weight *w, const void *x, nnq_dtype xd, int64_t m, int64_t k, const float *bias,
                        int64_t bias_len, void *y, nnq_dtype yd) {
    if (!w) return fail(NNQ_ERR_NOT_QUANTIZED, "weight tensor is not quantized (null handle)");
    if (m < 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "m = %lld", (long long)m);
    if (k != w->L.k)
        return fail(NNQ_ERR_SHAPE_MISMATCH,
                    "quantized matmul shape mismatch: input last dim %lld != weight in_features %lld", (long long)k,
                    (long long)w->L.k);
    if (bias && bias_len != w->L.n)
        return fail(NNQ_ERR_BIAS_MISMATCH, "bias shape mismatch: expected [%lld], got [%lld]", (long long)w->L.n,
                    (long long)bias_len);
    if (m > 0 && (!x || !y)) return fail(NNQ_ERR_INVALID_ARGUMENT, "x or y is null");
    if (xd != NNQ_F32 && xd != NNQ_BF16) return fail(NNQ_ERR_UNSUPPORTED, "input dtype %d (f32 or bf16)", (int)xd);
    if (yd != NNQ_F32 && yd != NNQ_BF16) return fail(NNQ_ERR_UNSUPPORTED, "output dtype %d (f32 or bf16)", (int)yd);
    return NNQ_OK;
}

}  // extern "C"

// One validated linear call: the MFMA GEMM (gemm_batch) or GEMV passes of up to
// 8 tokens.  GEMV-only options: x_swiglu (x holds gate | up rows of 2k f32, the input
// is silu(gate) * up; m <= 2 so one pass) and a status (mode 1 clears it in the
// first pass, mode 2 flags non-finite outputs in every pass).
static GemmArgs gemm_args(const nnq_weight *w, const void *x, nnq_dtype x_dtype, int64_t m, const float *bias, void *y,
                          nnq_dtype y_dtype) {
    const Layout &L = w->L;
    GemmArgs g{};
    g.qs = w->dev;
    g.hdr = w->dev + L.qs_bytes;
    g.aux = w->dev + L.qs_bytes + L.hdr_bytes;
    g.x = x;
    g.x_bf16 = x_dtype == NNQ_BF16;
    g.bias = bias;
    g.y = y;
    g.y_bf16 = y_dtype == NNQ_BF16;
    g.n = L.n;
    g.k = L.k;
    g.m = m;
    g.ntile = L.ntile;
    g.nblk = L.nblk;
    g.blk = L.fmt == NNQ_FMT_Q4_K ? 0 : L.fmt;
    return g;
}

// scratch a linear call of m tokens needs (the prefill GEMM's staging and split-K slabs)
// MFMA GEMM or GEMV passes (of up to 8 tokens for Q8_0, 4 otherwise), by the measured
// crossover on MI355X: Q4_K from 3 tokens with bf16 activations (the one-launch thin
// GEMM: 3 and 4 tokens at 12288x4096 in 8.8 / 8.9 us against 10.3 / 10.5 as a GEMV pass,
// level at 4096x12288; 2 tokens: 8.7 against 7.7) and from 9 with f32 ones (23.6 against
// 28.4 at 8), Q6_K from 9 (8 tokens at 4096x12288: two batched passes 27 us, GEMM 36.8), Q8_0
// from 9 with bf16 activations and from 17 with f32 ones (8 tokens in one batched GEMV
// pass: 7.9 us at 4096x4096, 17.9 at 4096x12288; 9 f32 tokens as GEMM: 20.9 and 39.2 us)
static bool gemm_batch(const nnq_weight *w, int64_t m, nnq_dtype x_dtype) {
    if (w->L.fmt == NNQ_FMT_Q4_K) return m > (x_dtype == NNQ_BF16 ? 2 : 8);
    if (w->L.fmt == NNQ_FMT_Q6_K) return m > 8;
    return m > (x_dtype == NNQ_BF16 ? 8 : 16);
}

// the prefill GEMM's scratch for m tokens run in launches of gemm_chunk_rows rows (the
// first launch's rows, or the last, shorter one's when that plan needs more)
static size_t gemm_call_scratch(const nnq_weight *w, int64_t m, nnq_dtype x_dtype) {
    const int64_t mc = gemm_chunk_rows(m, w->L.k), tail = m % mc;
    size_t b = gemm_scratch_bytes(gemm_args(w, nullptr, x_dtype, mc, nullptr, nullptr, NNQ_F32));
    if (tail) b = std::max(b, gemm_scratch_bytes(gemm_args(w, nullptr, x_dtype, tail, nullptr, nullptr, NNQ_F32)));
    return b;
}

static size_t linear_scratch_bytes(const nnq_weight *w, int64_t m, nnq_dtype x_dtype) {
    if (!gemm_batch(w, m, x_dtype)) return 0;
    return gemm_call_scratch(w, m, x_dtype);
}

static int dispatch_linear(const nnq_weight *w, const void *x, nnq_dtype x_dtype, int64_t m, const float *bias,
                           void *y, nnq_dtype y_dtype, void *stream, int x_swiglu = 0, int32_t *status = nullptr,
                           int status_mode = 0, void *ext_scratch = nullptr, int swiglu_out = 0) {
    if (m == 0) return NNQ_OK;
    if (swiglu_out && (w->L.fmt != NNQ_FMT_Q4_K || m > 2 || x_swiglu || bias || w->L.n % 16))
        return fail(NNQ_ERR_INVALID_ARGUMENT, "SwiGLU epilogue needs a Q4_K decode GEMV over whole tiles");
    const Layout &L = w->L;
    const int64_t k = L.k;
    const size_t xe = x_dtype == NNQ_BF16 ? 2 : 4, ye = y_dtype == NNQ_BF16 ? 2 : 4;
    if (gemm_batch(w, m, x_dtype) && !x_swiglu) {
        // prefill: MFMA GEMM (Q4_K: nnq_gemm*.hip; Q8_0 / Q6_K: nnq_gemm_blk.hip), in launches
        // of gemm_chunk_rows rows (their 32-bit activation offsets; one launch up to ~43k
        // rows at K = 12288), one after another on the stream sharing the scratch
        const int64_t mc = gemm_chunk_rows(m, k);
        Scratch s;
        void *scr = ext_scratch;
        if (!scr) {
            HIP_TRY(s.alloc(gemm_call_scratch(w, m, x_dtype), (hipStream_t)stream), "scratch alloc");
            scr = s.p;
        }
        for (int64_t m0 = 0; m0 < m; m0 += mc) {
            const int64_t rows = std::min(mc, m - m0);
            GemmArgs g = gemm_args(w, (const uint8_t *)x + (size_t)m0 * k * xe, x_dtype, rows, bias,
                                   (uint8_t *)y + (size_t)m0 * L.n * ye, y_dtype);
            g.scratch = scr;
            int e = g.blk ? launch_gemm_blk(g, stream) : launch_gemm_q4k(g, stream);
            if (e) return hip_fail((hipError_t)e, "gemm launch");
        }
        return NNQ_OK;
    }
    // tokens per GEMV pass: Q4_K and Q6_K up to 4 (their decode kernels with four token
    // rows), Q8_0 up to 8 (its batched kernel)
    const int64_t mmax = L.fmt == NNQ_FMT_Q8_0 ? 8 : 4;
    const int64_t xrow = x_swiglu ? 2 * k : k;
    for (int64_t m0 = 0; m0 < m; m0 += mmax) {
        GemvArgs a{};
        a.qs = w->dev;
        a.hdr = w->dev + L.qs_bytes;
        a.x = (const uint8_t *)x + (size_t)m0 * xrow * xe;
        a.x_bf16 = x_dtype == NNQ_BF16;
        a.x_swiglu = x_swiglu;
        a.swiglu_out = swiglu_out;
        a.bias = bias;
        a.y = (uint8_t *)y + (size_t)m0 * L.n * ye;
        a.y_bf16 = y_dtype == NNQ_BF16;
        a.n = L.n;
        a.k = L.k;
        a.m = std::min(mmax, m - m0);
        a.ntile = L.ntile;
        a.nblk = L.nblk;
        if (status && (status_mode == 2 || m0 == 0)) {
            a.status = status;
            a.status_mode = status_mode;
        }
        int e = launch_gemv(L.fmt, a, stream);
        if (e) return hip_fail((hipError_t)e, "gemv launch");
    }
    return NNQ_OK;
}

extern "C" {

int nnq_linear(const nnq_weight *w, const void *x, nnq_dtype x_dtype, int64_t m, int64_t k, const float *bias,
               int64_t bias_len, void *y, nnq_dtype y_dtype, void *stream) {
    int rc = check_linear(w, x, x_dtype, m, k, bias, bias_len, y, y_dtype);
    if (rc) return rc;
    if (m == 0) return NNQ_OK;
    const bool xm = misaligned_in(x), ym = misaligned_out(y);
    if (!xm && !ym) return dispatch_linear(w, x, x_dtype, m, bias, y, y_dtype, stream);
    const hipStream_t st = (hipStream_t)stream;
    // workspace: [staged x][y computed here][the GEMM's scratch]
    size_t xbytes = 0, ybytes = 0, off[3], total = 0;
    if (!array_bytes(m, k, x_dtype == NNQ_BF16 ? 2 : 4, &xbytes) ||
        !array_bytes(m, w->L.n, y_dtype == NNQ_BF16 ? 2 : 4, &ybytes))
        return size_fail();
    const size_t lb = linear_scratch_bytes(w, m, x_dtype);
    const size_t sizes[3] = {xm ? xbytes : 0, ym ? ybytes : 0, lb};
    if (!plan_regions(sizes, 3, off, &total)) return size_fail();
    Scratch s;
    HIP_TRY(s.alloc(total, st), "scratch alloc");
    uint8_t *base = reinterpret_cast<uint8_t *>(s.p);
    if (xm) HIP_TRY(hipMemcpyAsync(base + off[0], x, xbytes, hipMemcpyDeviceToDevice, st), "stage x");
    rc = dispatch_linear(w, xm ? base + off[0] : x, x_dtype, m, bias, ym ? base + off[1] : y, y_dtype, stream, 0,
                         nullptr, 0, lb ? base + off[2] : nullptr);
    if (rc) return rc;
    if (ym) HIP_TRY(hipMemcpyAsync(y, base + off[1], ybytes, hipMemcpyDeviceToDevice, st), "copy y out");
    return NNQ_OK;
}

int nnq_argmax_f32(const float *logits, int64_t n, uint32_t *idx, int32_t *status_dev, void *stream) {
    if (!logits || !idx) return fail(NNQ_ERR_INVALID_ARGUMENT, "null pointer");
    if (n <= 0) return fail(NNQ_ERR_INVALID_SHAPE, "argmax over a zero-length dimension");
    if (n > 0xFFFFFFFFll) return fail(NNQ_ERR_INVALID_SHAPE, "argmax dim exceeds u32::MAX");
    Scratch s;
    const size_t bytes = 1024 * sizeof(unsigned long long);
    HIP_TRY(s.alloc(bytes, (hipStream_t)stream), "scratch alloc");
    int e = launch_argmax_reduce(logits, n, idx, status_dev, s.p, bytes, stream);
    if (e) return hip_fail((hipError_t)e, "argmax launch");
    return NNQ_OK;
}

int nnq_linear_argmax(const nnq_weight *w, const float *x, int64_t k, const float *bias, int64_t bias_len,
                      float *logits, uint32_t *idx, int32_t *status_dev, void *stream) {
    int rc = check_linear(w, x, NNQ_F32, 1, k, bias, bias_len, logits, NNQ_F32);
    if (rc) return rc;
    if (!idx) return fail(NNQ_ERR_INVALID_ARGUMENT, "idx is null");
    if (misaligned_out(logits)) return fail(NNQ_ERR_INVALID_ARGUMENT, "logits must be 4-byte aligned");
    const Layout &L = w->L;
    const bool xm = misaligned_in(x);
    // workspace: [per-tile argmax keys][staged x]
    const size_t sizes[2] = {(size_t)L.ntile * sizeof(unsigned long long), xm ? (size_t)k * 4 : 0};
    size_t off[2], total = 0;
    if (!plan_regions(sizes, 2, off, &total)) return size_fail();
    Scratch s;
    HIP_TRY(s.alloc(total, (hipStream_t)stream), "scratch alloc");
    if (xm) {
        HIP_TRY(hipMemcpyAsync(reinterpret_cast<uint8_t *>(s.p) + off[1], x, (size_t)k * 4, hipMemcpyDeviceToDevice,
                               (hipStream_t)stream),
                "stage x");
        x = reinterpret_cast<const float *>(reinterpret_cast<uint8_t *>(s.p) + off[1]);
    }
    GemvArgs a{};
    a.qs = w->dev;
    a.hdr = w->dev + L.qs_bytes;
    a.x = x;
    a.bias = bias;
    a.y = logits;
    a.n = L.n;
    a.k = L.k;
    a.m = 1;
    a.ntile = L.ntile;
    a.nblk = L.nblk;
    a.argmax_partial = (unsigned long long *)s.p;
    int64_t nkeys = L.ntile;  // the launch lowers it when it writes one key per workgroup
    a.argmax_count = &nkeys;
    int e = launch_gemv(L.fmt, a, stream);
    if (e) return hip_fail((hipError_t)e, "gemv launch");
    e = launch_argmax_final(a.argmax_partial, nkeys, idx, status_dev, stream);
    if (e) return hip_fail((hipError_t)e, "argmax launch");
    return NNQ_OK;
}

// ---- MoE ---------------------------------------------------------------------------

}  // extern "C"

// The expert shapes the kernels take: hidden and intermediate multiples of 32, at most
// 32768 (the expert kernels address a chunk's activation planes with 32-bit byte
// offsets), at most kMoeMaxExperts experts; checked before any allocation or copy.
static int moe_check_shape(int64_t E, int64_t H, int64_t I) {
    if (H % 32 || I % 32)
        return fail(NNQ_ERR_INVALID_SHAPE, "MoE hidden (%lld) and intermediate (%lld) sizes must be multiples of 32",
                    (long long)H, (long long)I);
    if (E > kMoeMaxExperts) return fail(NNQ_ERR_UNSUPPORTED, "at most %d experts", kMoeMaxExperts);
    if (H > 32768 || I > 32768) return fail(NNQ_ERR_UNSUPPORTED, "MoE hidden and intermediate sizes at most 32768");
    return 0;
}

// Upload of one layer's experts from GPT-OSS-ordered packed bytes and scale bytes
// (gptoss_scales: GPT-OSS E8M0 semantics, byte 0 = 2^-126; else nn-core OCP, 2^-127).
static int moe_create(int64_t E, int64_t H, int64_t I, const uint8_t *gu_packed, const uint8_t *gu_scales,
                      const float *gu_bias, const uint8_t *dn_packed, const uint8_t *dn_scales, const float *dn_bias,
                      bool gptoss_scales, nnq_moe **out) {
    if (!out) return fail(NNQ_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (E <= 0 || H <= 0 || I <= 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "bad MoE shape");
    if (!gu_packed || !gu_scales || !gu_bias || !dn_packed || !dn_scales || !dn_bias)
        return fail(NNQ_ERR_INVALID_ARGUMENT, "null weight pointer");
    if (int rc = moe_check_shape(E, H, I)) return rc;
    const size_t gu_el = (size_t)E * H * 2 * I, dn_el = (size_t)E * I * H;
    nnq_moe *m = new nnq_moe;
    hipGetDevice(&m->device);
    auto upload = [&](const void *src, size_t bytes, void **p) -> hipError_t {
        hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) return e;
        m->allocs.push_back(*p);
        return hipMemcpy(*p, src, bytes, hipMemcpyHostToDevice);
    };
    void *p[6] = {};
    std::vector<uint8_t> rq, rs;
    hipError_t e = hipSuccess;
    rq.resize(gu_el / 2);
    rs.resize(gu_el / 32);
    moe_repack(gu_packed, gu_scales, E, H, 2 * I, rq.data(), rs.data(), gptoss_scales);
    if ((e = upload(rq.data(), rq.size(), &p[0])) == hipSuccess) e = upload(rs.data(), rs.size(), &p[1]);
    if (e == hipSuccess) {
        rq.resize(dn_el / 2);
        rs.resize(dn_el / 32);
        moe_repack(dn_packed, dn_scales, E, I, H, rq.data(), rs.data(), gptoss_scales);
        if ((e = upload(rq.data(), rq.size(), &p[2])) == hipSuccess) e = upload(rs.data(), rs.size(), &p[3]);
    }
    if (e == hipSuccess) e = upload(gu_bias, (size_t)E * 2 * I * 4, &p[4]);
    if (e == hipSuccess) e = upload(dn_bias, (size_t)E * H * 4, &p[5]);
    if (e != hipSuccess) {
        for (void *q : m->allocs) hipFree(q);
        delete m;
        return hip_fail(e, "MoE upload");
    }
    m->d.E = E;
    m->d.H = H;
    m->d.I = I;
    m->d.gu_q = (const uint8_t *)p[0];
    m->d.gu_s = (const uint8_t *)p[1];
    m->d.dn_q = (const uint8_t *)p[2];
    m->d.dn_s = (const uint8_t *)p[3];
    m->d.gu_b = (const float *)p[4];
    m->d.dn_b = (const float *)p[5];
    *out = m;
    return NNQ_OK;
}

extern "C" {

int nnq_moe_create(int64_t E, int64_t H, int64_t I, const uint8_t *gu_packed, const uint8_t *gu_scales,
                   const float *gu_bias, const uint8_t *dn_packed, const uint8_t *dn_scales, const float *dn_bias,
                   nnq_moe **out) {
    return moe_create(E, H, I, gu_packed, gu_scales, gu_bias, dn_packed, dn_scales, dn_bias, true, out);
}

int nnq_moe_create_ocp(int64_t E, int64_t H, int64_t I, const uint8_t *gu_blocks, const float *gu_bias,
                       const uint8_t *dn_blocks, const float *dn_bias, nnq_moe **out) {
    if (!out) return fail(NNQ_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (E <= 0 || H <= 0 || I <= 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "bad MoE shape");
    if (!gu_blocks || !dn_blocks) return fail(NNQ_ERR_INVALID_ARGUMENT, "null weight pointer");
    if (int rc = moe_check_shape(E, H, I)) return rc;
    const size_t gnb = (size_t)E * H * 2 * I / 32, dnb = (size_t)E * I * H / 32;
    std::vector<uint8_t> gp(gnb * 16), gs(gnb), dp(dnb * 16), ds(dnb);
    ocp_split(gu_blocks, gnb, gp.data(), gs.data());
    ocp_split(dn_blocks, dnb, dp.data(), ds.data());
    return moe_create(E, H, I, gp.data(), gs.data(), gu_bias, dp.data(), ds.data(), dn_bias, false, out);
}

int nnq_dequant_mxfp4_ocp(const uint8_t *blocks, int64_t n, float *out, void *stream) {
    if (n < 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "n = %lld", (long long)n);
    if (n == 0) return NNQ_OK;
    if (!blocks || !out) return fail(NNQ_ERR_INVALID_ARGUMENT, "null pointer");
    int e = launch_ocp_dequant(blocks, n, out, stream);
    if (e) return hip_fail((hipError_t)e, "mxfp4 dequant launch");
    return NNQ_OK;
}

int nnq_moe_destroy(nnq_moe *m) {
    if (!m) return NNQ_OK;
    for (void *q : m->allocs) hipFree(q);
    delete m;
    return NNQ_OK;
}

int nnq_moe_forward(const nnq_moe *m, const void *x, nnq_dtype x_dtype, int64_t tokens, const float *router_logits,
                    int top_k, float swiglu_limit, float *y, uint32_t *topk_idx, float *topk_w, void *stream) {
    if (!m) return fail(NNQ_ERR_INVALID_ARGUMENT, "MoE handle is null");
    if (tokens < 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "tokens < 0");
    if (top_k <= 0 || top_k > m->d.E)
        return fail(NNQ_ERR_INVALID_SHAPE, "topk k=%d out of range for %lld experts", top_k, (long long)m->d.E);
    if (x_dtype != NNQ_F32 && x_dtype != NNQ_BF16) return fail(NNQ_ERR_UNSUPPORTED, "input dtype %d", (int)x_dtype);
    if (tokens == 0) return NNQ_OK;
    if (!x || !router_logits || !y) return fail(NNQ_ERR_INVALID_ARGUMENT, "null pointer");
    if (misaligned_out(y) || misaligned_out(router_logits))
        return fail(NNQ_ERR_INVALID_ARGUMENT, "y and router_logits must be 4-byte aligned");
    // tokens are routed independently, so a long batch runs as chunks of at most
    // kMoeChunkAssign token-expert assignments, one after another on the stream
    const int64_t tc = moe_chunk_tokens(tokens, top_k);
    const size_t xe = x_dtype == NNQ_BF16 ? 2 : 4;
    size_t xbytes = 0;
    if (!array_bytes(tokens, m->d.H, xe, &xbytes)) return size_fail();
    const bool xm = misaligned_in(x);
    // workspace: [the MoE launches' scratch][staged x]
    const size_t sizes[2] = {moe_scratch_bytes(tc, m->d.E, m->d.H, m->d.I, top_k, x_dtype == NNQ_BF16),
                             xm ? xbytes : 0};
    size_t off[2], total = 0;
    if (!plan_regions(sizes, 2, off, &total)) return size_fail();
    Scratch s;
    HIP_TRY(s.alloc(total, (hipStream_t)stream), "scratch alloc");
    if (xm) {
        HIP_TRY(hipMemcpyAsync(reinterpret_cast<uint8_t *>(s.p) + off[1], x, xbytes, hipMemcpyDeviceToDevice,
                               (hipStream_t)stream),
                "stage x");
        x = reinterpret_cast<uint8_t *>(s.p) + off[1];
    }
    for (int64_t t0 = 0; t0 < tokens; t0 += tc) {
        const int64_t n = std::min(tc, tokens - t0);
        int e = launch_moe(m->d, (const uint8_t *)x + (size_t)t0 * m->d.H * xe, x_dtype == NNQ_BF16, n,
                           router_logits + t0 * m->d.E, 1, nullptr, top_k, swiglu_limit, y + t0 * m->d.H,
                           topk_idx ? topk_idx + t0 * top_k : nullptr, topk_w ? topk_w + t0 * top_k : nullptr, nullptr,
                           s.p, stream);
        if (e) return hip_fail((hipError_t)e, "moe launch");
    }
    return NNQ_OK;
}

int nnq_moe_dequant_expert(const nnq_moe *m, int64_t expert, float *gate_up, float *down, void *stream) {
    if (!m) return fail(NNQ_ERR_INVALID_ARGUMENT, "MoE handle is null");
    if (expert < 0 || expert >= m->d.E) return fail(NNQ_ERR_INVALID_ARGUMENT, "expert %lld", (long long)expert);
    int e = launch_moe_dequant(m->d, expert, gate_up, down, stream);
    if (e) return hip_fail((hipError_t)e, "moe dequant launch");
    return NNQ_OK;
}

// ---- Qwen3 SwiGLU MLP -------------------------------------------------------------

int nnq_mlp_create(nnq_format gu_fmt, nnq_layout gu_layout, const uint8_t *gate, const uint8_t *up,
                   size_t gu_nbytes, nnq_format down_fmt, nnq_layout down_layout, const uint8_t *down,
                   size_t down_nbytes, int64_t hidden, int64_t inter, nnq_mlp **out) {
    if (!out) return fail(NNQ_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (!gate || !up || !down) return fail(NNQ_ERR_INVALID_ARGUMENT, "weight bytes are null");
    if (hidden <= 0 || inter <= 0)
        return fail(NNQ_ERR_INVALID_ARGUMENT, "MLP shape hidden=%lld inter=%lld", (long long)hidden, (long long)inter);
    // gate_proj and up_proj are W[inter, hidden]: stacked they are one W[2 * inter, hidden]
    // (block rows are independent), so a single GEMV computes both.  Q4_K with inter a
    // multiple of 8 stacks them 8 rows at a time (8 gate rows, the same 8 up rows, ...), so
    // every 16-row tile holds matching gate and up rows and the decode GEMV can write
    // silu(gate) * up directly.
    std::vector<uint8_t> cat(2 * gu_nbytes);
    const bool il8 = gu_fmt == NNQ_FMT_Q4_K && inter % 8 == 0 && gu_nbytes % (size_t)inter == 0;
    if (il8) {
        const size_t rb = gu_nbytes / (size_t)inter;  // bytes of one row (whole blocks)
        for (int64_t g8 = 0; g8 < inter / 8; g8++) {
            std::memcpy(cat.data() + (size_t)(16 * g8) * rb, gate + (size_t)(8 * g8) * rb, 8 * rb);
            std::memcpy(cat.data() + (size_t)(16 * g8 + 8) * rb, up + (size_t)(8 * g8) * rb, 8 * rb);
        }
    } else {
        std::memcpy(cat.data(), gate, gu_nbytes);
        std::memcpy(cat.data() + gu_nbytes, up, gu_nbytes);
    }
    nnq_weight *gu = nullptr, *dn = nullptr;
    int rc = nnq_weight_create(gu_fmt, gu_layout, cat.data(), cat.size(), 2 * inter, hidden, &gu);
    if (rc) return rc;
    rc = nnq_weight_create(down_fmt, down_layout, down, down_nbytes, hidden, inter, &dn);
    if (rc) {
        nnq_weight_destroy(gu);
        return rc;
    }
    nnq_mlp *p = new nnq_mlp;
    p->gu = gu;
    p->down = dn;
    p->hidden = hidden;
    p->inter = inter;
    p->interleaved8 = il8;
    *out = p;
    return NNQ_OK;
}

int nnq_mlp_destroy(nnq_mlp *p) {
    if (!p) return NNQ_OK;
    nnq_weight_destroy(p->gu);
    nnq_weight_destroy(p->down);
    delete p;
    return NNQ_OK;
}

}  // extern "C"

// the MLP's launches on prepared pointers (nnq_mlp_forward)
static int mlp_run(const nnq_mlp *p, const void *x, nnq_dtype x_dtype, int64_t m, void *y, nnq_dtype y_dtype,
                   int32_t *status_dev, void *stream, uint8_t *base, size_t gu_bytes, void *lin, bool fused,
                   bool hout) {
    const int64_t I = p->inter;
    int rc = 0;
    float *gu = reinterpret_cast<float *>(base);
    rc = dispatch_linear(p->gu, x, x_dtype, m, nullptr, gu, NNQ_F32, stream, 0, status_dev, fused ? 1 : 0, lin,
                         hout ? 1 : 0);
    if (rc) return rc;
    if (hout) return dispatch_linear(p->down, gu, NNQ_F32, m, nullptr, y, y_dtype, stream, 0, status_dev, 2);
    if (fused) return dispatch_linear(p->down, gu, NNQ_F32, m, nullptr, y, y_dtype, stream, 1, status_dev, 2);
    float *h = reinterpret_cast<float *>(base + gu_bytes);
    int e = launch_swiglu(gu, m, I, h, status_dev, stream, p->interleaved8 ? 1 : 0);
    if (e) return hip_fail((hipError_t)e, "swiglu launch");
    rc = dispatch_linear(p->down, h, NNQ_F32, m, nullptr, y, y_dtype, stream, 0, nullptr, 0, lin);
    if (rc) return rc;
    if (status_dev) {
        e = launch_nonfinite_check(y, y_dtype == NNQ_BF16, m * p->hidden, status_dev, stream);
        if (e) return hip_fail((hipError_t)e, "output check launch");
    }
    return NNQ_OK;
}

extern "C" {

int nnq_mlp_forward(const nnq_mlp *p, const void *x, nnq_dtype x_dtype, int64_t m, int64_t k, void *y,
                    nnq_dtype y_dtype, int32_t *status_dev, void *stream) {
    if (!p) return fail(NNQ_ERR_INVALID_ARGUMENT, "MLP handle is null");
    int rc = check_linear(p->gu, x, x_dtype, m, k, nullptr, 0, y, y_dtype);
    if (rc) return rc;
    if (m == 0) return NNQ_OK;
    const int64_t I = p->inter;
    // m <= 2: interleaved Q4_K gate | up -> the GEMV writes h = silu(gate) * up and the
    // down GEMV reads h; otherwise the down GEMV takes gate | up and applies SwiGLU while
    // staging.  m > 2: linear, swiglu_kernel, linear.
    const bool fused = m <= 2, hout = fused && p->interleaved8;
    // one workspace: gate | up [m, 2I] f32 (h [m, I] when hout), h [m, I] f32, the GEMM
    // scratch of either linear, then a misaligned x or y staged
    size_t gu_bytes = 0, h_bytes = 0, xbytes = 0, ybytes = 0;
    if (!array_bytes(m, (hout ? 1 : 2) * I, 4, &gu_bytes) || !array_bytes(m, fused ? 0 : I, 4, &h_bytes) ||
        !array_bytes(m, k, x_dtype == NNQ_BF16 ? 2 : 4, &xbytes) ||
        !array_bytes(m, p->hidden, y_dtype == NNQ_BF16 ? 2 : 4, &ybytes))
        return size_fail();
    const size_t lin_bytes =
        std::max(linear_scratch_bytes(p->gu, m, x_dtype), fused ? 0 : linear_scratch_bytes(p->down, m, NNQ_F32));
    const bool xm = misaligned_in(x), ym = misaligned_out(y);
    const size_t sizes[5] = {gu_bytes, h_bytes, lin_bytes, xm ? xbytes : 0, ym ? ybytes : 0};
    size_t off[5], total = 0;
    if (!plan_regions(sizes, 5, off, &total)) return size_fail();
    Scratch s;
    HIP_TRY(s.alloc(total, (hipStream_t)stream), "scratch alloc");
    uint8_t *base = reinterpret_cast<uint8_t *>(s.p);
    void *lin = lin_bytes ? base + off[2] : nullptr;
    void *const y_user = y;
    if (xm) {
        HIP_TRY(hipMemcpyAsync(base + off[3], x, xbytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "stage x");
        x = base + off[3];
    }
    if (ym) y = base + off[4];
    rc = mlp_run(p, x, x_dtype, m, y, y_dtype, status_dev, stream, base, off[1], lin, fused, hout);
    if (rc) return rc;
    if (ym) HIP_TRY(hipMemcpyAsync(y_user, y, ybytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "copy y out");
    return NNQ_OK;
}

// ---- GPT-OSS router and the whole MoE block ---------------------------------------

int nnq_router_create(int64_t num_experts, int64_t hidden, const float *weight, const float *bias, nnq_router **out) {
    if (!out) return fail(NNQ_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (!weight) return fail(NNQ_ERR_INVALID_ARGUMENT, "router weight is null");
    if (num_experts <= 0 || num_experts > kMoeMaxExperts)
        return fail(NNQ_ERR_INVALID_SHAPE, "router experts %lld (1..%d)", (long long)num_experts, kMoeMaxExperts);
    if (hidden <= 0 || hidden % 32)
        return fail(NNQ_ERR_INVALID_SHAPE, "router hidden %lld is not a positive multiple of 32", (long long)hidden);
    nnq_router *r = new nnq_router;
    r->E = num_experts;
    r->H = hidden;
    const size_t wb = (size_t)num_experts * hidden * 4;
    hipError_t e = hipMalloc(&r->w, wb);
    if (e == hipSuccess) e = hipMemcpy(r->w, weight, wb, hipMemcpyHostToDevice);
    if (e == hipSuccess && bias) {
        e = hipMalloc(&r->b, (size_t)num_experts * 4);
        if (e == hipSuccess) e = hipMemcpy(r->b, bias, (size_t)num_experts * 4, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        if (r->w) hipFree(r->w);
        if (r->b) hipFree(r->b);
        delete r;
        return hip_fail(e, "router upload");
    }
    *out = r;
    return NNQ_OK;
}

int nnq_router_destroy(nnq_router *r) {
    if (!r) return NNQ_OK;
    if (r->w) hipFree(r->w);
    if (r->b) hipFree(r->b);
    delete r;
    return NNQ_OK;
}

static int check_router_input(const nnq_router *r, const void *x, nnq_dtype x_dtype, int64_t tokens) {
    if (!r) return fail(NNQ_ERR_INVALID_ARGUMENT, "router handle is null");
    if (tokens < 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "tokens < 0");
    if (x_dtype != NNQ_F32 && x_dtype != NNQ_BF16) return fail(NNQ_ERR_UNSUPPORTED, "input dtype %d", (int)x_dtype);
    if (tokens > 0 && !x) return fail(NNQ_ERR_INVALID_ARGUMENT, "x is null");
    return NNQ_OK;
}

// a misaligned x of the router / MoE block copied to `dst` (the call's workspace)
static int stage_tokens(const void **x, size_t bytes, uint8_t *dst, void *stream) {
    HIP_TRY(hipMemcpyAsync(dst, *x, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "stage x");
    *x = dst;
    return NNQ_OK;
}

int nnq_router_logits(const nnq_router *r, const void *x, nnq_dtype x_dtype, int64_t tokens, float *logits,
                      void *stream) {
    int rc = check_router_input(r, x, x_dtype, tokens);
    if (rc) return rc;
    if (tokens == 0) return NNQ_OK;
    if (!logits) return fail(NNQ_ERR_INVALID_ARGUMENT, "logits is null");
    if (misaligned_out(logits)) return fail(NNQ_ERR_INVALID_ARGUMENT, "logits must be 4-byte aligned");
    const size_t pb = router_partial_bytes(tokens, r->H, (int)r->E);
    size_t xbytes = 0;
    if (!array_bytes(tokens, r->H, x_dtype == NNQ_BF16 ? 2 : 4, &xbytes)) return size_fail();
    const bool xm = misaligned_in(x);
    // workspace (when needed): [K-part slabs][staged x]
    const size_t sizes[2] = {pb, xm ? xbytes : 0};
    size_t off[2], total = 0;
    if (!plan_regions(sizes, 2, off, &total)) return size_fail();
    Scratch s;
    if (total) HIP_TRY(s.alloc(total, (hipStream_t)stream), "scratch alloc");
    if (xm && (rc = stage_tokens(&x, xbytes, reinterpret_cast<uint8_t *>(s.p) + off[1], stream))) return rc;
    int ks = 1;
    int e = launch_router_logits(x, x_dtype == NNQ_BF16, tokens, r->H, r->w, r->b, (int)r->E,
                                 pb ? reinterpret_cast<float *>(s.p) : logits, &ks, nullptr, stream);
    if (e) return hip_fail((hipError_t)e, "router launch");
    if (ks > 1) {
        e = launch_router_finalize(reinterpret_cast<float *>(s.p), ks, tokens, (int)r->E, r->b, logits, stream);
        if (e) return hip_fail((hipError_t)e, "router finalize launch");
    }
    return NNQ_OK;
}

int nnq_moe_block_forward(const nnq_moe *m, const nnq_router *r, const void *x, nnq_dtype x_dtype, int64_t tokens,
                          int top_k, float swiglu_limit, float *y, uint32_t *topk_idx, float *topk_w,
                          int32_t *status_dev, void *stream) {
    if (!m) return fail(NNQ_ERR_INVALID_ARGUMENT, "MoE handle is null");
    int rc = check_router_input(r, x, x_dtype, tokens);
    if (rc) return rc;
    if (r->E != m->d.E || r->H != m->d.H)
        return fail(NNQ_ERR_SHAPE_MISMATCH, "router [%lld, %lld] does not match the MoE's %lld experts x hidden %lld",
                    (long long)r->E, (long long)r->H, (long long)m->d.E, (long long)m->d.H);
    if (top_k <= 0 || top_k > m->d.E)
        return fail(NNQ_ERR_INVALID_SHAPE, "topk k=%d out of range for %lld experts", top_k, (long long)m->d.E);
    if (tokens == 0) return NNQ_OK;
    if (!y) return fail(NNQ_ERR_INVALID_ARGUMENT, "y is null");
    if (misaligned_out(y)) return fail(NNQ_ERR_INVALID_ARGUMENT, "y must be 4-byte aligned");
    // chunks of at most kMoeChunkAssign token-expert assignments (tokens are independent)
    const int64_t tc = moe_chunk_tokens(tokens, top_k);
    const size_t xe = x_dtype == NNQ_BF16 ? 2 : 4;
    size_t xbytes = 0;
    if (!array_bytes(tokens, m->d.H, xe, &xbytes)) return size_fail();
    const bool xm = misaligned_in(x);
    // workspace: [a chunk's router logits or K-part slabs][the MoE launches' scratch][staged x]
    const size_t sizes[3] = {std::max(router_partial_bytes(tc, r->H, (int)r->E), (size_t)tc * m->d.E * 4),
                             moe_scratch_bytes(tc, m->d.E, m->d.H, m->d.I, top_k, x_dtype == NNQ_BF16),
                             xm ? xbytes : 0};
    size_t off[3], total = 0;
    if (!plan_regions(sizes, 3, off, &total)) return size_fail();
    Scratch s;
    HIP_TRY(s.alloc(total, (hipStream_t)stream), "scratch alloc");
    if (xm && (rc = stage_tokens(&x, xbytes, reinterpret_cast<uint8_t *>(s.p) + off[2], stream))) return rc;
    float *logits = reinterpret_cast<float *>(s.p);
    for (int64_t t0 = 0; t0 < tokens; t0 += tc) {
        const int64_t n = std::min(tc, tokens - t0);
        const void *xc = (const uint8_t *)x + (size_t)t0 * m->d.H * xe;
        int ks = 1;
        // the router clears the status of the call, so only the first chunk passes it; every
        // chunk's combine flags a non-finite output
        int e = launch_router_logits(xc, x_dtype == NNQ_BF16, n, r->H, r->w, r->b, (int)r->E, logits, &ks,
                                     t0 == 0 ? status_dev : nullptr, stream);
        if (e) return hip_fail((hipError_t)e, "router launch");
        // the routing kernel sums the K-part slabs and adds the bias (with one part the
        // router kernel already did)
        e = launch_moe(m->d, xc, x_dtype == NNQ_BF16, n, logits, ks, ks > 1 ? r->b : nullptr, top_k, swiglu_limit,
                       y + t0 * m->d.H, topk_idx ? topk_idx + t0 * top_k : nullptr,
                       topk_w ? topk_w + t0 * top_k : nullptr, status_dev,
                       reinterpret_cast<uint8_t *>(s.p) + off[1], stream);
        if (e) return hip_fail((hipError_t)e, "moe launch");
    }
    return NNQ_OK;
}

// ---- token sampling ------------------------------------------------------------------

// the top-k a sampling call keeps (min(top_k, n); n for None), and whether the device
// path holds it
static int sample_k(const nnq_sampling *cfg, int64_t n, int64_t *k) {
    *k = cfg->top_k < 0 ? n : std::min<int64_t>(cfg->top_k, n);
    if (!sample_supported(n, *k))
        return fail(NNQ_ERR_UNSUPPORTED, "sampling over %lld logits: at most 2^32 - 1 (u32 token indices)",
                    (long long)n);
    return NNQ_OK;
}

// ext_scratch: scratch the caller provides (sample_scratch_bytes(n, k) bytes), or null to
// take the stream's workspace
static int run_sample(const float *logits, int64_t n, const uint32_t *past, int64_t n_past, const nnq_sampling *cfg,
                      uint32_t *token, void *stream, void *ext_scratch = nullptr) {
    int64_t k = 0;
    int rc = sample_k(cfg, n, &k);
    if (rc) return rc;
    Scratch s;
    if (ext_scratch)
        s.p = ext_scratch;
    else
        HIP_TRY(s.alloc(sample_scratch_bytes(n, k), (hipStream_t)stream), "scratch alloc");
    // sample_token's conditions for applying the penalties (sampling.rs:155-162)
    const int rep_on = std::fabs(cfg->repetition_penalty - 1.0f) > 1.1920929e-7f;
    const int freq_on = std::fabs(cfg->frequency_penalty) > 1.1920929e-7f;
    int e = launch_sample(logits, n, past, n_past, cfg->temperature, k, cfg->top_k < 0, cfg->use_top_p != 0, cfg->top_p,
                          cfg->repetition_penalty, rep_on, cfg->frequency_penalty, freq_on, cfg->seed, token, s.p,
                          stream);
    if (e) return hip_fail((hipError_t)e, "sample launch");
    return NNQ_OK;
}

static int check_sampling(const nnq_sampling *cfg, const uint32_t *past, int64_t n_past, const uint32_t *token) {
    if (!cfg || !token) return fail(NNQ_ERR_INVALID_ARGUMENT, "sampling config or token is null");
    if (!(cfg->temperature > 0.0f) || !std::isfinite(cfg->temperature))
        return fail(NNQ_ERR_INVALID_ARGUMENT, "temperature must be positive and finite");
    if (n_past < 0 || (n_past > 0 && !past)) return fail(NNQ_ERR_INVALID_ARGUMENT, "past tokens");
    return NNQ_OK;
}

int nnq_sample_token(const float *logits, int64_t n, const uint32_t *past_tokens, int64_t n_past,
                     const nnq_sampling *cfg, uint32_t *token, void *stream) {
    if (!logits || n <= 0) return fail(NNQ_ERR_INVALID_ARGUMENT, "logits must be non-empty");
    int rc = check_sampling(cfg, past_tokens, n_past, token);
    if (rc) return rc;
    return run_sample(logits, n, past_tokens, n_past, cfg, token, stream);
}

int nnq_linear_sample(const nnq_weight *w, const float *x, int64_t k, const float *bias, int64_t bias_len,
                      float *logits, const uint32_t *past_tokens, int64_t n_past, const nnq_sampling *cfg,
                      uint32_t *token, void *stream) {
    int rc = check_linear(w, x, NNQ_F32, 1, k, bias, bias_len, logits, NNQ_F32);
    if (rc) return rc;
    rc = check_sampling(cfg, past_tokens, n_past, token);
    if (rc) return rc;
    if (misaligned_out(logits)) return fail(NNQ_ERR_INVALID_ARGUMENT, "logits must be 4-byte aligned");
    Scratch xs;  // a misaligned x: staged in the workspace, read by the GEMV before the sampling reuses it
    if (misaligned_in(x)) {
        HIP_TRY(xs.alloc((size_t)k * 4, (hipStream_t)stream), "scratch alloc");
        HIP_TRY(hipMemcpyAsync(xs.p, x, (size_t)k * 4, hipMemcpyDeviceToDevice, (hipStream_t)stream), "stage x");
        x = reinterpret_cast<const float *>(xs.p);
    }
    rc = dispatch_linear(w, x, NNQ_F32, 1, bias, logits, NNQ_F32, stream);
    if (rc) return rc;
    return run_sample(logits, w->L.n, past_tokens, n_past, cfg, token, stream);
}

int nnq_linear_sample_noalloc(const nnq_weight *w, const float *x, int64_t k, const float *bias, int64_t bias_len,
                              float *logits, const uint32_t *past_tokens, int64_t n_past, const nnq_sampling *cfg,
                              uint32_t *token, void *stream) {
    int rc = check_linear(w, x, NNQ_F32, 1, k, bias, bias_len, logits, NNQ_F32);
    if (rc) return rc;
    rc = check_sampling(cfg, past_tokens, n_past, token);
    if (rc) return rc;
    if (misaligned_in(x) || misaligned_out(logits))
        return fail(NNQ_ERR_INVALID_ARGUMENT,
                    "x must be 16-byte and logits 4-byte aligned (this entry point has no workspace to stage them)");
    int64_t kk = 0;
    rc = sample_k(cfg, w->L.n, &kk);
    if (rc) return rc;
    const size_t need = sample_scratch_bytes(w->L.n, kk);
    if (!sample_two_pass(w->L.n, kk) || need > kSampleStaticScratchBytes)
        return fail(NNQ_ERR_UNSUPPORTED,
                    "top_k %lld over %lld logits exceeds the allocation-free top-k capacity (ceil(n / 2048) * "
                    "min(k, 2048) <= 16384 candidates in %zu bytes of fixed scratch)",
                    (long long)kk, (long long)w->L.n, kSampleStaticScratchBytes);
    void *scr = nullptr;
    HIP_TRY((hipError_t)sample_static_scratch(&scr), "fixed scratch address");
    // the single-token GEMV takes no scratch; the sampling kernels write every scratch
    // byte they read, so nothing needs clearing
    rc = dispatch_linear(w, x, NNQ_F32, 1, bias, logits, NNQ_F32, stream);
    if (rc) return rc;
    return run_sample(logits, w->L.n, past_tokens, n_past, cfg, token, stream, scr);
}

}  // extern "C"
