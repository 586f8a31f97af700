// Prefill GEMM for Q4_K weights at 3 .. 16 bf16 token rows on gfx950, in one launch:
// Y[m, n] = X[m, k] . W[n, k]^T (+ bias), the arithmetic of QLinear::forward with a few
// tokens (crates/nn-core/src/layers/quantized/linear.rs:366-400; the bf16 result dtype of
// crates/nn-core/src/dyn_tensor/ops/matmul.rs:37-38).
//
// At this size the weight is read once and the product is HBM-bound, so the kernel has
// no staging launch and reads no derived weight data: the activation enters the bf16
// MFMA as it is in memory, and the weight's codes as exact bf16 integers.
//
// Arithmetic per 32-k sub-block j of a column n (w = d*sc_j*q - dmin*m_j):
//  * B' = 128 + q as bf16 (0x4300 | q: exponent 2^7, the code in the low mantissa bits,
//    exact), so P' = sum(x * (128 + q)) = sum(x * q) + 128 * S with S = sum(x) over the
//    sub-block; S comes from one more MFMA against ones, shared by every column tile;
//  * y += d*sc_j * P' - (128*d*sc_j + dmin*m_j) * S = d*sc_j * sum(x*q) - dmin*m_j * S.
// Every product is exact in f32 (8-bit by 8-bit significands); the sums round in f32.  A
// NaN or infinity in a token's x makes that token's outputs NaN (inf - inf in the second
// line), as the other GEMM paths do.
//
// Organisation: one workgroup per R consecutive 16-column weight tiles; its W waves split
// K by super-blocks (unit u to wave u % W).  A wave loads a unit's A fragments (MT row
// tiles x 8 steps, 16 bytes per lane straight from x: lane 16G + r takes row r's
// elements 8G .. 8G + 7 of the step) and the R tiles' raw tile16 codes and headers, the
// next unit's loads issued before the current unit's math so the loads of one unit are
// in flight while the previous one computes.  Rows past M read as zeros (buffer offsets
// past the range).  The waves' totals meet in LDS at the end.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

struct ThinArgs {
    const uint8_t *qs;   // tile16 code plane
    const uint8_t *hdr;  // super-block headers (d, dmin, scales[12]) per (tile, block, row)
    const uint16_t *x;   // bf16 [m][k]
    const float *bias;
    void *y;
    int y_bf16;
    int m, nblk, ntile;
    int64_t k, n;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t thin_rsrc(const void *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)min(bytes, (int64_t)0x7FFFFFF0), 0x00020000);
}
__device__ __forceinline__ u32x4 thin_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, soff, 0));
}
// the weight stream: non-temporal (aux 2), so it does not push the activation out of L2
__device__ __forceinline__ u32x2 thin_load2_nt(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 2));
}
__device__ __forceinline__ u32x4 thin_load4_nt(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2));
}

// bf16 pair (128 + q0, 128 + q1) of the codes in bits 0..3 and 16..19 of v
__device__ __forceinline__ uint32_t thin_code2(uint32_t v) { return (v & 0x000F000Fu) | 0x43004300u; }

// ONE: K has at most W units (one per wave), so a wave holds one unit's loads only
template <int R, int MT, int W, bool ONE>
__global__ __launch_bounds__(W * 64) void gemm_q4k_thin_kernel(ThinArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = lane >> 4, c16 = lane & 15;
    const int nblk = a.nblk;
    const int t0 = (int)blockIdx.x * R;  // the plan keeps ntile % R == 0

    // activation: row 16 mt + c16, elements 8G .. 8G + 7 of each 32-k step; rows past M
    // take an offset past the range (zeros)
    const __amdgpu_buffer_rsrc_t rx = thin_rsrc(a.x, (int64_t)a.m * a.k * 2);
    uint32_t xoff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int row = 16 * mt + c16;
        xoff[mt] = row < a.m ? (uint32_t)(((int64_t)row * a.k + 8 * G) * 2) : 0x80000000u;
    }
    const __amdgpu_buffer_rsrc_t rq = thin_rsrc(a.qs + (size_t)t0 * nblk * 2048, (int64_t)R * nblk * 2048);
    const __amdgpu_buffer_rsrc_t rh = thin_rsrc(a.hdr + (size_t)t0 * nblk * 256, (int64_t)R * nblk * 256);
    // consumer lane (G, c) of group p takes bytes 8G .. 8G + 7 of row c's group: plane
    // G >> 1, chunk 16 p + c, half G & 1 (low nibbles: sub-block 2p, high: 2p + 1)
    const int qoff = (G >> 1) * 1024 + c16 * 16 + 8 * (G & 1), hoff = c16 * 16;

    struct Raw {
        u32x4 x[MT][8];
        u32x2 q[R][4];
        u32x4 h[R];
    };
    // issue order = use order (loads retire in order): the headers, then per pair of steps
    // their A fragments and the tiles' codes, so a step waits only for its own loads
    auto load = [&](int u, Raw &w) {
#pragma unroll
        for (int r = 0; r < R; r++) w.h[r] = thin_load4_nt(rh, hoff, (r * nblk + u) * 256);
#pragma unroll
        for (int p = 0; p < 4; p++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int s = 2 * p; s < 2 * p + 2; s++) w.x[mt][s] = thin_load4(rx, xoff[mt], (u * 256 + 32 * s) * 2);
#pragma unroll
            for (int r = 0; r < R; r++) w.q[r][p] = thin_load2_nt(rq, qoff + 256 * p, (r * nblk + u) * 2048);
        }
    };

    floatx4 tot[R][MT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) tot[r][mt] = floatx4{0.f, 0.f, 0.f, 0.f};

    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
    auto unit = [&](const Raw &w) {
        // per tile: d * 2^0, -128 d, -dmin and the sub-blocks' 6-bit scales and mins
        // (get_scale_min_k4, crates/nn-core/src/layers/quantized/linear.rs:166-176)
        float d[R], d128n[R], dminn[R];
        uint32_t sc[R][2], mn[R][2];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const u32x4 h = w.h[r];
            d[r] = f16_to_f32(h[0] & 0xFFFFu);
            d128n[r] = -128.0f * d[r];
            dminn[r] = -f16_to_f32(h[0] >> 16);
            sc[r][0] = h[1] & 0x3F3F3F3Fu;
            sc[r][1] = (h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u);
            mn[r][0] = h[2] & 0x3F3F3F3Fu;
            mn[r][1] = ((h[3] >> 4) & 0x0F0F0F0Fu) | ((h[2] >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int p = s >> 1;
            floatx4 S[MT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) S[mt] = mfma16x16x32_bf16(w.x[mt][s], ones, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t w0 = w.q[r][p][0], w1 = w.q[r][p][1];
                const int sh = (s & 1) * 4;  // low nibbles: sub-block 2p; high: 2p + 1
                const u32x4 b = {thin_code2(w0 >> sh), thin_code2(w0 >> (8 + sh)), thin_code2(w1 >> sh),
                                 thin_code2(w1 >> (8 + sh))};
                const float scf = (float)((sc[r][s >> 2] >> (8 * (s & 3))) & 0xFFu);
                const float mf = (float)((mn[r][s >> 2] >> (8 * (s & 3))) & 0xFFu);
                const float dsc = d[r] * scf;
                const float nc = __builtin_fmaf(d128n[r], scf, dminn[r] * mf);  // -(128 d sc + dmin m)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const floatx4 P = mfma16x16x32_bf16(w.x[mt][s], b, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        tot[r][mt][e] = __builtin_fmaf(nc, S[mt][e], __builtin_fmaf(dsc, P[e], tot[r][mt][e]));
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // one step's MFMA results live at a time
        }
    };

    // this wave's units wv, wv + W, ...: the next unit's loads go out before this one's math
    const int nu = nblk > wv ? (nblk - wv + W - 1) / W : 0;
    if constexpr (ONE) {
        Raw w1;
        if (nu > 0) {
            load(wv, w1);
            __builtin_amdgcn_sched_barrier(0);
            unit(w1);
        }
    } else {
    Raw buf[2];
    if (nu > 0) load(wv, buf[0]);
    for (int i = 0; i < nu; i += 2) {
        if (i + 1 < nu) load(wv + (i + 1) * W, buf[1]);
        __builtin_amdgcn_sched_barrier(0);
        unit(buf[0]);
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 >= nu) break;
        if (i + 2 < nu) load(wv + (i + 2) * W, buf[0]);
        __builtin_amdgcn_sched_barrier(0);
        unit(buf[1]);
        __builtin_amdgcn_sched_barrier(0);
    }
    }

    // the waves' totals meet in LDS: [wave][tile][row tile][row][column] f32
    float *red = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++) red[(((wv * R + r) * MT + mt) * 16 + 4 * G + e) * 16 + c16] = tot[r][mt][e];
    __syncthreads();
    for (int o = tid; o < R * MT * 256; o += W * 64) {
        const int col16 = o & 15, row = (o >> 4) % (16 * MT), r = o / (256 * MT);
        if (row >= a.m) continue;
        float y = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < W; w2++) y += red[(((w2 * R + r) * MT + (row >> 4)) * 16 + (row & 15)) * 16 + col16];
        const int64_t col = (int64_t)(t0 + r) * 16 + col16;
        if (col >= a.n) continue;
        if (a.bias) y += a.bias[col];
        if (a.y_bf16)
            reinterpret_cast<uint16_t *>(a.y)[(int64_t)row * a.n + col] = (uint16_t)f32_to_bf16_bits(y);
        else
            reinterpret_cast<float *>(a.y)[(int64_t)row * a.n + col] = y;
    }
}

template <int R, int MT, int W, bool ONE>
int launch_thin_cfg(const ThinArgs &t, hipStream_t st) {
    constexpr int LDS = W * R * MT * 1024;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_thin_kernel<R, MT, W, ONE>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    hipLaunchKernelGGL((gemm_q4k_thin_kernel<R, MT, W, ONE>), dim3((unsigned)(t.ntile / R)), dim3(W * 64), LDS, st,
                       t);
    return (int)hipGetLastError();
}

}  // namespace

// The thin kernel's shape rules: Q4_K, bf16 activations, 3 to 16 rows.  R = 3 tiles per
// workgroup when that gives at least 192 workgroups, else 1 (two tiles on 128 workgroups
// measured slower: every workgroup reads the whole activation, but half the CUs stream
// the weight).  Sixteen waves, except three tiles over more than 16 units (eight: the
// double-buffered loads of three tiles take 199 registers).  Returns 1 when it takes the
// shape (and R, W: tiles per workgroup and waves).
int gemm_thin_plan(const GemmArgs &a, int *R, int *W) {
    // (32-bit buffer offsets: the activation's m * k * 2 bytes and three tiles' codes,
    // 3 * nblk * 2048 bytes, stay below 2^31)
    if (a.blk || !a.x_bf16 || a.m <= 2 || a.m > 16 || a.k % 256 || (int64_t)a.m * a.k > (int64_t)1 << 29 ||
        a.nblk > 65536)
        return 0;
    const int r = (a.ntile % 3 == 0 && a.ntile / 3 >= 192) ? 3 : 1;
    if (R) *R = r;
    if (W) *W = (r == 3 && a.nblk > 16) ? 8 : 16;
    return 1;
}

int launch_gemm_thin(const GemmArgs &a, void *stream) {
    int R = 0, W = 0;
    if (!gemm_thin_plan(a, &R, &W)) return (int)hipErrorInvalidValue;
    ThinArgs t;
    t.qs = a.qs;
    t.hdr = a.hdr;
    t.x = reinterpret_cast<const uint16_t *>(a.x);
    t.bias = a.bias;
    t.y = a.y;
    t.y_bf16 = a.y_bf16;
    t.m = (int)a.m;
    t.nblk = (int)a.nblk;
    t.ntile = (int)a.ntile;
    t.k = a.k;
    t.n = a.n;
    hipStream_t st = (hipStream_t)stream;
    const bool one = a.nblk <= W;
    if (R == 3) return one ? launch_thin_cfg<3, 1, 16, true>(t, st) : launch_thin_cfg<3, 1, 8, false>(t, st);
    return one ? launch_thin_cfg<1, 1, 16, true>(t, st) : launch_thin_cfg<1, 1, 16, false>(t, st);
}

}  // namespace nnq
