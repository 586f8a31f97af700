// GPT-OSS MXFP4 mixture-of-experts layer on gfx950 (QuantizedDecoderLayer::moe_forward /
// expert_forward, crates/nn-gptoss/src/quantized_model.rs:99-194).
//
// Pipeline (all on the device, no host synchronisation):
//   route    softmax over the router logits, first-index top-k by total order,
//            renormalisation (crates/nn-core/src/dyn_tensor/ops_ext/sorting.rs:22-104)
//   permute  per-expert counts, offsets and a stable (token, slot) order of the
//            assignments: expert e's rows are its tokens in ascending order, as the
//            host grouping of moe_forward (:157-169) builds them
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
// E8M0 byte 0 means 2^-126 in Mxfp4Tensor::decode (crates/nn-gptoss/src/quantize.rs:84-90)
// but 2^-127 here; such blocks hold values below 1e-37.
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
// routing: one wave per token, lane c holds logits c, c + 64, ... (E <= 256)
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float *logits, int64_t T, int E, int k, uint32_t *ti,
                                                        float *tw, uint32_t *ti_out, float *tw_out) {
    __shared__ float ex[4][256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + wv;
    if (t >= T) return;  // wave-uniform; no barrier below
    const float *x = logits + t * E;
    float v[4];
    float mx = -INFINITY;
    int ninf = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = lane + 64 * j;
        v[j] = c < E ? x[c] : -INFINITY;
        mx = fmaxf(mx, v[j]);
        ninf += (c < E && v[j] == INFINITY);
    }
    mx = wave_max(mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ninf += __shfl_xor(ninf, o, 64);
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
        float sum = -0.0f;
        for (int c = 0; c < E; c++) sum = sum + ex[wv][c];
#pragma unroll
        for (int j = 0; j < 4; j++) p[j] = p[j] / sum;
    }
    // top-k: descending by total order, ties to the lowest index (key = orderable value, ~index)
    uint32_t idx[8];
    float val[8];
    bool taken[4] = {false, false, false, false};
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
        pv = __shfl(pv, (int)(c & 63), 64);
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

// One workgroup of 1024 threads, one token per thread per chunk of 1024 tokens.  For
// each expert a ballot gives every token its rank among the wave's tokens that chose
// the expert; per-wave counts in LDS turn that into the rank over all earlier tokens.
// Expert e's rows are then its tokens in ascending order (stable by token, the order
// moe_forward's grouping loop builds, crates/nn-gptoss/src/quantized_model.rs:157-169).
template <int k>
__global__ __launch_bounds__(1024) void moe_permute_kernel(const uint32_t *ti, int64_t T, int E, int32_t *off,
                                                           int32_t *stok, int32_t *pos) {
    __shared__ int32_t wcnt[16][256];
    __shared__ int32_t base[256];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int e = tid; e < E; e += 1024) base[e] = 0;
    __syncthreads();
    for (int64_t t0 = 0; t0 < T; t0 += 1024) {
        const int64_t t = t0 + tid;
        uint32_t ex[k];
        int32_t rk[k];
#pragma unroll
        for (int s = 0; s < k; s++) {
            ex[s] = t < T ? ti[t * k + s] : 0xFFFFFFFFu;
            rk[s] = 0;
        }
        for (int e = 0; e < E; e++) {
            bool hit = false;
#pragma unroll
            for (int s = 0; s < k; s++) hit |= ex[s] == (uint32_t)e;
            const uint64_t m = __ballot(hit);
            const int32_t r = __popcll(m & lt);
#pragma unroll
            for (int s = 0; s < k; s++)
                if (ex[s] == (uint32_t)e) rk[s] = r;
            if (lane == 0) wcnt[wv][e] = __popcll(m);
        }
        __syncthreads();
        if (t < T)
#pragma unroll
            for (int s = 0; s < k; s++) {
                const uint32_t e = ex[s];
                int32_t r = base[e] + rk[s];
                for (int w = 0; w < wv; w++) r += wcnt[w][e];
                pos[t * k + s] = r;  // rank within the expert; the offset is added below
            }
        __syncthreads();
        for (int e = tid; e < E; e += 1024) {
            int32_t c = 0;
            for (int w = 0; w < 16; w++) c += wcnt[w][e];
            base[e] += c;
        }
        __syncthreads();
    }
    if (tid == 0) {
        int32_t acc = 0;
        for (int e = 0; e < E; e++) {
            const int32_t c = base[e];
            base[e] = acc;
            off[e] = acc;
            acc += c;
        }
        off[E] = acc;
    }
    __syncthreads();
    for (int64_t i = tid; i < T * k; i += 1024) {
        const int32_t p = pos[i] + base[ti[i]];
        pos[i] = p;
        stok[p] = (int32_t)(i / k);
    }
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
};

constexpr int kMoeRows = 64;  // token rows per pass (4 MFMA row tiles)
constexpr int kMoeKbc = 8;    // 32-row blocks of K staged in LDS per chunk
constexpr int kMoeAst = kMoeKbc * 32 + 8;  // LDS row stride of a staged activation chunk (bf16)

__host__ __device__ constexpr size_t moe_lds_bytes(int nw, int P, bool gu) {
    return (size_t)P * kMoeRows * kMoeAst * 2 > (gu ? (size_t)(nw / 2) * kMoeRows * 33 * 4 : 0)
               ? (size_t)P * kMoeRows * kMoeAst * 2
               : (size_t)(nw / 2) * kMoeRows * 33 * 4;
}

// Workgroup = (expert, NW column blocks): for gate_up (GU) waves 0 .. NW/2 - 1 own gate
// blocks and waves NW/2 .. NW - 1 the matching up blocks; for down wave w owns block w
// of its group.  Per chunk of 8 K-blocks the workgroup stages the expert's token rows
// (P bf16 planes) in LDS once; every wave then streams its own weight block and reuses
// the staged rows.  The activation loads are issued before the weight loads, so the
// wait before the LDS store does not cover the weights.
template <int NW, int P, bool GU>
__global__ __launch_bounds__(NW * 64) void moe_expert_kernel(MoeDev d, MoeScratch sc, MoeRun run) {
    constexpr int NTH = NW * 64;
    constexpr int APIECE = P * kMoeRows * kMoeKbc * 4;  // 16-byte activation pieces per chunk
    constexpr int APT = (APIECE + NTH - 1) / NTH;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint16_t *As = reinterpret_cast<uint16_t *>(smem);  // [P][kMoeRows][kMoeAst]
    float *gbuf = reinterpret_cast<float *>(smem);      // gate_up epilogue: [NW/2][kMoeRows][33]

    const int64_t H = d.H, I = d.I;
    const int64_t K = GU ? H : I, KB = K / 32;
    const int64_t NB = GU ? 2 * I / 32 : H / 32;
    const int64_t ngrp = GU ? (I / 32) / (NW / 2) : (NB + NW - 1) / NW;
    const int64_t e = blockIdx.x / ngrp, grp = blockIdx.x % ngrp;
    const int32_t r0 = sc.off[e], ne = sc.off[e + 1] - r0;
    if (ne == 0) return;  // workgroup-uniform
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int p = lane >> 4, l16 = lane & 15;
    int64_t nb, col0;
    int half = 0;
    if (GU) {
        half = wv / (NW / 2);
        const int64_t cb = grp * (NW / 2) + wv % (NW / 2);
        col0 = cb * 32;  // gate column of this wave's block
        nb = half * (I / 32) + cb;
    } else {
        nb = grp * NW + wv;
        col0 = nb * 32;
    }
    const bool active = nb < NB;  // tail waves of the last down group join the barriers only
    const int64_t nbs = active ? nb : 0;
    const uint8_t *cq = (GU ? d.gu_q : d.dn_q) + (e * NB + nbs) * KB * 512;
    const uint8_t *cs = (GU ? d.gu_s : d.dn_s) + (e * NB + nbs) * KB * 32;

    for (int32_t m0 = 0; m0 < ne; m0 += kMoeRows) {
        const int mtn = (ne - m0) >= kMoeRows ? 4 : (ne - m0 + 15) / 16;  // live row tiles
        floatx4 acc[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) acc[mt][0] = acc[mt][1] = zero4();
        for (int64_t kb0 = 0; kb0 < KB; kb0 += kMoeKbc) {
            const int kbc = (KB - kb0) < kMoeKbc ? (int)(KB - kb0) : kMoeKbc;
            // activation pieces of this chunk (zeros past the expert's rows / the chunk)
            u32x4 ra[APT];
#pragma unroll
            for (int i = 0; i < APT; i++) {
                const int c = tid + i * NTH;
                ra[i] = u32x4{0u, 0u, 0u, 0u};
                if (c < APIECE) {
                    const int pl = c / (kMoeRows * kMoeKbc * 4), rem = c % (kMoeRows * kMoeKbc * 4);
                    const int row = rem / (kMoeKbc * 4), c16 = rem % (kMoeKbc * 4);
                    if (m0 + row < ne && c16 < 4 * kbc) {
                        const int64_t kk = kb0 * 32 + c16 * 8;
                        const uint16_t *src =
                            GU ? run.xa[pl] + (int64_t)sc.stok[r0 + m0 + row] * H + kk
                               : sc.hb + (int64_t)pl * run.A * I + (int64_t)(r0 + m0 + row) * I + kk;
                        ra[i] = *reinterpret_cast<const u32x4 *>(src);
                    }
                }
            }
            // this wave's weight block for the chunk
            u32x2 bcq[kMoeKbc], bcs[kMoeKbc];
#pragma unroll
            for (int j = 0; j < kMoeKbc; j++) {
                bcq[j] = bcs[j] = u32x2{0u, 0u};
                if (active && j < kbc) {
                    bcq[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(cq + (kb0 + j) * 512 + 8 * lane));
                    bcs[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(cs + (kb0 + j) * 32 + 8 * p));
                }
            }
            __syncthreads();  // the previous chunk's rows have been read
#pragma unroll
            for (int i = 0; i < APT; i++) {
                const int c = tid + i * NTH;
                if (c < APIECE) {
                    const int pl = c / (kMoeRows * kMoeKbc * 4), rem = c % (kMoeRows * kMoeKbc * 4);
                    const int row = rem / (kMoeKbc * 4), c16 = rem % (kMoeKbc * 4);
                    *reinterpret_cast<u32x4 *>(As + (pl * kMoeRows + row) * kMoeAst + c16 * 8) = ra[i];
                }
            }
            __syncthreads();
            if (active) {
#pragma unroll
                for (int j = 0; j < kMoeKbc; j++) {
                    if (j >= kbc) break;
                    uint32_t r[8];
                    fp4_rows(bcq[j], bcs[j], r);
                    u32x4 be, bo;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        bo[q] = __builtin_amdgcn_perm(r[2 * q + 1], r[2 * q], 0x05040100u);  // column 2c + 1
                        be[q] = __builtin_amdgcn_perm(r[2 * q + 1], r[2 * q], 0x07060302u);  // column 2c
                    }
#pragma unroll
                    for (int mt = 0; mt < 4; mt++) {
                        if (mt >= mtn) break;  // wave-uniform
#pragma unroll
                        for (int pl = 0; pl < P; pl++) {
                            const u32x4 a = *reinterpret_cast<const u32x4 *>(
                                As + (pl * kMoeRows + mt * 16 + l16) * kMoeAst + j * 32 + 8 * p);
                            acc[mt][0] = mfma16x16x32_bf16(a, be, acc[mt][0]);
                            acc[mt][1] = mfma16x16x32_bf16(a, bo, acc[mt][1]);
                        }
                    }
                }
            }
        }
        // lane holds rows 4p + i of each tile; tile 0 = columns 2 * l16, tile 1 = 2 * l16 + 1
        if (GU) {
            __syncthreads();  // the staged rows are dead; gbuf reuses their LDS
            if (half == 0) {
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int o = 0; o < 2; o++) {
                            const int c = 2 * l16 + o;
                            gbuf[((wv % (NW / 2)) * kMoeRows + mt * 16 + 4 * p + i) * 33 + c] =
                                acc[mt][o][i] + d.gu_b[e * 2 * I + col0 + c];
                        }
            }
            __syncthreads();
            if (half == 1) {
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int32_t r = m0 + mt * 16 + 4 * p + i;
                        if (r >= ne) continue;
#pragma unroll
                        for (int o = 0; o < 2; o++) {
                            const int c = 2 * l16 + o;
                            const float g = gbuf[((wv % (NW / 2)) * kMoeRows + mt * 16 + 4 * p + i) * 33 + c];
                            const float u = acc[mt][o][i] + d.gu_b[e * 2 * I + I + col0 + c];
                            // silu (crates/nn-core/src/dyn_tensor/ops/math.rs:140), clamped to +-limit
                            float sg = g / (1.0f + expf(-g));
                            sg = sg < -run.limit ? -run.limit : (sg > run.limit ? run.limit : sg);
                            const float h = sg * u;
                            const uint16_t hh = bf16_rne(h);
                            const int64_t o2 = (int64_t)(r0 + r) * I + col0 + c;
                            sc.hb[o2] = hh;
                            sc.hb[run.A * I + o2] = bf16_rne(h - bf16_to_f32(hh));
                        }
                    }
            }
        } else if (active) {
#pragma unroll
            for (int mt = 0; mt < 4; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int32_t r = m0 + mt * 16 + 4 * p + i;
                    if (r >= ne) continue;
#pragma unroll
                    for (int o = 0; o < 2; o++) {
                        const int64_t col = col0 + 2 * l16 + o;
                        sc.yb[(int64_t)(r0 + r) * H + col] = acc[mt][o][i] + d.dn_b[e * H + col];
                    }
                }
        }
        __syncthreads();  // LDS is restaged by the next row pass
    }
}

// y[t] = ((0 + w_a * y_a) + w_b * y_b) + ... over the token's experts a < b < ...
template <int k>
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeScratch sc, int64_t H, float *y) {
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
    for (int64_t c = threadIdx.x; c < H; c += 256) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < k; s++) acc = acc + sc.yb[(int64_t)ps[s] * H + c] * ws[s];
        y[t * H + c] = acc;
    }
}

// ---------------------------------------------------------------------------------
// bit-exact decode of one expert (Mxfp4Tensor::dequantize, crates/nn-gptoss/src/quantize.rs:167-188)
// ---------------------------------------------------------------------------------
__constant__ float kFp4Lut[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// FP4_LUT[code] * 2^(E - 127) (E = 1 for scale byte 0) as f32 bits, built with integer
// arithmetic so that subnormal results are exact whatever the f32 denormal mode.
__device__ __forceinline__ float fp4_decode(uint32_t code, uint32_t sbyte) {
    const uint32_t mag = code & 7u, sign = (code & 8u) << 28;
    if (mag == 0 || sbyte == 255) {  // zeros, and the inf scale (x * inf, 0 * inf = NaN)
        const float s = __uint_as_float(sbyte << 23);
        return kFp4Lut[code] * s;
    }
    // magnitude = m * 2^x with m in {1, 3}: 0.5 = 1*2^-1, 1, 1.5 = 3*2^-1, 2, 3 = 3*2^0, 4, 6 = 3*2^1
    const int m3 = (mag == 3 || mag == 5 || mag == 7);
    const int x = m3 ? (int)(mag >> 1) - 2 : (int)(mag >> 1) - 1;
    const int E = sbyte == 0 ? 1 : (int)sbyte;
    const int q = x + m3 + E - 127;  // unbiased exponent of the value (m = 3 -> 1.5 * 2^(x + 1))
    uint32_t bits;
    if (q > 127)
        bits = 0x7F800000u;
    else if (q >= -126)
        bits = ((uint32_t)(q + 127) << 23) | (m3 ? 0x400000u : 0u);
    else
        bits = (m3 ? 3u : 1u) << (x + E + 22);  // m * 2^(x + E - 127) as a multiple of 2^-149
    return __uint_as_float(bits | sign);
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

template <int NW, int P, bool GU>
static int launch_expert_nw(const MoeDev &d, const MoeScratch &sc, const MoeRun &run, hipStream_t st) {
    constexpr size_t lds = moe_lds_bytes(NW, P, GU);
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&moe_expert_kernel<NW, P, GU>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const int64_t NB = GU ? 2 * d.I / 32 : d.H / 32;
    const int64_t ngrp = GU ? (d.I / 32) / (NW / 2) : (NB + NW - 1) / NW;
    hipLaunchKernelGGL((moe_expert_kernel<NW, P, GU>), dim3((unsigned)(d.E * ngrp)), dim3(NW * 64), lds, st, d, sc,
                       run);
    return (int)hipGetLastError();
}

// gate_up: NW / 2 column-block pairs, the largest of 3, 2, 1 dividing I / 32; down: 6 blocks
template <int P, bool GU>
static int launch_expert(const MoeDev &d, const MoeScratch &sc, const MoeRun &run, hipStream_t st) {
    if (GU) {
        const int64_t cb = d.I / 32;
        if (cb % 3 == 0) return launch_expert_nw<6, P, GU>(d, sc, run, st);
        if (cb % 2 == 0) return launch_expert_nw<4, P, GU>(d, sc, run, st);
        return launch_expert_nw<2, P, GU>(d, sc, run, st);
    }
    return launch_expert_nw<6, P, GU>(d, sc, run, st);
}

int launch_moe(const MoeDev &d, const void *x, int x_bf16, int64_t T, const float *logits, int k, float limit,
               float *y, uint32_t *topk_idx, float *topk_w, void *scratch, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    int e = 0;
    const MoeScratch sc = carve(scratch, T, d.E, d.H, d.I, k, x_bf16);
    MoeRun run;
    run.A = T * k;
    run.limit = limit;
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, logits, T, (int)d.E, k,
                       sc.ti, sc.tw, topk_idx, topk_w);
    switch (k) {
#define NNQ_PERM(K)                                                                                              \
    case K:                                                                                                      \
        hipLaunchKernelGGL(moe_permute_kernel<K>, dim3(1), dim3(1024), 0, st, sc.ti, T, (int)d.E, sc.off, sc.stok, \
                           sc.pos);                                                                              \
        break;
        NNQ_PERM(1) NNQ_PERM(2) NNQ_PERM(3) NNQ_PERM(4) NNQ_PERM(5) NNQ_PERM(6) NNQ_PERM(7) NNQ_PERM(8)
#undef NNQ_PERM
    default:
        return (int)hipErrorInvalidValue;
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
        e = launch_expert<1, true>(d, sc, run, st);
    else
        e = launch_expert<2, true>(d, sc, run, st);
    if (e) return e;
    e = launch_expert<2, false>(d, sc, run, st);
    if (e) return e;
    switch (k) {
#define NNQ_COMB(K)                                                                                  \
    case K:                                                                                          \
        hipLaunchKernelGGL(moe_combine_kernel<K>, dim3((unsigned)T), dim3(256), 0, st, sc, d.H, y); \
        break;
        NNQ_COMB(1) NNQ_COMB(2) NNQ_COMB(3) NNQ_COMB(4) NNQ_COMB(5) NNQ_COMB(6) NNQ_COMB(7) NNQ_COMB(8)
#undef NNQ_COMB
    default:
        return (int)hipErrorInvalidValue;
    }
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

}  // namespace nnq
