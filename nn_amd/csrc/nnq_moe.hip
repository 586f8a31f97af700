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
// routing
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void moe_route_kernel(const float *logits, int64_t T, int E, int k, uint32_t *ti,
                                                       float *tw, uint32_t *ti_out, float *tw_out) {
    const int64_t t = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (t >= T) return;
    const float *x = logits + t * E;
    // probs = softmax(logits) (DynTensor::softmax, crates/nn-core/src/dyn_tensor/softmax.rs:30-60,
    // called at crates/nn-gptoss/src/quantized_model.rs:140): exp(x - max) / sum
    float mx = -INFINITY;
    for (int c = 0; c < E; c++) mx = fmaxf(mx, x[c]);
    int ninf = 0;
    for (int c = 0; c < E; c++) ninf += x[c] == INFINITY;
    float sum = -0.0f;
    if (mx != -INFINITY && mx != INFINITY)
        for (int c = 0; c < E; c++) sum = sum + expf(x[c] - mx);
    auto prob = [&](int c) -> float {
        if (mx == -INFINITY) return 0.0f;
        if (mx == INFINITY) return x[c] == INFINITY ? 1.0f / (float)ninf : 0.0f;
        return expf(x[c] - mx) / sum;
    };
    uint32_t idx[8];
    float val[8];
    for (int s = 0; s < k; s++) {
        int best = -1;
        int32_t bk = 0;
        float bv = 0.0f;
        for (int c = 0; c < E; c++) {
            bool taken = false;
            for (int q = 0; q < s; q++) taken |= (int)idx[q] == c;
            if (taken) continue;
            const float p = prob(c);
            const int32_t key = total_key(p);
            if (best < 0 || key > bk) {
                best = c;
                bk = key;
                bv = p;
            }
        }
        idx[s] = (uint32_t)best;
        val[s] = bv;
    }
    float ssum = -0.0f;
    for (int s = 0; s < k; s++) ssum = ssum + val[s];
    for (int s = 0; s < k; s++) {
        const float w = val[s] / ssum;
        ti[t * k + s] = idx[s];
        tw[t * k + s] = w;
        if (ti_out) ti_out[t * k + s] = idx[s];
        if (tw_out) tw_out[t * k + s] = w;
    }
}

// One workgroup: counts, offsets and the stable per-expert order.  The slot list is
// staged in LDS; thread e walks it in (token, slot) order for expert e.
__global__ __launch_bounds__(256) void moe_permute_kernel(const uint32_t *ti, int64_t T, int E, int k, int32_t *off,
                                                          int32_t *stok, int32_t *pos) {
    extern __shared__ uint32_t sti[];  // [T * k]
    __shared__ int32_t cnt[257];
    const int tid = threadIdx.x;
    const int64_t A = T * k;
    for (int64_t i = tid; i < A; i += 256) sti[i] = ti[i];
    __syncthreads();
    if (tid < E) {
        int32_t c = 0;
        for (int64_t i = 0; i < A; i++) c += sti[i] == (uint32_t)tid;
        cnt[tid] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int32_t acc = 0;
        for (int e = 0; e < E; e++) {
            const int32_t c = cnt[e];
            cnt[e] = acc;
            off[e] = acc;
            acc += c;
        }
        off[E] = acc;
    }
    __syncthreads();
    if (tid < E) {
        int32_t p = cnt[tid];
        for (int64_t i = 0; i < A; i++)
            if (sti[i] == (uint32_t)tid) {
                stok[p] = (int32_t)(i / k);
                pos[i] = p;
                p++;
            }
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
// gate_up grouped GEMM with the SwiGLU epilogue
// ---------------------------------------------------------------------------------
struct MoeRun {
    const uint16_t *xa[2];  // activation planes (bf16), rows of H
    int64_t A;              // assignments (T * k): rows of the sorted buffers
    float limit;
};

// Workgroup = (expert, CPW gate column blocks + the matching CPW up blocks); wave w
// owns block w.  Token rows go in chunks of 16 * MT.
template <int CPW, int P, int MT>
__global__ __launch_bounds__(2 * CPW * 64) void moe_gate_up_kernel(MoeDev d, MoeScratch sc, MoeRun run) {
    const int64_t H = d.H, I = d.I;
    const int64_t ncg = I / 32 / CPW;
    const int64_t e = blockIdx.x / ncg, cg = blockIdx.x % ncg;
    const int32_t r0 = sc.off[e], ne = sc.off[e + 1] - r0;
    if (ne == 0) return;  // workgroup-uniform
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int half = wv / CPW, cbl = wv % CPW;  // half 0: gate, 1: up
    const int64_t gcol0 = (cg * CPW + cbl) * 32;  // first gate column of this wave's block
    const int64_t nbg = 2 * I / 32;               // column blocks of W_gu
    const int64_t nb = half * (I / 32) + cg * CPW + cbl;
    const int64_t KB = H / 32;
    const uint8_t *cq = d.gu_q + (e * nbg + nb) * KB * 512;
    const uint8_t *cs = d.gu_s + (e * nbg + nb) * KB * 32;
    const int p = lane >> 4, l16 = lane & 15;
    __shared__ float gbuf[CPW][MT * 16][33];
    for (int32_t m0 = 0; m0 < ne; m0 += MT * 16) {
        floatx4 acc[MT][2];
        const uint16_t *arow[MT][P];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            acc[mt][0] = acc[mt][1] = zero4();
            const int32_t r = m0 + mt * 16 + l16;
            const int64_t tok = r < ne ? (int64_t)sc.stok[r0 + r] : -1;
#pragma unroll
            for (int pl = 0; pl < P; pl++) arow[mt][pl] = tok >= 0 ? run.xa[pl] + tok * H + 8 * p : nullptr;
        }
        for (int64_t kb = 0; kb < KB; kb++) {
            u32x4 be, bo;
            fp4_b_operands(cq + kb * 512, cs + kb * 32, lane, be, bo);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                if (m0 + mt * 16 >= ne) break;  // wave-uniform
#pragma unroll
                for (int pl = 0; pl < P; pl++) {
                    const u32x4 a = arow[mt][pl] ? *reinterpret_cast<const u32x4 *>(arow[mt][pl] + kb * 32)
                                                 : u32x4{0u, 0u, 0u, 0u};
                    acc[mt][0] = mfma16x16x32_bf16(a, be, acc[mt][0]);
                    acc[mt][1] = mfma16x16x32_bf16(a, bo, acc[mt][1]);
                }
            }
        }
        // lane holds rows 4p + i of each tile; tile 0 = columns 2 * l16, tile 1 = 2 * l16 + 1
        if (half == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int o = 0; o < 2; o++) {
                        const int c = 2 * l16 + o;
                        gbuf[cbl][mt * 16 + 4 * p + i][c] = acc[mt][o][i] + d.gu_b[e * 2 * I + gcol0 + c];
                    }
        }
        __syncthreads();
        if (half == 1) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int32_t r = m0 + mt * 16 + 4 * p + i;
                    if (r >= ne) continue;
#pragma unroll
                    for (int o = 0; o < 2; o++) {
                        const int c = 2 * l16 + o;
                        const float g = gbuf[cbl][mt * 16 + 4 * p + i][c];
                        const float u = acc[mt][o][i] + d.gu_b[e * 2 * I + I + gcol0 + c];
                        // silu (crates/nn-core/src/dyn_tensor/ops/math.rs:140), clamped to +-limit
                        float sg = g / (1.0f + expf(-g));
                        sg = sg < -run.limit ? -run.limit : (sg > run.limit ? run.limit : sg);
                        const float h = sg * u;
                        const uint16_t hh = bf16_rne(h);
                        const int64_t o2 = (int64_t)(r0 + r) * I + gcol0 + c;
                        sc.hb[o2] = hh;
                        sc.hb[run.A * I + o2] = bf16_rne(h - bf16_to_f32(hh));
                    }
                }
        }
        __syncthreads();  // gbuf is reused by the next row chunk
    }
}

// ---------------------------------------------------------------------------------
// down grouped GEMM: y_e = h x W_down[e] + b_down[e], per sorted row
// ---------------------------------------------------------------------------------
// Workgroup = (expert, 4 column blocks); wave w owns block 4 * blk + w (waves past the
// last block return at once: there is no barrier in this kernel).
template <int MT>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeDev d, MoeScratch sc, MoeRun run) {
    const int64_t H = d.H, I = d.I;
    const int64_t NB = H / 32, nblk = (NB + 3) / 4;
    const int64_t e = blockIdx.x / nblk;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t nb = (blockIdx.x % nblk) * 4 + wv;
    const int32_t r0 = sc.off[e], ne = sc.off[e + 1] - r0;
    if (ne == 0 || nb >= NB) return;
    const int64_t KB = I / 32;
    const uint8_t *cq = d.dn_q + (e * NB + nb) * KB * 512;
    const uint8_t *cs = d.dn_s + (e * NB + nb) * KB * 32;
    const int p = lane >> 4, l16 = lane & 15;
    for (int32_t m0 = 0; m0 < ne; m0 += MT * 16) {
        floatx4 acc[MT][2];
        const uint16_t *arow[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            acc[mt][0] = acc[mt][1] = zero4();
            const int32_t r = m0 + mt * 16 + l16;
            arow[mt] = r < ne ? sc.hb + (int64_t)(r0 + r) * I + 8 * p : nullptr;
        }
        for (int64_t kb = 0; kb < KB; kb++) {
            u32x4 be, bo;
            fp4_b_operands(cq + kb * 512, cs + kb * 32, lane, be, bo);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                if (m0 + mt * 16 >= ne) break;  // wave-uniform
#pragma unroll
                for (int pl = 0; pl < 2; pl++) {
                    const u32x4 a = arow[mt] ? *reinterpret_cast<const u32x4 *>(arow[mt] + pl * run.A * I + kb * 32)
                                             : u32x4{0u, 0u, 0u, 0u};
                    acc[mt][0] = mfma16x16x32_bf16(a, be, acc[mt][0]);
                    acc[mt][1] = mfma16x16x32_bf16(a, bo, acc[mt][1]);
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int32_t r = m0 + mt * 16 + 4 * p + i;
                if (r >= ne) continue;
#pragma unroll
                for (int o = 0; o < 2; o++) {
                    const int64_t col = nb * 32 + 2 * l16 + o;
                    sc.yb[(int64_t)(r0 + r) * H + col] = acc[mt][o][i] + d.dn_b[e * H + col];
                }
            }
    }
}

// y[t] = ((0 + w_a * y_a) + w_b * y_b) + ... over the token's experts a < b < ...
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeScratch sc, int64_t H, int k, float *y) {
    const int64_t t = blockIdx.x;
    uint32_t ex[8];
    int32_t ps[8];
    float ws[8];
    for (int s = 0; s < k; s++) {
        ex[s] = sc.ti[t * k + s];
        ps[s] = sc.pos[t * k + s];
        ws[s] = sc.tw[t * k + s];
    }
    for (int s = 1; s < k; s++)  // insertion sort by expert (the k experts are distinct)
        for (int q = s; q > 0 && ex[q - 1] > ex[q]; q--) {
            const uint32_t te = ex[q];
            ex[q] = ex[q - 1];
            ex[q - 1] = te;
            const int32_t tp = ps[q];
            ps[q] = ps[q - 1];
            ps[q - 1] = tp;
            const float tw2 = ws[q];
            ws[q] = ws[q - 1];
            ws[q - 1] = tw2;
        }
    for (int64_t c = threadIdx.x; c < H; c += 256) {
        float acc = 0.0f;
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

int launch_moe(const MoeDev &d, const void *x, int x_bf16, int64_t T, const float *logits, int k, float limit,
               float *y, uint32_t *topk_idx, float *topk_w, void *scratch, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    const MoeScratch sc = carve(scratch, T, d.E, d.H, d.I, k, x_bf16);
    MoeRun run;
    run.A = T * k;
    run.limit = limit;
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((T + 63) / 64)), dim3(64), 0, st, logits, T, (int)d.E, k,
                       sc.ti, sc.tw, topk_idx, topk_w);
    const size_t perm_lds = (size_t)T * k * 4;
    if (perm_lds > 64 * 1024) return (int)hipErrorInvalidValue;  // more than 16384 assignments
    hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(256), perm_lds, st, sc.ti, T, (int)d.E, k, sc.off, sc.stok,
                       sc.pos);
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
    const int64_t ncb = d.I / 32;
    if (ncb % 2 == 0) {
        const unsigned grid = (unsigned)(d.E * (ncb / 2));
        if (x_bf16)
            hipLaunchKernelGGL((moe_gate_up_kernel<2, 1, 4>), dim3(grid), dim3(256), 0, st, d, sc, run);
        else
            hipLaunchKernelGGL((moe_gate_up_kernel<2, 2, 4>), dim3(grid), dim3(256), 0, st, d, sc, run);
    } else {
        const unsigned grid = (unsigned)(d.E * ncb);
        if (x_bf16)
            hipLaunchKernelGGL((moe_gate_up_kernel<1, 1, 4>), dim3(grid), dim3(128), 0, st, d, sc, run);
        else
            hipLaunchKernelGGL((moe_gate_up_kernel<1, 2, 4>), dim3(grid), dim3(128), 0, st, d, sc, run);
    }
    const int64_t NB = d.H / 32;
    hipLaunchKernelGGL((moe_down_kernel<4>), dim3((unsigned)(d.E * ((NB + 3) / 4))), dim3(256), 0, st, d, sc, run);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)T), dim3(256), 0, st, sc, d.H, k, y);
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
