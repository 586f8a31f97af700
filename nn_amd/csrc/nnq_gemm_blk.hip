// Prefill GEMM for Q8_0 and Q6_K weights on gfx950 (M > 8 tokens):
// Y[m, n] = X[m, k] . W[n, k]^T (+ bias), f32 accumulation, f32 or bf16 output: the
// arithmetic of QLinear::forward with a batch of tokens for these formats
// (crates/nn-core/src/layers/quantized/linear.rs:366-400; quantized_matmul_core,
// crates/nn-core/src/dyn_tensor/quantized_matmul.rs:232-272), on the 16x16x32 f16 MFMA.
//
// Activations: staged once per call by the Q4_K GEMM's gemm_prep (each row of x times a
// power of two 2^s_row, in f16; f32 input as hi + lo planes, P = 2), undone per row in
// the epilogue.
//
// Weights are read in the tile16 device image the decode GEMVs stream (no second copy):
//   Q8_0  w = d * q (d f16 per 32 k, q int8).  B = q, exact in f16; each 32-k block's MFMA
//         partial (from zero) is added as d_n * partial to the f32 totals.
//   Q6_K  w = (d * sc) * (q - 32) (d f16 per 256 k, sc int8 per 16 k, q 6-bit).  With
//         q' = q - 32, B = sc * (q' & ~1) + sc * (q' & 1): two operands, each an exact f16
//         (|sc * (q' & ~1)| = 2 |sc| |q' >> 1| needs at most 11 bits), two MFMAs per 32 k;
//         a super-block's MFMAs accumulate from zero and d_n * partial is added at its end.
//
// Tiling: a workgroup computes BM x BN outputs (BN 64, or 128 for large bf16 batches)
// with 2 x WGN waves (4 waves of BM/2 x 32 for 64-wide tiles, 8 waves of 64 x 32 for
// 128 x 128 tiles: two waves per SIMD), MT x NT MFMA tiles per wave.  K advances 256 per
// stage: the stage's activation rows, the raw weight bytes of its BN / 16 column tiles
// and their headers go to LDS; the next stage is prefetched into registers (buffer loads
// at a scalar per-stage offset) during the current one's compute.  The MFMA partials are
// written to VGPRs (a per-file compiler option), so scaling them needs no register
// moves; Q8_0 scales each block's partials one block after their MFMAs.  Split-K (KS > 1, when
// the output tiles alone would leave CUs idle): workgroup (tile, ks) covers stages
// [ks * S / KS, (ks + 1) * S / KS) and stores its f32 partial in slab ks of the scratch;
// gemm_blk_finalize_kernel sums the slabs in order (deterministic), adds the bias and
// converts.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

template <int FMT, int BM, int P, int BN_, int WGN>
struct BlkCfg {
    // waves: 2 (rows) x WGN (columns), wave tile WM x (BN / WGN)
    static constexpr int NW = 2 * WGN, NTH = NW * 64, BN = BN_, NTILE = BN / 16;
    static constexpr int WM = BM / 2, MT = WM / 16, NT = NTILE / WGN;
    static_assert(NTILE % WGN == 0, "whole column tiles per wave");
    static constexpr int AST = 264;  // LDS row stride of the staged activation (f16): 256 + 8 pad
    static constexpr int TB = FMT == NNQ_FMT_Q8_0 ? 4096 : 3072;  // raw bytes per column tile and stage
    static constexpr int HB = FMT == NNQ_FMT_Q8_0 ? 256 : 288;    // header bytes per column tile and stage
    static constexpr size_t A_BYTES = (size_t)P * BM * AST * 2;
    static constexpr size_t B_BYTES = (size_t)NTILE * TB;
    static constexpr size_t H_BYTES = (size_t)NTILE * HB;
    static constexpr size_t LDS = A_BYTES + B_BYTES + H_BYTES;
    static constexpr int ACH = P * BM * 32;      // 16-byte activation chunks per stage
    static constexpr int BCH = NTILE * TB / 16;  // 16-byte weight chunks per stage
    static constexpr int HCH = NTILE * HB / 16;  // 16-byte header chunks per stage
    static constexpr int APT = (ACH + NTH - 1) / NTH, BPT = (BCH + NTH - 1) / NTH, HPT = (HCH + NTH - 1) / NTH;
    static_assert(HB % 16 == 0 && TB % 16 == 0, "16-byte chunks");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
};

__device__ __forceinline__ uint32_t pk_add_f16(uint32_t a, half2v b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) + b);
}
__device__ __forceinline__ uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) * __builtin_bit_cast(half2v, b));
}

// Q8_0: the 8 codes of a lane (bytes in (e0, e2, e1, e3) order per word, so bytes 0 and 2
// are the pair (e0, e1)) as the f16 B operand: the byte q + 128 under the high byte 0x64
// (one byte permute per pair) is the f16 1024 + q + 128, exact, and 1152 is subtracted
// exactly.
__device__ __forceinline__ u32x4 q8_b_operand(u32x2 raw) {
    const half2v off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t k = 0x64646464u;
    const uint32_t t0 = raw[0] ^ 0x80808080u, t1 = raw[1] ^ 0x80808080u;
    // selector bytes 0-3 take bytes of the second operand (t), 4 the first byte of k
    return u32x4{pk_add_f16(__builtin_amdgcn_perm(k, t0, 0x04020400u), off),
                 pk_add_f16(__builtin_amdgcn_perm(k, t0, 0x04030401u), off),
                 pk_add_f16(__builtin_amdgcn_perm(k, t1, 0x04020400u), off),
                 pk_add_f16(__builtin_amdgcn_perm(k, t1, 0x04030401u), off)};
}

// Q6_K: the 8 values of one 32-k step of a lane (pairs j = 4h .. 4h + 3: nibbles in word
// W at bits 4(j % 4) and 16 + 4(j % 4), crumbs of word C at bits 2j and 16 + 2j) as the
// two f16 B operands sc * (q' & ~1) and sc * (q' & 1), q' = q - 32.  (q & 0x3E) | 0x6400
// is the f16 1024 + (q & ~1), and 1056 is subtracted exactly; (q & 1) times the f16 bits
// of sc is sc or 0.
template <int H>
__device__ __forceinline__ void q6_b_operands(uint32_t W, uint32_t Cw, uint32_t sch, u32x4 &b1, u32x4 &b2) {
    const half2v off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const uint32_t sc2 = sch | (sch << 16);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const int j = 4 * H + jj;
        const uint32_t q = ((W >> (4 * jj)) & 0x000F000Fu) | (((Cw >> (2 * j)) & 0x00030003u) << 4);
        b1[jj] = pk_mul_f16(pk_add_f16((q & 0x003E003Eu) | 0x64006400u, off), sc2);
        b2[jj] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q & 0x00010001u) * __builtin_bit_cast(u16x2, sc2));
    }
}

}  // namespace

template <int FMT, int BM, int P, int BN, int WGN>
__global__ __launch_bounds__(2 * WGN * 64) void gemm_blk_kernel(GemmArgs a, GemmScratch sc) {
    using C = BlkCfg<FMT, BM, P, BN, WGN>;
    constexpr int NTH = C::NTH, MT = C::MT, NT = C::NT, AST = C::AST;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint16_t *As = reinterpret_cast<uint16_t *>(smem);
    uint8_t *Bs = smem + C::A_BYTES;
    uint8_t *Hs = Bs + C::B_BYTES;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv / WGN, wn = wv % WGN;
    const int p = lane >> 4, l16 = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * C::BN, m0 = (int64_t)blockIdx.y * BM;
    const int64_t t0 = n0 / 16;
    const int64_t K = a.k, M = a.m;
    const int64_t nstage_all = FMT == NNQ_FMT_Q8_0 ? a.nblk / 8 : a.nblk;  // 256 k per stage
    const int KS = (int)gridDim.z, ks = (int)blockIdx.z;
    const int64_t s_begin = ks * nstage_all / KS, nstage = (ks + 1) * nstage_all / KS - s_begin;

    floatx4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    u32x4 ra[C::APT], rb[C::BPT], rh[C::HPT];
    // global -> registers for stage s: buffer loads from the workgroup's bases, a 32-bit
    // lane offset fixed for the whole loop plus a scalar per-stage offset (no per-lane
    // address arithmetic in the loop).  Rows past M read row M - 1 and column tiles past
    // the weight read its last tile (their outputs are never stored); activation columns
    // past K (Q8_0 pads its blocks to groups of 8) are zeroed in the last stage.  The
    // ranges are exact, so an access outside them would read zeros.
    constexpr bool Q8 = FMT == NNQ_FMT_Q8_0;
    const int64_t tile_q = Q8 ? (a.nblk / 2) * 1024 : a.nblk * 3072;  // quant bytes per column tile
    const int64_t tile_h = Q8 ? (a.nblk / 8) * 256 : a.nblk * 288;    // header bytes per column tile
    const int mlast = (int)min((int64_t)BM - 1, M - 1 - m0);
    const int tlast = (int)min((int64_t)C::NTILE - 1, a.ntile - 1 - t0);
    auto range = [](int64_t bytes) { return (int)(uint32_t)min(bytes, (int64_t)0xFFFFFFFF); };
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(sc.xh + m0 * K), 0, range(((int64_t)P * M - m0) * K * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.qs + t0 * tile_q), 0, range((a.ntile - t0) * tile_q), 0x00020000);
    const __amdgpu_buffer_rsrc_t rhd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.hdr + t0 * tile_h), 0, range((a.ntile - t0) * tile_h), 0x00020000);
    const int plane = (int)(M * K * 2);  // bytes per activation plane (the host keeps P * M * K * 2 < 2^31)
    int aof[C::APT], bof[C::BPT], hof[C::HPT], acol[C::APT];
#pragma unroll
    for (int i = 0; i < C::APT; i++) {
        const int c = min(tid + i * NTH, C::ACH - 1), rem = c % (BM * 32);
        acol[i] = (rem % 32) * 8;
        aof[i] = (c / (BM * 32)) * plane + (min(rem / 32, mlast) * (int)K + acol[i]) * 2;
    }
#pragma unroll
    for (int i = 0; i < C::BPT; i++) {
        const int c = min(tid + i * NTH, C::BCH - 1);
        bof[i] = (int)(min(c / (C::TB / 16), tlast) * tile_q + (c % (C::TB / 16)) * 16);
    }
#pragma unroll
    for (int i = 0; i < C::HPT; i++) {
        const int c = min(tid + i * NTH, C::HCH - 1);
        hof[i] = (int)(min(c / (C::HB / 16), tlast) * tile_h + (c % (C::HB / 16)) * 16);
    }
    auto gload = [&](int64_t s) {
        const int sx = (int)s * 512, sq = (int)s * (Q8 ? 4096 : 3072), sh = (int)s * (Q8 ? 256 : 288);
#pragma unroll
        for (int i = 0; i < C::APT; i++)
            ra[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, aof[i], sx, 0));
        if (Q8 && s * 256 + 256 > K) {  // workgroup-uniform: the last, padded stage
#pragma unroll
            for (int i = 0; i < C::APT; i++)
                if (s * 256 + acol[i] >= K) ra[i] = u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < C::BPT; i++)
            rb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, bof[i], sq, 0));
#pragma unroll
        for (int i = 0; i < C::HPT; i++)
            if (tid + i * NTH < C::HCH)
                rh[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rhd, hof[i], sh, 0));
    };
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
#pragma unroll
        for (int i = 0; i < C::HPT; i++) {
            const int c = tid + i * NTH;
            if (c < C::HCH) *reinterpret_cast<u32x4 *>(Hs + c * 16) = rh[i];
        }
    };
    // A fragments of 32 k at column offset kc of the stage: lane (p, l16) takes row l16 of
    // each tile, k = kc + 8p .. + 7
    auto afrag = [&](int kc, u32x4 (&af)[P][MT]) {
#pragma unroll
        for (int pl = 0; pl < P; pl++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                af[pl][mt] = *reinterpret_cast<const u32x4 *>(As + (pl * BM + wm * C::WM + mt * 16 + l16) * AST + kc +
                                                              8 * p);
    };

    if (nstage > 0) gload(s_begin);
    for (int64_t st = 0; st < nstage; st++) {
        __syncthreads();  // the previous stage's fragments have been read
        sstore();
        __syncthreads();
        if (st + 1 < nstage) gload(s_begin + st + 1);
        if constexpr (FMT == NNQ_FMT_Q8_0) {
            // each block's MT x NT partials go to their own registers, and d * partial is
            // added to the totals one block later, so no MFMA result is waited on at once
            // per column tile: the lane's row's eight d of the stage (one 16-byte read), and
            // per pair of blocks its 16 code bytes of both (one 16-byte read: consecutive
            // lanes read consecutive 16 bytes, no bank conflicts)
            floatx4 part[2][MT][NT];
            float dcol[2][NT];
            u32x4 hd[NT], raw2[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                hd[nt] = *reinterpret_cast<const u32x4 *>(Hs + (wn * NT + nt) * 256 + 16 * l16);
#pragma unroll
            for (int blk = 0; blk <= 8; blk++) {
                if (blk < 8) {
                    u32x4 af[P][MT];
                    afrag(32 * blk, af);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const int tt = wn * NT + nt;  // column tile within the workgroup
                        if ((blk & 1) == 0)
                            raw2[nt] = *reinterpret_cast<const u32x4 *>(Bs + tt * 4096 + (blk >> 1) * 1024 +
                                                                        16 * (16 * p + l16));
                        const u32x2 raw = {raw2[nt][2 * (blk & 1)], raw2[nt][2 * (blk & 1) + 1]};
                        dcol[blk & 1][nt] = f16_to_f32((hd[nt][blk >> 1] >> (16 * (blk & 1))) & 0xFFFFu);
                        const u32x4 b = q8_b_operand(raw);
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) {
                            floatx4 pt = mfma16x16x32_f16(af[0][mt], b, floatx4{0.f, 0.f, 0.f, 0.f});
                            if constexpr (P == 2) pt = mfma16x16x32_f16(af[1][mt], b, pt);
                            part[blk & 1][mt][nt] = pt;
                        }
                    }
                }
                if (blk > 0) {
                    const int q = (blk - 1) & 1;
                    // the d of column l16 applies to all four rows this lane holds
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
#pragma unroll
                        for (int mt = 0; mt < MT; mt++)
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                acc[mt][nt][i] = __builtin_fmaf(dcol[q][nt], part[q][mt][nt][i], acc[mt][nt][i]);
                }
            }
        } else {
            floatx4 part[MT][NT];
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int j = 0; j < NT; j++) part[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; c++) {  // 64-value chunk of the super-block
                uint32_t WA[NT], WB[NT], WC[NT], s0[NT], s1[NT];
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const int tt = wn * NT + nt;
                    const uint32_t *q = reinterpret_cast<const uint32_t *>(Bs + tt * 3072 + c * 768 + 12 * (16 * p + l16));
                    WA[nt] = q[0];
                    WB[nt] = q[1];
                    WC[nt] = q[2];
                    // sub-block scales of this lane's k: 64c + 8p (step 0), 64c + 32 + 8p (step 1)
                    const int8_t *scp = reinterpret_cast<const int8_t *>(Hs + tt * 288 + 16 * l16);
                    s0[nt] = f32_to_f16_bits((float)scp[4 * c + (p >> 1)]);
                    s1[nt] = f32_to_f16_bits((float)scp[4 * c + 2 + (p >> 1)]);
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    u32x4 af[P][MT];
                    afrag(64 * c + 32 * h, af);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        u32x4 b1, b2;
                        if (h == 0)
                            q6_b_operands<0>(WA[nt], WC[nt], s0[nt], b1, b2);
                        else
                            q6_b_operands<1>(WB[nt], WC[nt], s1[nt], b1, b2);
#pragma unroll
                        for (int pl = 0; pl < P; pl++)
#pragma unroll
                            for (int mt = 0; mt < MT; mt++) {
                                part[mt][nt] = mfma16x16x32_f16(af[pl][mt], b1, part[mt][nt]);
                                part[mt][nt] = mfma16x16x32_f16(af[pl][mt], b2, part[mt][nt]);
                            }
                    }
                }
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int tt = wn * NT + nt;
                const float d = f16_to_f32(*reinterpret_cast<const uint16_t *>(Hs + tt * 288 + 256 + 2 * l16));
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[mt][nt][i] = __builtin_fmaf(d, part[mt][nt][i], acc[mt][nt][i]);
            }
        }
    }

    // store: lane holds rows 4p + i of each 16 x 16 tile, column l16; with a K split the
    // f32 partial goes to slab ks (bias and conversion in the finalize)
    float *slab = KS > 1 ? sc.ysplit + (int64_t)ks * M * a.n : nullptr;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int64_t col = n0 + wn * (NT * 16) + nt * 16 + l16;
        if (col >= a.n) continue;
        const float bcol = (a.bias && KS == 1) ? a.bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t row = m0 + wm * C::WM + mt * 16 + 4 * p + i;
                if (row >= M) continue;
                const float y = acc[mt][nt][i] * sc.rowback[row] + bcol;
                if (slab)
                    slab[row * a.n + col] = y;
                else if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[row * a.n + col] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[row * a.n + col] = y;
            }
    }
}

// split-K result: the slabs summed in order plus the bias, stored as f32 or bf16
__global__ __launch_bounds__(256) void gemm_blk_finalize_kernel(const float *ys, int ks, const float *bias, void *y,
                                                                int y_bf16, int64_t m, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= m * n) return;
    float v = ys[i];
    for (int j = 1; j < ks; j++) v += ys[(int64_t)j * m * n + i];
    if (bias) v += bias[i % n];
    if (y_bf16)
        reinterpret_cast<uint16_t *>(y)[i] = (uint16_t)f32_to_bf16_bits(v);
    else
        reinterpret_cast<float *>(y)[i] = v;
}

template <int FMT, int BM, int P, int BN, int WGN = 2>
static int launch_blk_cfg(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    using C = BlkCfg<FMT, BM, P, BN, WGN>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_blk_kernel<FMT, BM, P, BN, WGN>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const dim3 grid((unsigned)((a.ntile * 16 + C::BN - 1) / C::BN), (unsigned)((a.m + BM - 1) / BM),
                    (unsigned)sc.ksplit);
    constexpr size_t lds = C::LDS;
    hipLaunchKernelGGL((gemm_blk_kernel<FMT, BM, P, BN, WGN>), grid, dim3(C::NTH), lds, st, a, sc);
    int e = (int)hipGetLastError();
    if (e || sc.ksplit == 1) return e;
    const int64_t cnt = a.m * a.n;
    hipLaunchKernelGGL(gemm_blk_finalize_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, st, sc.ysplit,
                       sc.ksplit, a.bias, a.y, a.y_bf16, a.m, a.n);
    return (int)hipGetLastError();
}

// Tile shape and K split: 64 x 64 tiles, 128 x 64 from 1024 rows on; with bf16 input
// 128 x 128 tiles on eight waves from 256 rows on for Q6_K and from 1024 for Q8_0 (the
// operand work per MFMA halves: Q6_K 512x4096x12288 150 us against 184 with 64-wide
// tiles, Q8_0 2048x4096x4096 133 against 165; Q8_0 at 512 rows 60 against 50).
// The K split doubles (up to 16, at least one stage each) while the tiles alone fill
// fewer than 512 workgroups (two per CU), or 256 for the 128 x 128 tiles, whose LDS
// holds one workgroup per CU (Q6_K 512 rows: split 2 instead of 4, 149 -> 135 us).
int gemm_blk_plan(const GemmArgs &a, int *bm, int *bn) {
    const int64_t nstage = a.blk == NNQ_FMT_Q8_0 ? a.nblk / 8 : a.nblk;
    const bool wide = a.x_bf16 && a.m >= (a.blk == NNQ_FMT_Q6_K ? 256 : 1024);
    const int b = (wide || a.m >= 1024) ? 128 : 64, c = wide ? 128 : 64;
    const int64_t tiles = ((a.ntile * 16 + c - 1) / c) * ((a.m + b - 1) / b);
    int ks = 1;
    while (tiles * ks < (wide ? 256 : 512) && ks * 2 <= 16 && ks * 2 <= nstage) ks *= 2;
    if (bm) *bm = b;
    if (bn) *bn = c;
    return ks;
}

template <int FMT, int P>
static int launch_blk_p(const GemmArgs &a, const GemmScratch &sc, hipStream_t st) {
    int bm = 64, bn = 64;
    const int ks = gemm_blk_plan(a, &bm, &bn);
    if (ks != sc.ksplit || (ks > 1 && !sc.ysplit)) return (int)hipErrorInvalidValue;
    if constexpr (P == 1)
        if (bn == 128) return launch_blk_cfg<FMT, 128, P, 128, 4>(a, sc, st);
    if (bm == 128) return launch_blk_cfg<FMT, 128, P, 64>(a, sc, st);
    return launch_blk_cfg<FMT, 64, P, 64>(a, sc, st);
}

int launch_gemm_blk(const GemmArgs &a, void *stream) {
    if (a.m <= 0) return 0;
    if (a.blk != NNQ_FMT_Q8_0 && a.blk != NNQ_FMT_Q6_K) return (int)hipErrorInvalidValue;
    const GemmScratch sc = gemm_carve(a.scratch, a, nullptr);
    if (gemm_wide8_plan(a, nullptr)) return launch_gemm_wide8(a, sc, stream);  // Q8_0, bf16, M > 128
    hipStream_t st = (hipStream_t)stream;
    int e = launch_gemm_prep(a, sc, st);
    if (e) return e;
    if (a.blk == NNQ_FMT_Q8_0)
        return a.x_bf16 ? launch_blk_p<NNQ_FMT_Q8_0, 1>(a, sc, st) : launch_blk_p<NNQ_FMT_Q8_0, 2>(a, sc, st);
    return a.x_bf16 ? launch_blk_p<NNQ_FMT_Q6_K, 1>(a, sc, st) : launch_blk_p<NNQ_FMT_Q6_K, 2>(a, sc, st);
}

}  // namespace nnq
