// Prefill GEMM for Q8_0 weights and bf16 activations on gfx950, wide-wave-tile kernel:
// Y[m, n] = X[m, k] . W[n, k]^T (+ bias), the arithmetic of QLinear::forward with a batch of
// tokens over Q8_0 (crates/nn-core/src/layers/quantized/linear.rs:366-400; quantized_matmul_core,
// crates/nn-core/src/dyn_tensor/quantized_matmul.rs:232-272), f32 accumulation.
//
// The workgroup organisation of the Q4_K wide kernel (nnq_gemm_wide.hip): eight waves stacked
// along M, 256 rows x NT * 16 columns; each wave owns 32 rows (two 16-row MFMA tiles) across
// all NT column tiles; the activation (staged once per call as f16 of x * 2^s_row, exact for
// bf16 input, fragment-major) is read from L2 straight into registers PD steps ahead, and the
// weight is shared through LDS.
//
// Per 256-k stage (eight 32-k Q8_0 blocks = eight MFMA steps):
//  * the workgroup's 512 threads turn the NT tiles' int8 codes (tile16 image: per tile and
//    stage four 1 KB block pairs, lane 16 p + r holding bytes 8 p .. 8 p + 7 of row r for both
//    blocks) into f16 B fragments in a double-buffered LDS area, ONCE per workgroup: q as the
//    f16 1024 + (q + 128) minus 1152, exact; and the blocks' d (f16, per row and block) as f32;
//  * each step's MFMAs start from zero (their results in VGPRs: the build's VGPR-form option
//    for this file) and every lane adds d(row n, block) * partial to its totals: four FMAs
//    per MFMA, the Q8_0 scale per 32 k that no exact f16 operand can carry (d * q needs up to
//    19 significant bits);
//  * one barrier per stage (lgkmcnt only: the A prefetches stay in flight).
// Epilogue: y = tot * 2^-s_row (+ bias), assembled in LDS and written as 16-byte row chunks;
// with the K range split, f32 slabs summed in order by gemm_finalize_kernel.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

constexpr int WV = 8;             // waves per workgroup (stacked along M)
constexpr int MT = 2;             // 16-row MFMA tiles per wave
constexpr int BM = WV * MT * 16;  // 256 rows per workgroup
constexpr int NTH = WV * 64;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

template <int NT>
struct Wide8 {
    // A-fragment prefetch distance in 32-k steps: a step of two column tiles is only four
    // MFMAs, so the L2 latency of the staged activation needs seven steps (39 against 44 us
    // at 512 x 4096 x 4096 with three); four tiles leave no registers for more than three.
    // The ring of PD + 1 fragments is indexed by the step within the stage, so PD + 1
    // divides the stage's 8 steps.
    static constexpr int PD = NT == 2 ? 7 : 3;
    static_assert(8 % (PD + 1) == 0, "A ring indexed by the step within a stage");
    static constexpr int BN = NT * 16;
    static constexpr int BFRAG = NT * 8 * 1024;  // B fragments of a stage: tiles x steps x 1 KB
    static constexpr int D_OFF = BFRAG;          // d per (tile, column, block), f32
    static constexpr int BUF = D_OFF + NT * 16 * 8 * 4;
    static constexpr int OUT = BM * (BN * 4 + 16);  // the epilogue's f32 tile (rows padded by 16 bytes)
    static constexpr int LDS = 2 * BUF > OUT ? 2 * BUF : OUT;
    // 16-byte code pieces per stage (tile x block pair x lane) and per thread
    static constexpr int NPC = NT * 256, PPT = NPC / NTH;
    static_assert(NPC % NTH == 0, "whole pieces per thread");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
};

struct Wide8Args {
    const uint8_t *qs;     // tile16 code plane
    const uint8_t *hdr;    // d per (tile, stage, row): eight f16
    const u32x4 *xa;       // staged activation, fragment-major [row group][k / 32][16 rows][4 x 16 B]
    const float *rowback;  // [row groups * 16] 2^-s_row
    const float *bias;
    void *y;
    float *ysplit;         // [ks][m][n] f32 slabs when ks > 1
    int y_bf16;
    int m, nst, ntile, ks, nrg;  // nst: 256-k stages per row
    int64_t n;
};

__device__ __forceinline__ uint32_t pk_add(uint32_t a, half2v b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) + b);
}

// the 8 codes of one lane and block (two words, bytes in (e0, e2, e1, e3) order) as the f16
// B slice: the byte q + 128 under the high byte 0x64 is the f16 1024 + q + 128, exact, and
// 1152 is subtracted exactly
__device__ __forceinline__ u32x4 q8_slice(uint32_t w0, uint32_t w1) {
    const half2v off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t k = 0x64646464u, t0 = w0 ^ 0x80808080u, t1 = w1 ^ 0x80808080u;
    return u32x4{pk_add(__builtin_amdgcn_perm(k, t0, 0x04020400u), off), pk_add(__builtin_amdgcn_perm(k, t0, 0x04030401u), off),
                 pk_add(__builtin_amdgcn_perm(k, t1, 0x04020400u), off), pk_add(__builtin_amdgcn_perm(k, t1, 0x04030401u), off)};
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc8(const void *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)min(bytes, (int64_t)0x7FFFFFF0), 0x00020000);
}
__device__ __forceinline__ u32x4 load8(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

template <int NT>
__global__ __launch_bounds__(NTH, 1) void gemm_q80_wide_kernel(Wide8Args a) {
    using C = Wide8<NT>;
    constexpr int PPT = C::PPT, PD = C::PD;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = lane >> 4, c16 = lane & 15;
    const int nst_all = a.nst;

    // tile order: workgroup ids go round-robin over the 8 XCDs, so each XCD gets a contiguous
    // run of T (the column tiles of one row tile: its activation rows shared in that L2)
    const int nct = a.ntile / NT, nrt = (a.m + BM - 1) / BM, total = nct * nrt * a.ks;
    const int bid = (int)blockIdx.x;
    const int T = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
    const int kp = T / (nct * nrt), Tt = T % (nct * nrt);
    const int rt = Tt / nct, ct = Tt % nct;
    const int t0 = ct * NT;
    const int nst = nst_all / a.ks, st0 = kp * nst, nsteps = nst * 8;

    __amdgpu_buffer_rsrc_t ra[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int rg = min(rt * (BM / 16) + wv * MT + mt, a.nrg - 1);
        ra[mt] = rsrc8(a.xa + ((size_t)rg * nst_all * 8 + (size_t)st0 * 8) * 64, (int64_t)nsteps * 1024);
    }
    const int loff = (c16 * 4 + G) * 16;  // lane (G, r) of a fragment: row r's 16 bytes G
    // code pieces of this thread: piece u = tid + NTH * j is tile u >> 8, block pair (u >> 6) & 3
    // (this wave's index & 3), lane u & 63; the first tile is wave-uniform
    const int pair = wv & 3;
    const int tw = __builtin_amdgcn_readfirstlane(tid >> 8);
    const __amdgpu_buffer_rsrc_t rq = rsrc8(a.qs + ((size_t)t0 * nst_all + st0) * 4096, (int64_t)NT * nst_all * 4096);
    const __amdgpu_buffer_rsrc_t rh = rsrc8(a.hdr + ((size_t)t0 * nst_all + st0) * 256, (int64_t)NT * nst_all * 256);
    const bool hdr_lane = pair == 0 && G == 0;  // lanes 0-15 of waves 0 and 4: row c16's eight d
    float bc[NT], rb[MT][4];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) bc[nt] = (a.bias && a.ks == 1) ? a.bias[(int64_t)(t0 + nt) * 16 + c16] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(
            a.rowback + min(rt * BM + wv * 32 + mt * 16, a.nrg * 16 - 16) + 4 * G);
#pragma unroll
        for (int e = 0; e < 4; e++) rb[mt][e] = v[e];
    }

    u32x4 raw[PPT], hd[PPT];
    auto load_raw = [&](int s) {
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            const int t = tw + 2 * j;
            raw[j] = load8(rq, 16 * lane, (t * nst_all + s) * 4096 + pair * 1024);
            if (hdr_lane) hd[j] = load8(rh, 16 * c16, (t * nst_all + s) * 256);
        }
    };
    auto store_piece = [&](unsigned char *buf, int j) {
        const int t = tw + 2 * j;
        // blocks 2 pair and 2 pair + 1 of lane `lane`
        *reinterpret_cast<u32x4 *>(buf + ((t * 8 + 2 * pair) * 64 + lane) * 16) = q8_slice(raw[j][0], raw[j][1]);
        *reinterpret_cast<u32x4 *>(buf + ((t * 8 + 2 * pair + 1) * 64 + lane) * 16) = q8_slice(raw[j][2], raw[j][3]);
        if (hdr_lane) {
            floatx4 d0, d1;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                d0[b] = f16_to_f32((hd[j][b >> 1] >> (16 * (b & 1))) & 0xFFFFu);
                d1[b] = f16_to_f32((hd[j][2 + (b >> 1)] >> (16 * (b & 1))) & 0xFFFFu);
            }
            *reinterpret_cast<floatx4 *>(buf + C::D_OFF + ((t * 16 + c16) * 8) * 4) = d0;
            *reinterpret_cast<floatx4 *>(buf + C::D_OFF + ((t * 16 + c16) * 8 + 4) * 4) = d1;
        }
    };

    floatx4 tot[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) tot[mt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};

    // prologue: stage 0 into buffer 0, the A ring filled
    load_raw(0);
    u32x4 af[PD + 1][MT];
#pragma unroll
    for (int s = 0; s < PD; s++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) af[s][mt] = load8(ra[mt], loff, s * 1024);
#pragma unroll
    for (int j = 0; j < PPT; j++) store_piece(smem, j);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    for (int sb = 0; sb < nst; sb++) {
        const unsigned char *cur = smem + (sb & 1) * C::BUF;
        unsigned char *nxt = smem + ((sb + 1) & 1) * C::BUF;
        const bool more = sb + 1 < nst;
        if (more) load_raw(sb + 1);
        floatx4 dv[NT];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            // A fragments PD steps ahead (past the range: zeros, never used)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) af[(s + PD) % (PD + 1)][mt] = load8(ra[mt], loff, (sb * 8 + s + PD) * 1024);
            __builtin_amdgcn_sched_barrier(0);
            u32x4 bf[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) bf[nt] = *reinterpret_cast<const u32x4 *>(cur + ((nt * 8 + s) * 64 + lane) * 16);
            if ((s & 3) == 0) {
                // d of column c16 for blocks s .. s + 3
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    dv[nt] = *reinterpret_cast<const floatx4 *>(cur + C::D_OFF + ((nt * 16 + c16) * 8 + s) * 4);
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const float d = dv[nt][s & 3];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const floatx4 part = mfma16x16x32_f16(af[s % (PD + 1)][mt], bf[nt], floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int e = 0; e < 4; e++) tot[mt][nt][e] += d * part[e];
                }
            }
            // the next stage's operands into the other buffer (read by nobody since the
            // barrier that ended the previous stage), one piece per odd step
            if (more && (s & 1) && (s >> 1) < PPT) store_piece(nxt, s >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads and writes
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }

    // epilogue: y = tot * 2^-s_row (+ bias), assembled in LDS (every wave is past its last
    // read of the B buffers: the loop's final barrier), 16-byte row chunks
    const bool f32out = a.ks > 1 || !a.y_bf16;
    const int es = f32out ? 4 : 2, rs = C::BN * es + 16;
    if (f32out) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<float *>(smem + (wv * 32 + mt * 16 + 4 * G + e) * rs + (nt * 16 + c16) * 4) =
                        tot[mt][nt][e] * rb[mt][e] + bc[nt];
    } else {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<uint16_t *>(smem + (wv * 32 + mt * 16 + 4 * G + e) * rs + (nt * 16 + c16) * 2) =
                        (uint16_t)f32_to_bf16_bits(tot[mt][nt][e] * rb[mt][e] + bc[nt]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    const int cpr = C::BN * es / 16;  // 16-byte chunks per row
    const int m0 = rt * BM;
    unsigned char *ybase = a.ks > 1 ? reinterpret_cast<unsigned char *>(a.ysplit + (int64_t)kp * a.m * a.n)
                                    : reinterpret_cast<unsigned char *>(a.y);
    for (int c = tid; c < BM * cpr; c += NTH) {
        const int rl = c / cpr, ch = c - rl * cpr;
        if (m0 + rl >= a.m) break;  // rows run in order: the rest are past M as well
        const u32x4 v = *reinterpret_cast<const u32x4 *>(smem + rl * rs + ch * 16);
        *reinterpret_cast<u32x4 *>(ybase + ((int64_t)(m0 + rl) * a.n + (int64_t)t0 * 16) * es + ch * 16) = v;
    }
}

template <int NT>
int launch_nt(const Wide8Args &w, hipStream_t st) {
    using C = Wide8<NT>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q80_wide_kernel<NT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const int total = (w.ntile / NT) * ((w.m + BM - 1) / BM) * w.ks;
    hipLaunchKernelGGL((gemm_q80_wide_kernel<NT>), dim3((unsigned)total), dim3(NTH), C::LDS, st, w);
    return (int)hipGetLastError();
}

}  // namespace

// Shape rules: Q8_0, bf16 activations, more than 128 rows, K a multiple of 256 (whole stages:
// no padded blocks) up to 4096 * 3 (the activation staging), whole 16-row weight tiles and a
// 16-byte aligned output.  Column tiles per workgroup: 4 when that gives at least 192
// workgroups, else 2 (6 would need more than the 256 registers of a lane: its MFMA
// partials, A ring and d's spill); the K range split in two when the workgroups alone would leave
// CUs idle (fewer than 256) and the stages divide evenly.  Returns NT (0: the block kernel
// takes the shape) and the split.
int gemm_wide8_plan(const GemmArgs &a, int *ks) {
    if (a.blk != NNQ_FMT_Q8_0 || !a.x_bf16 || a.m <= 128 || a.k % 256 || a.k > 4096 * 3 ||
        a.n != a.ntile * 16 || (reinterpret_cast<uintptr_t>(a.y) & 15))
        return 0;
    const int64_t nrt = (a.m + BM - 1) / BM, nst = a.k / 256;
    int nt = 0;
    for (int c : {4, 2})
        if (a.ntile % c == 0 && nrt * (a.ntile / c) >= (c == 2 ? 1 : 192)) {
            nt = c;
            break;
        }
    if (!nt) return 0;
    const int64_t wg = nrt * (a.ntile / nt);
    const int split = (wg < 256 && nst % 2 == 0 && nst >= 4) ? 2 : 1;
    if (ks) *ks = split;
    return nt;
}

// scratch: the staged activation | rowback | slabs
size_t gemm_wide8_scratch(const GemmArgs &a, GemmScratch *s, uint8_t *base) {
    auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
    const int64_t nrg = (a.m + 15) / 16;
    int ks = 1;
    gemm_wide8_plan(a, &ks);
    size_t off = 0;
    if (s) s->xh = reinterpret_cast<uint16_t *>(base + off);
    off += al((size_t)nrg * 16 * a.k * 2);
    if (s) {
        s->xs = nullptr;
        s->rowback = reinterpret_cast<float *>(base + off);
    }
    off += al((size_t)nrg * 16 * 4);
    if (s) {
        s->ksplit = ks;
        s->ysplit = nullptr;
    }
    if (ks > 1) {
        if (s) s->ysplit = reinterpret_cast<float *>(base + off);
        off += al((size_t)ks * a.m * a.n * 4);
    }
    return off;
}

int launch_gemm_wide8(const GemmArgs &a, const GemmScratch &sc, void *stream) {
    int ks = 1;
    const int nt = gemm_wide8_plan(a, &ks);
    if (!nt || sc.ksplit != ks || (ks > 1 && !sc.ysplit)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int64_t nrg = (a.m + 15) / 16;
    int e = launch_stage_wide(reinterpret_cast<const uint16_t *>(a.x), a.m, a.k, sc.xh, nullptr, sc.rowback, stream);
    if (e) return e;
    Wide8Args w{};
    w.qs = a.qs;
    w.hdr = a.hdr;
    w.xa = reinterpret_cast<const u32x4 *>(sc.xh);
    w.rowback = sc.rowback;
    w.bias = a.bias;
    w.y = a.y;
    w.ysplit = sc.ysplit;
    w.y_bf16 = a.y_bf16;
    w.m = (int)a.m;
    w.n = a.n;
    w.nst = (int)(a.k / 256);
    w.ntile = (int)a.ntile;
    w.ks = ks;
    w.nrg = (int)nrg;
    e = nt == 4 ? launch_nt<4>(w, st) : launch_nt<2>(w, st);
    if (e || ks == 1) return e;
    return launch_gemm_finalize(sc.ysplit, ks, a.bias, a.y, a.y_bf16, a.m, a.n, stream);
}

}  // namespace nnq
