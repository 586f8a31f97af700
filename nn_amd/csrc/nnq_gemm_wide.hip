// Prefill GEMM for Q4_K weights and bf16 activations on gfx950, wide-wave-tile kernel:
// Y[m, n] = X[m, k] . W[n, k]^T (+ bias), the arithmetic of QLinear::forward with a batch of
// tokens (crates/nn-core/src/layers/quantized/linear.rs:366-400; the bf16 result dtype of
// crates/nn-core/src/dyn_tensor/ops/matmul.rs:37-38).
//
// Workgroup: eight waves stacked along M, 256 rows x NT * 16 columns (NT = 6: 96 columns, one
// workgroup per CU at 512 x 12288; NT = 4 with the K range split in two at 512 x 4096).  Each
// wave owns 32 rows (two 16-row MFMA tiles) across all NT column tiles, so a B fragment read
// from LDS serves two MFMAs and an A fragment NT of them; the activation is the operand with
// the higher reuse and is read from L2 straight into registers, the weight is the one shared
// through LDS.
//
// Per super-block (256 k, eight 32-k MFMA steps):
//  * the B operands sc_j * q of the workgroup's NT weight tiles are dequantized ONCE per
//    workgroup into a double-buffered LDS area, in MFMA fragment order (tile, step, lane,
//    16 bytes), while the MFMAs of the previous super-block run; a thread decodes one or two
//    16-byte pieces of the tile16 code plane (with the row's whole 16-byte header): masked
//    nibble pairs are f16 subnormals q * 2^-24 (low nibbles) or 16 q * 2^-24 (high nibbles),
//    times sc or sc / 16, all exact;
//  * each wave's A fragments come from the fragment-major staged activation (one contiguous
//    1 KB per 16 rows x 32 k, each row's 64 bytes together), PD steps ahead in a register ring;
//  * the super-block's MFMAs accumulate from zero into `part`; after its last step's MFMAs
//    for a column tile every lane adds (d * 2^16 * s_n) * part into its totals `tot`, and
//    the min term is one more MFMA per 16 x 16 tile, issued in the first step of the next
//    super-block: the staged negated sub-block sums of x (f16 hi / lo) against the weight's
//    aux plane (dmin * m_j * s_n as exact f16 hi / lo), accumulated straight into `tot`
//    (both carry the column factor 2^16 * s_n);
//  * one barrier per super-block (lgkmcnt only: the A prefetches stay in flight).
// Epilogue: y = tot * 2^8 / s_n * 2^-s_row (+ bias), assembled in LDS and written as 16-byte
// row chunks; with the K range split, f32 slabs summed in order by gemm_finalize_kernel.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {

namespace {

constexpr int WV = 8;             // waves per workgroup (stacked along M)
constexpr int MT = 2;             // 16-row MFMA tiles per wave
constexpr int BM = WV * MT * 16;  // 256 rows per workgroup
constexpr int NTH = WV * 64;
constexpr int PD = 3;             // A-fragment prefetch distance in 32-k steps

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

template <int NT>
struct Wide {
    static constexpr int BN = NT * 16;
    static constexpr int BFRAG = NT * 8 * 1024;  // dequantized B of a super-block: tiles x steps x 1 KB
    static constexpr int D_OFF = BFRAG;          // d of each column (f32)
    static constexpr int BUF = D_OFF + NT * 16 * 4;
    // min-term B operands (tiles x 1 KB) in a ring of three: the MFMAs that use a
    // super-block's run in the first step of the next one
    static constexpr int AUX_OFF = 2 * BUF, AUXB = NT * 1024;
    static constexpr int LDS = AUX_OFF + 3 * AUXB;
    // 16-byte decode pieces per super-block (tile x group x plane x row), and per thread (the
    // first NPC - NTH * (PPT - 1) threads take one more)
    static constexpr int NPC = NT * 128, PPT = (NPC + NTH - 1) / NTH;
    static_assert(NPC % (NTH / 2) == 0, "each wave pair of a SIMD shares the pieces evenly");
    static_assert(LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");
    // the epilogue tile (bf16 or f32 rows padded by 16 bytes) fits in the two buffers
    static_assert((size_t)BM * (BN * 4 + 16) <= (size_t)LDS, "output tile fits in LDS");
};

struct WideArgs {
    const uint8_t *qs;   // tile16 code plane
    const uint8_t *hdr;  // super-block headers (d, dmin, scales[12]) per (tile, block, row)
    const uint8_t *aux;  // per (tile, block): dmin * m_j * s_n hi | lo (512 B); then s_n per row
    const u32x4 *xa;     // staged activation, fragment-major [row group][k / 32][16 rows][4 x 16 B]
    const u32x4 *xs;     // min-term A operands, fragment-major [row group][k / 256][16 rows][4 x 16 B]
    const float *rowback;  // [row groups * 16] 2^-s_row
    const float *bias;
    void *y;
    float *ysplit;       // [ks][m][n] f32 slabs when ks > 1
    int y_bf16;
    int m, nblk, ntile, ks, nrg;
    int64_t n;
};

// f16 pair product a * (s.lo, s.lo) (HI = 0) or a * (s.hi, s.hi) (HI = 1)
template <int HI>
__device__ __forceinline__ uint32_t pk_mul_bcast(uint32_t a, uint32_t s) {
    const half2v sv = __builtin_bit_cast(half2v, s);
    const half2v b = HI ? half2v{sv[1], sv[1]} : half2v{sv[0], sv[0]};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) * b);
}

// One 16-byte piece of a tile16 group: bytes 16 h .. 16 h + 15 of row r's 32-byte group p,
// which consumer lanes G = 2h and 2h + 1 take 8 bytes each of: their low nibbles are
// k = 64p + 8G + i of sub-block 2p (step 2p), their high nibbles k = 64p + 32 + 8G + i of
// sub-block 2p + 1 (step 2p + 1).  out[g][hh] is the B fragment slice of lane G = 2h + g at
// step 2p + hh.  h is the row's header (BlockQ4K: d | dmin, scales[12]; get_scale_min_k4,
// crates/nn-core/src/layers/quantized/linear.rs:166-176).
__device__ __forceinline__ void decode_piece(u32x4 raw, u32x4 h, int p, u32x4 out[2][2]) {
    const uint32_t sc03 = h[1] & 0x3F3F3F3Fu;
    const uint32_t sc47 = (h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u);
    const uint32_t w = p < 2 ? sc03 : sc47;
    const uint32_t pair = (w >> (16 * (p & 1))) & 0xFFFFu;  // sc_2p | sc_2p+1 << 8
    // f16 (sc_2p, sc_2p+1 / 16): 0x6400 | v is 1024 + v, exact; subtract 1024, scale the high half
    const uint32_t biased = 0x64006400u | (pair & 0xFFu) | ((pair & 0xFF00u) << 8);
    const half2v sh = (__builtin_bit_cast(half2v, biased) - half2v{(_Float16)1024.0f, (_Float16)1024.0f}) *
                      half2v{(_Float16)1.0f, (_Float16)0.0625f};
    const uint32_t sw = __builtin_bit_cast(uint32_t, sh);
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const uint32_t w0 = raw[2 * g], w1 = raw[2 * g + 1], w0s = w0 >> 8, w1s = w1 >> 8;
        out[g][0] = u32x4{pk_mul_bcast<0>(w0 & 0x000F000Fu, sw), pk_mul_bcast<0>(w0s & 0x000F000Fu, sw),
                          pk_mul_bcast<0>(w1 & 0x000F000Fu, sw), pk_mul_bcast<0>(w1s & 0x000F000Fu, sw)};
        out[g][1] = u32x4{pk_mul_bcast<1>(w0 & 0x00F000F0u, sw), pk_mul_bcast<1>(w0s & 0x00F000F0u, sw),
                          pk_mul_bcast<1>(w1 & 0x00F000F0u, sw), pk_mul_bcast<1>(w1s & 0x00F000F0u, sw)};
    }
}

// a buffer resource over [p, p + bytes) (reads past the range return zero)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)min(bytes, (int64_t)0x7FFFFFF0), 0x00020000);
}
__device__ __forceinline__ u32x4 bload4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ u32x2 bload2(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload1(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

template <int NT>
__global__ __launch_bounds__(NTH, 1) void gemm_q4k_wide_kernel(WideArgs a) {
    using C = Wide<NT>;
    constexpr int PPT = C::PPT;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = lane >> 4, c16 = lane & 15;
    const int nblk = a.nblk;

    // Tile order: workgroup ids go round-robin over the 8 XCDs, so each XCD gets a contiguous
    // run of T: the column tiles of one row tile (its activation rows shared in that L2).
    const int nct = a.ntile / NT, nrt = (a.m + BM - 1) / BM, total = nct * nrt * a.ks;
    const int bid = (int)blockIdx.x;
    const int T = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
    const int kp = T / (nct * nrt), Tt = T % (nct * nrt);
    const int rt = Tt / nct, ct = Tt % nct;
    const int t0 = ct * NT;
    const int nsb = nblk / a.ks, sb0 = kp * nsb, nsteps = nsb * 8;

    // Buffer resources over wave-uniform bases; per-lane 32-bit offsets, per-step scalar
    // offsets.  A fragments: the wave's two row groups (past the last: clamped, not stored),
    // steps [sb0 * 8, sb0 * 8 + nsteps); reads past the range (prefetch beyond the end) give 0.
    __amdgpu_buffer_rsrc_t ra[MT], rxs[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int rg = min(rt * (BM / 16) + wv * MT + mt, a.nrg - 1);
        ra[mt] = rsrc(a.xa + ((size_t)rg * nblk * 8 + (size_t)sb0 * 8) * 64, (int64_t)nsteps * 1024);
        rxs[mt] = rsrc(a.xs + ((size_t)rg * nblk + sb0) * 64, (int64_t)nsb * 1024);
    }
    const int loff = (c16 * 4 + G) * 16;  // lane (G, r) of a fragment: row r's 16 bytes G
    // decode pieces of this thread: piece u = tid + NTH * j (j < PPT, u < NPC) is tile u >> 7,
    // group (u >> 5) & 3, plane (u >> 4) & 1, row u & 15
    const int pgp = (tid >> 5) & 3, ph = (tid >> 4) & 1;
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.qs + ((size_t)t0 * nblk + sb0) * 2048, (int64_t)NT * nblk * 2048);
    const __amdgpu_buffer_rsrc_t rh = rsrc(a.hdr + ((size_t)t0 * nblk + sb0) * 256, (int64_t)NT * nblk * 256);
    const __amdgpu_buffer_rsrc_t rx = rsrc(a.aux + ((size_t)t0 * nblk + sb0) * 512, (int64_t)NT * nblk * 512);
    const int qoff = ph * 1024 + (16 * pgp + c16) * 16, hoff = c16 * 16;
    const int xoff = (lane >> 5) * 256 + c16 * 16;
    const int tw = __builtin_amdgcn_readfirstlane(tid >> 7);  // tile of this thread's first piece
    // per column: 2^16 * s_n, the totals' unit (s_n a normal power of two), and the epilogue's
    // factors, loaded now: 2^8 / s_n and the bias per column, 2^-s_row per row
    const float *srow = reinterpret_cast<const float *>(a.aux + (size_t)a.ntile * nblk * 512);
    float f1[NT], f2[NT], bc[NT], rb[MT][4];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const uint32_t eb = __float_as_uint(srow[(size_t)(t0 + nt) * 16 + c16]) >> 23;
        f1[nt] = __uint_as_float((eb + 16u) << 23);
        f2[nt] = __uint_as_float((262u - eb) << 23);
        bc[nt] = (a.bias && a.ks == 1) ? a.bias[(int64_t)(t0 + nt) * 16 + c16] : 0.0f;
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        // rows 4G .. 4G + 3 of the tile: one 16-byte load (the rowback plane is padded to 16 rows)
        const floatx4 v = *reinterpret_cast<const floatx4 *>(
            a.rowback + min(rt * BM + wv * 32 + mt * 16, a.nrg * 16 - 16) + 4 * G);
#pragma unroll
        for (int e = 0; e < 4; e++) rb[mt][e] = v[e];
    }

    // the next super-block's raw operands (issued one super-block ahead)
    u32x4 raw[PPT], hd[PPT];
    u32x4 auxv;
    auto load_raw = [&](int sb) {
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            if (tid + NTH * j < C::NPC) {
                const int t = tw + 4 * j;
                raw[j] = bload4(rq, qoff, (t * nblk + sb) * 2048);
                hd[j] = bload4(rh, hoff, (t * nblk + sb) * 256);
            }
        }
        if (wv < NT) auxv = bload4(rx, xoff, (wv * nblk + sb) * 512);
    };
    auto store_piece = [&](unsigned char *buf, int j) {
        if (tid + NTH * j >= C::NPC) return;
        const int t = tw + 4 * j;
        u32x4 o[2][2];
        // the header's third word is not needed, but its register must stay allocated until
        // here: reused as a temporary while the load is in flight, it would make the wave
        // wait for that (HBM-latency) load at once
        asm volatile("" ::"v"(hd[j][2]));
        decode_piece(raw[j], hd[j], pgp, o);
#pragma unroll
        for (int g = 0; g < 2; g++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
                *reinterpret_cast<u32x4 *>(buf + ((t * 8 + 2 * pgp + hh) * 64 + 16 * (2 * ph + g) + c16) * 16) = o[g][hh];
        if (pgp == 0 && ph == 0) *reinterpret_cast<float *>(buf + C::D_OFF + (t * 16 + c16) * 4) = f16_to_f32(hd[j][0] & 0xFFFFu);
    };

    floatx4 tot[MT][NT], part[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) tot[mt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};

    // prologue: super-block 0 into buffer 0, the A ring filled
    load_raw(0);
    u32x4 af[PD + 1][MT];
#pragma unroll
    for (int s = 0; s < PD; s++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) af[s][mt] = bload4(ra[mt], loff, s * 1024);
#pragma unroll
    for (int j = 0; j < PPT; j++) store_piece(smem, j);
    if (wv < NT) *reinterpret_cast<u32x4 *>(smem + C::AUX_OFF + (wv * 64 + lane) * 16) = auxv;
    u32x4 xsp_prev[MT];  // the previous super-block's min-term A operands
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // the min term of super-block b: one MFMA per 16 x 16 tile into the totals
    auto min_term = [&](int b, const u32x4 *xsv) {
        const unsigned char *ab = smem + C::AUX_OFF + (b % 3) * C::AUXB;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const u32x4 auxf = *reinterpret_cast<const u32x4 *>(ab + (nt * 64 + lane) * 16);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) tot[mt][nt] = mfma16x16x32_f16(xsv[mt], auxf, tot[mt][nt]);
        }
    };

    for (int sb = 0; sb < nsb; sb++) {
        unsigned char *cur = smem + (sb & 1) * C::BUF;
        unsigned char *nxt = smem + ((sb + 1) & 1) * C::BUF;
        const bool more = sb + 1 < nsb;
        if (more) load_raw(sb + 1);
        u32x4 xsf[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) xsf[mt] = bload4(rxs[mt], loff, sb * 1024);
        float dn[NT];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            // A fragments PD steps ahead (past the range: zeros, never used)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) af[(s + PD) % (PD + 1)][mt] = bload4(ra[mt], loff, (sb * 8 + s + PD) * 1024);
            __builtin_amdgcn_sched_barrier(0);
            u32x4 bf[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) bf[nt] = *reinterpret_cast<const u32x4 *>(cur + ((nt * 8 + s) * 64 + lane) * 16);
            if (s == 0 && sb > 0) min_term(sb - 1, xsp_prev);
            if (s == 6) {
                // the super-block's factor d per column (2^16 * s_n folded in)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    dn[nt] = *reinterpret_cast<const float *>(cur + C::D_OFF + (nt * 16 + c16) * 4) * f1[nt];
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    part[mt][nt] = mfma16x16x32_f16(af[s % (PD + 1)][mt], bf[nt],
                                                    s == 0 ? floatx4{0.f, 0.f, 0.f, 0.f} : part[mt][nt]);
                if (s == 7) {
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
#pragma unroll
                        for (int e = 0; e < 4; e++) tot[mt][nt][e] += dn[nt] * part[mt][nt][e];
                }
            }
            // the next super-block's operands into the other buffer (read by nobody since
            // the barrier that ended the previous super-block), one piece every other step;
            // its min-term operands into the ring slot last read two super-blocks ago
            if (more && (s == 3 || s == 5) && (s >> 2) < PPT) store_piece(nxt, s >> 2);
            if (more && s == 5 && wv < NT)
                *reinterpret_cast<u32x4 *>(smem + C::AUX_OFF + ((sb + 1) % 3) * C::AUXB + (wv * 64 + lane) * 16) = auxv;
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) xsp_prev[mt] = xsf[mt];
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads and writes
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }
    min_term(nsb - 1, xsp_prev);
    // every wave has read the aux ring before the output tile (f32: over the ring) is written
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();

    // epilogue: y = tot * 2^8 / s_n * 2^-s_row (+ bias), assembled in LDS, 16-byte row chunks
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
                        tot[mt][nt][e] * f2[nt] * rb[mt][e] + bc[nt];
    } else {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<uint16_t *>(smem + (wv * 32 + mt * 16 + 4 * G + e) * rs + (nt * 16 + c16) * 2) =
                        (uint16_t)f32_to_bf16_bits(tot[mt][nt][e] * f2[nt] * rb[mt][e] + bc[nt]);
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

// ---------------------------------------------------------------------------------
// Skinny GEMM (17 .. 32 rows, bf16 activations; up to 16 rows take the one-launch thin
// kernel of nnq_gemm_thin.hip): the weight is streamed once, like a decode GEMV.  One workgroup per R consecutive weight tiles (16 columns each); its W waves split
// K by units of 256 (unit u to wave u % W).  Each wave runs all MT row tiles of the batch
// against its R tiles: it dequantizes its B fragments in registers straight from the tile16
// bytes (the wide kernel's exact sc * q operands, here without any LDS or barrier in the
// loop), shares every A fragment (the same staged activation planes) across the R tiles,
// and keeps the d-scaled totals and the min term as the wide kernel does.  The raw bytes of
// a wave's next unit are loaded while it computes the current one.  At the end the waves'
// totals meet in LDS and the workgroup writes its M x 16 R outputs.
// ---------------------------------------------------------------------------------
template <int R, int MT, int W>
struct Skinny {
    static constexpr int LDS = W * R * MT * 1024;  // every wave's totals, f32
};

template <int R, int MT, int W>
__global__ __launch_bounds__(W * 64) void gemm_q4k_skinny_kernel(WideArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = lane >> 4, c16 = lane & 15;
    const int nblk = a.nblk;
    const int t0 = (int)blockIdx.x * R;  // the plan keeps ntile % R == 0

    __amdgpu_buffer_rsrc_t ra[MT], rxs[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int rg = min(mt, a.nrg - 1);
        ra[mt] = rsrc(a.xa + (size_t)rg * nblk * 8 * 64, (int64_t)nblk * 8 * 1024);
        rxs[mt] = rsrc(a.xs + (size_t)rg * nblk * 64, (int64_t)nblk * 1024);
    }
    const int loff = (c16 * 4 + G) * 16;  // lane (G, r) of a fragment: row r's 16 bytes G
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.qs + (size_t)t0 * nblk * 2048, (int64_t)R * nblk * 2048);
    const __amdgpu_buffer_rsrc_t rh = rsrc(a.hdr + (size_t)t0 * nblk * 256, (int64_t)R * nblk * 256);
    const __amdgpu_buffer_rsrc_t rx = rsrc(a.aux + (size_t)t0 * nblk * 512, (int64_t)R * nblk * 512);
    // consumer lane (G, r) of group p takes bytes 8G .. 8G + 7 of row r's group: plane G >> 1,
    // chunk 16 p + r, half G & 1
    const int qoff = (G >> 1) * 1024 + c16 * 16 + 8 * (G & 1), hoff = c16 * 16;
    const int xoff = (lane >> 5) * 256 + c16 * 16;
    const float *srow = reinterpret_cast<const float *>(a.aux + (size_t)a.ntile * nblk * 512);
    float f1[R];
#pragma unroll
    for (int r = 0; r < R; r++)
        f1[r] = __uint_as_float(((__float_as_uint(srow[(size_t)(t0 + r) * 16 + c16]) >> 23) + 16u) << 23);

    struct Raw {
        u32x2 q[R][4];
        u32x4 h[R], x[R];
    };
    auto load_raw = [&](int u, Raw &w) {
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int p = 0; p < 4; p++) w.q[r][p] = bload2(rq, qoff + 256 * p, (r * nblk + u) * 2048);
            w.h[r] = bload4(rh, hoff, (r * nblk + u) * 256);
            w.x[r] = bload4(rx, xoff, (r * nblk + u) * 512);
        }
    };

    floatx4 tot[R][MT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) tot[r][mt] = floatx4{0.f, 0.f, 0.f, 0.f};

    // the unit body: unit u from the raw bytes `cur`; each step loads its A fragments
    auto unit = [&](int u, const Raw &cur) {
        u32x4 xsf[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) xsf[mt] = bload4(rxs[mt], loff, u * 1024);
        // f16 (sc_j, sc_j+1 / 16) per tile and group
        uint32_t sw[R][4];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const u32x4 h = cur.h[r];
            const uint32_t sc03 = h[1] & 0x3F3F3F3Fu;
            const uint32_t sc47 = (h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint32_t pair = ((p < 2 ? sc03 : sc47) >> (16 * (p & 1))) & 0xFFFFu;
                const uint32_t biased = 0x64006400u | (pair & 0xFFu) | ((pair & 0xFF00u) << 8);
                const half2v sh = (__builtin_bit_cast(half2v, biased) - half2v{(_Float16)1024.0f, (_Float16)1024.0f}) *
                                  half2v{(_Float16)1.0f, (_Float16)0.0625f};
                sw[r][p] = __builtin_bit_cast(uint32_t, sh);
            }
        }
        floatx4 part[R][MT];
        u32x4 af[MT];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int p = s >> 1;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) af[mt] = bload4(ra[mt], loff, (u * 8 + s) * 1024);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t w0 = cur.q[r][p][0], w1 = cur.q[r][p][1], w0s = w0 >> 8, w1s = w1 >> 8;
                u32x4 b;
                if ((s & 1) == 0)
                    b = u32x4{pk_mul_bcast<0>(w0 & 0x000F000Fu, sw[r][p]), pk_mul_bcast<0>(w0s & 0x000F000Fu, sw[r][p]),
                              pk_mul_bcast<0>(w1 & 0x000F000Fu, sw[r][p]), pk_mul_bcast<0>(w1s & 0x000F000Fu, sw[r][p])};
                else
                    b = u32x4{pk_mul_bcast<1>(w0 & 0x00F000F0u, sw[r][p]), pk_mul_bcast<1>(w0s & 0x00F000F0u, sw[r][p]),
                              pk_mul_bcast<1>(w1 & 0x00F000F0u, sw[r][p]), pk_mul_bcast<1>(w1s & 0x00F000F0u, sw[r][p])};
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    part[r][mt] = mfma16x16x32_f16(af[mt], b, s == 0 ? floatx4{0.f, 0.f, 0.f, 0.f} : part[r][mt]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float dn = f16_to_f32(cur.h[r][0] & 0xFFFFu) * f1[r];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int e = 0; e < 4; e++) tot[r][mt][e] += dn * part[r][mt][e];
                tot[r][mt] = mfma16x16x32_f16(xsf[mt], cur.x[r], tot[r][mt]);
            }
        }
    };
    // this wave's units wv, wv + W, ...
    const int nu = nblk > wv ? (nblk - wv + W - 1) / W : 0;
    // one unit's raw bytes ahead
    Raw cur, nxt;
    if (nu > 0) load_raw(wv, cur);
    for (int i = 0; i < nu; i++) {
        if (i + 1 < nu) load_raw(wv + (i + 1) * W, nxt);
        unit(wv + i * W, cur);
        if (i + 1 < nu) cur = nxt;
    }
    // the waves' totals meet in LDS: [W][R][MT][64 lanes] floatx4
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            *reinterpret_cast<floatx4 *>(smem + ((((wv * R + r) * MT + mt) * 64) + lane) * 16) = tot[r][mt];
    __syncthreads();
    // thread (r, mt, lane) for the first R * MT * 64 threads: sum over the waves, epilogue
    for (int i = tid; i < R * MT * 64; i += W * 64) {
        const int l = i & 63, rm = i >> 6, r = rm / MT, mt = rm % MT;
        floatx4 v = *reinterpret_cast<const floatx4 *>(smem + (rm * 64 + l) * 16);
#pragma unroll
        for (int w2 = 1; w2 < W; w2++) v += *reinterpret_cast<const floatx4 *>(smem + (((w2 * R * MT) + rm) * 64 + l) * 16);
        const int lg = l >> 4, col = (t0 + r) * 16 + (l & 15);
        if (col >= a.n) continue;  // the padded rows of a last, partial weight tile
        const float f2 = __uint_as_float((262u - (__float_as_uint(srow[col]) >> 23)) << 23);
        const float bc = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int row = mt * 16 + 4 * lg + e;
            if (row < a.m) {
                const float y = v[e] * f2 * a.rowback[row] + bc;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[(int64_t)row * a.n + col] = (uint16_t)f32_to_bf16_bits(y);
                else
                    reinterpret_cast<float *>(a.y)[(int64_t)row * a.n + col] = y;
            }
        }
    }
}

// ---------------------------------------------------------------------------------
// Activation staging for the wide kernel: one workgroup of 512 threads per row, the row
// loaded at once into registers (NG groups of 8 per thread, K <= 4096 NG), its max found by
// wave reductions and one exchange through LDS, then written as f16 of x * 2^s_row (exact
// for bf16 input) into the fragment-major plane: fragment (row group g, step s) is 1 KB, row
// r's 64 bytes at 64 r, so that the 16 bytes of MFMA lane 16 G + r,
// x[16 g + r][32 s + 8 G .. + 7], sit at 64 r + 16 G (four consecutive threads store one
// 64-byte segment).  The min-term operands: per (row group, super-block) one fragment in
// the same order whose lane 16 G + r holds the f16 hi (G even) or lo (G odd) parts of
// -2^-8 * sum(x * 2^s_row) over the row's eight 32-element sub-blocks.  Rows past M
// (padding to 16) are written as zeros.
// ---------------------------------------------------------------------------------
template <int NG, bool XS>
__global__ __launch_bounds__(512) void gemm_stage_wide_kernel(const uint16_t *x, int64_t m, int64_t k, u32x4 *xa,
                                                              u32x4 *xs, float *rowback) {
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wvi = tid >> 6;
    __shared__ float wred[8];
    __shared__ float sums[NG * 128];  // the row's sub-block sums (k / 32 <= 128 NG)
    const bool valid = row < m;
    const int64_t ng = k / 8, nks = k / 32;
    const int g = (int)(row >> 4), r = (int)(row & 15);
    u32x4 w[NG];
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int64_t c = tid + 512 * j;
        w[j] = (valid && c < ng) ? *reinterpret_cast<const u32x4 *>(x + row * k + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NG; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            amax = fmaxf(amax, fmaxf(fabsf(bf16_to_f32(w[j][i] & 0xFFFFu)), fabsf(bf16_to_f32(w[j][i] >> 16))));
    amax = wave_max(amax);
    if (lane == 0) wred[wvi] = amax;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, wred[i]);
    float s, back;
    f16_prescale(amax, s, back);
    if (tid == 0) rowback[row] = valid ? back : 1.0f;
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int64_t c = tid + 512 * j;  // chunk of 8: step c / 4, lane group c % 4
        if (j * 512 < ng) {               // wave-uniform: whole groups of 64 chunks (k % 512 == 0)
            uint32_t h[4];
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a0 = bf16_to_f32(w[j][i] & 0xFFFFu) * s, a1 = bf16_to_f32(w[j][i] >> 16) * s;
                sum += a0 + a1;
                h[i] = f32_to_f16_bits(a0) | (f32_to_f16_bits(a1) << 16);
            }
            // the sub-block's sum over its four chunks (lanes c .. c + 3 of one quad)
            sum += dpp_xor1(sum);
            sum += dpp_xor2(sum);
            if (c < ng) {
                xa[((int64_t)g * nks + c / 4) * 64 + r * 4 + (c % 4)] = u32x4{h[0], h[1], h[2], h[3]};
                if ((c & 3) == 0) sums[c / 4] = sum;
            }
        }
    }
    if constexpr (!XS) return;  // no min-term operands (Q8_0)
    __syncthreads();
    // min-term fragments: lane group G of super-block b: part G & 1 of -2^-8 * sum, 8 sub-blocks
    const int64_t nsb = k / 256;
    for (int64_t i = tid; i < nsb * 4; i += 512) {
        const int64_t b = i >> 2;
        const int G = (int)(i & 3);
        uint32_t h[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t hl[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                uint32_t hi, lo;
                split_f16(-0.00390625f * sums[b * 8 + 2 * q + e], hi, lo);
                hl[e] = (G & 1) ? lo : hi;
            }
            h[q] = hl[0] | (hl[1] << 16);
        }
        xs[((int64_t)g * nsb + b) * 64 + r * 4 + G] = u32x4{h[0], h[1], h[2], h[3]};
    }
}

}  // namespace

// The wide kernel's shape rules: bf16 activations, more than 128 rows (smaller batches are
// HBM-bound and take the other kernels), whole 16-row weight tiles and a 16-byte aligned
// output (the epilogue writes 16-byte row chunks), K <= 4096 * 3 (the staging
// keeps the row in one workgroup's registers and its sub-block sums in LDS), and enough workgroups to fill
// the CUs: 96-column tiles when they give at least 192 workgroups, else 64-column tiles
// (an even super-block count) when they give 128 with the K range split in two below 256.
// Returns the column tiles per workgroup (6 or 4; 0: the ring kernel takes the shape) and
// the K split.
int gemm_wide_plan(const GemmArgs &a, int *ks) {
    if (a.blk || !a.x_bf16 || a.m <= 128 || a.k > 4096 * 3 || a.n != a.ntile * 16 ||
        (reinterpret_cast<uintptr_t>(a.y) & 15))
        return 0;
    const int64_t nrt = (a.m + BM - 1) / BM;
    if (a.ntile % 6 == 0 && nrt * (a.ntile / 6) >= 192) {
        if (ks) *ks = 1;
        return 6;
    }
    if (a.ntile % 4 == 0) {
        const int64_t wg = nrt * (a.ntile / 4);
        const int split = wg >= 256 ? 1 : 2;
        if (wg * split >= 128 && a.nblk % split == 0 && a.nblk / split >= 2) {
            if (ks) *ks = split;
            return 4;
        }
    }
    return 0;
}

// The skinny kernel's shape rules: bf16 activations, 17 to 32 rows (fewer: the thin
// kernel), K <= 4096 * 3 (the staging), R = 3 tiles per workgroup giving at least 192
// workgroups (with one tile per workgroup every workgroup reads the whole staged
// activation: there, and at 48 and 64 rows, the ring kernel measured as fast or faster
// on MI355X).  W = 8 waves over K (measured against 4).  Returns 1 when the kernel takes
// the shape.
int gemm_skinny_plan(const GemmArgs &a, int *R, int *W) {
    if (a.blk || !a.x_bf16 || a.m <= 16 || a.m > 32 || a.k > 4096 * 3) return 0;
    if (a.ntile % 3 != 0 || a.ntile / 3 < 192) return 0;
    if (R) *R = 3;
    if (W) *W = 8;
    return 1;
}

size_t gemm_wide_scratch(const GemmArgs &a, GemmScratch *s, uint8_t *base) {
    auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
    const int64_t nrg = (a.m + 15) / 16;
    int ks = 1;
    if (!gemm_skinny_plan(a, nullptr, nullptr)) gemm_wide_plan(a, &ks);
    size_t off = 0;
    if (s) s->xh = reinterpret_cast<uint16_t *>(base + off);
    off += al((size_t)nrg * 16 * a.k * 2);
    if (s) s->xs = reinterpret_cast<uint16_t *>(base + off);
    off += al((size_t)nrg * (a.k / 256) * 1024);
    if (s) s->rowback = reinterpret_cast<float *>(base + off);
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

template <int NT>
static int launch_wide_nt(const WideArgs &w, hipStream_t st) {
    using C = Wide<NT>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_wide_kernel<NT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    const int total = (w.ntile / NT) * ((w.m + BM - 1) / BM) * w.ks;
    hipLaunchKernelGGL((gemm_q4k_wide_kernel<NT>), dim3((unsigned)total), dim3(NTH), C::LDS, st, w);
    return (int)hipGetLastError();
}

template <int R, int MT, int W>
static int launch_skinny_cfg(const WideArgs &w, hipStream_t st) {
    using C = Skinny<R, MT, W>;
    static bool attr_set = false;  // idempotent attribute write; races only repeat it
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_skinny_kernel<R, MT, W>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
        if (e != hipSuccess) return (int)e;
        attr_set = true;
    }
    hipLaunchKernelGGL((gemm_q4k_skinny_kernel<R, MT, W>), dim3((unsigned)(w.ntile / R)), dim3(W * 64), C::LDS, st, w);
    return (int)hipGetLastError();
}

int launch_stage_wide(const uint16_t *x, int64_t m, int64_t k, void *xa, void *xs, float *rowback, void *stream) {
    const dim3 sg((unsigned)((m + 15) / 16 * 16));
    hipStream_t st = (hipStream_t)stream;
    auto fa = reinterpret_cast<u32x4 *>(xa), fs = reinterpret_cast<u32x4 *>(xs);
    if (k > 4096 * 3 || k % 256) return (int)hipErrorInvalidValue;
    if (k <= 4096) {
        if (xs)
            hipLaunchKernelGGL((gemm_stage_wide_kernel<1, true>), sg, dim3(512), 0, st, x, m, k, fa, fs, rowback);
        else
            hipLaunchKernelGGL((gemm_stage_wide_kernel<1, false>), sg, dim3(512), 0, st, x, m, k, fa, fs, rowback);
    } else {
        if (xs)
            hipLaunchKernelGGL((gemm_stage_wide_kernel<3, true>), sg, dim3(512), 0, st, x, m, k, fa, fs, rowback);
        else
            hipLaunchKernelGGL((gemm_stage_wide_kernel<3, false>), sg, dim3(512), 0, st, x, m, k, fa, fs, rowback);
    }
    return (int)hipGetLastError();
}

int launch_gemm_wide(const GemmArgs &a, const GemmScratch &sc, void *stream) {
    int ks = 0, sr = 0, sw = 0;
    const bool skinny = gemm_skinny_plan(a, &sr, &sw);
    const int nt = skinny ? 0 : gemm_wide_plan(a, &ks);
    if (!skinny && (!nt || sc.ksplit != ks || (ks > 1 && !sc.ysplit))) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int64_t nrg = (a.m + 15) / 16;
    auto xa = reinterpret_cast<u32x4 *>(sc.xh);
    auto xs = reinterpret_cast<u32x4 *>(sc.xs);
    auto xin = reinterpret_cast<const uint16_t *>(a.x);
    int e = launch_stage_wide(xin, a.m, a.k, xa, xs, sc.rowback, stream);
    if (e) return e;
    WideArgs w{};
    w.qs = a.qs;
    w.hdr = a.hdr;
    w.aux = a.aux;
    w.xa = xa;
    w.xs = xs;
    w.rowback = sc.rowback;
    w.bias = a.bias;
    w.y = a.y;
    w.ysplit = sc.ysplit;
    w.y_bf16 = a.y_bf16;
    w.m = (int)a.m;
    w.n = a.n;
    w.nblk = (int)a.nblk;
    w.ntile = (int)a.ntile;
    w.ks = skinny ? 1 : ks;
    w.nrg = (int)nrg;
    if (skinny) {
        return launch_skinny_cfg<3, 2, 8>(w, st);  // the plan: 17 to 32 rows, three tiles, eight waves
    }
    e = nt == 6 ? launch_wide_nt<6>(w, st) : launch_wide_nt<4>(w, st);
    if (e || ks == 1) return e;
    return launch_gemm_finalize(sc.ysplit, ks, a.bias, a.y, a.y_bf16, a.m, a.n, stream);
}

}  // namespace nnq
