// Internal declarations shared by the C-ABI implementation, the host repack
// code and the HIP kernels.  Not part of the public ABI.
//
// Device weight layout ("tile16"): rows are grouped in tiles of 16 (the N side
// of a 16x16xK MFMA).  For every (tile, K-chunk) the quantized bytes of the 16
// rows are stored so that one wave-wide 16-byte load puts exactly the MFMA
// B-operand bytes of lane l = 16*p + n (row n of the tile, k-group p) into that
// lane, and each 4-byte word is byte-permuted (e0,e2,e1,e3) so that masking
// yields packed-f16 pairs in natural k order.  Scale/header bytes live in a
// separate plane per (tile, block).  The repack is a bijection on the block
// bytes: device bytes == host bytes except for zero padding of the last tile.
#pragma once

#include <cstddef>
#include <cstdint>

#include "../../include/nnq.h"

namespace nnq {

constexpr int kTile = 16;  // rows per tile

// ---- per-format device layout geometry --------------------------------------------
struct Layout {
    int fmt = 0;        // nnq_format
    int layout = 0;     // nnq_layout of the source bytes
    int64_t n = 0, k = 0;
    int64_t ntile = 0;  // ceil(n/16)
    int64_t nblk = 0;   // format blocks per row after padding (Q8_0: padded to a multiple of 8)
    size_t qs_bytes = 0;   // bytes of the quant plane
    size_t hdr_bytes = 0;  // bytes of the scale/header plane
    size_t aux_bytes = 0;  // bytes of the derived plane (Q4_K: min-term operands of the GEMM)
    size_t total() const { return qs_bytes + hdr_bytes + aux_bytes; }
};

// Q4_K: per (tile, block of 256): qs 2048 B (two 1 KB planes; lane 16p + r of plane h
//       holds bytes [16h, 16h + 16) of row r's 32-byte group p, i.e. the nibbles of
//       sub-blocks 2p (low) and 2p + 1 (high)), header 16 rows x 16 B (d, dmin,
//       scales[12] in GGUF-spec packing).
//       aux (derived from the headers for the prefill GEMM): per (tile, block) 512 B =
//       16 rows x 8 f16 hi parts, then 16 x 8 lo parts, of dmin * m_j * s_row (exact as
//       hi + lo: 17 significant bits); then per row one f32 s_row, the power of two that
//       puts max_b |dmin_b| * 63 in [2^14, 2^15).
// Q8_0: per (tile, block pair): qs 1024 B; per (tile, 8 blocks): 16 rows x 8 f16 scales.
// Q6_K: per (tile, block of 256): qs 3072 B (four 64-k chunks x 64 lanes x 12 B),
//       header 16 rows x 16 int8 scales + 16 rows x f16 d (288 B).
bool make_layout(int fmt, int layout, int64_t n, int64_t k, Layout *out, const char **err);

// Host repack: source block bytes (format/layout as given) -> device image (Layout::total bytes).
void repack_q4k(const uint8_t *src, int legacy, const Layout &L, uint8_t *dst);
void repack_q8_0(const uint8_t *src, const Layout &L, uint8_t *dst);
void repack_q6k(const uint8_t *src, const Layout &L, uint8_t *dst);

// nn-gguf legacy Q4_K block -> GGUF-spec (BlockQ4K) block with identical decoded values.
void q4k_legacy_to_gguf(const uint8_t *legacy, uint8_t *gguf);
// Q4_K aux plane of tiles [t0, t1) from the device header plane (GGUF-spec headers).
void q4k_aux_plane(const uint8_t *hdr, const Layout &L, uint8_t *aux, int64_t t0, int64_t t1);

// the calling thread's last-error message (nnq_last_error); returns `code`
int set_error(int code, const char *msg);

// ---- host arithmetic of the ABI calls (nnq_plan.cpp) -------------------------------
// token-expert assignments per MoE launch sequence; longer batches run in token chunks
constexpr int64_t kMoeChunkAssign = 16384;
size_t align256(size_t v);
// rows * cols * elem bytes; false when negative or beyond size_t
bool array_bytes(int64_t rows, int64_t cols, size_t elem, size_t *out);
// regions one after another, each at a 256-byte boundary (a zero size takes no space):
// offsets[i] and the total; false on size_t overflow
bool plan_regions(const size_t *sizes, int n, size_t *offsets, size_t *total);
// tokens per MoE launch sequence (at most kMoeChunkAssign / top_k, at least 1)
int64_t moe_chunk_tokens(int64_t tokens, int top_k);
// rows per prefill-GEMM launch: the kernels' 32-bit activation offsets need
// 4 * rows * k < 2^31
int64_t gemm_chunk_rows(int64_t m, int64_t k);

// ---- kernel launch parameters ------------------------------------------------------
struct GemvArgs {
    const uint8_t *qs;    // quant plane
    const uint8_t *hdr;   // header plane
    const void *x;        // [m, k] f32 or bf16
    int x_bf16;
    const float *bias;    // [n] or null
    void *y;              // [m, n] f32 or bf16
    int y_bf16;
    int64_t n, k, m;
    int64_t ntile, nblk;
    int kc;               // K elements staged in LDS per chunk (multiple of 256)
    float *logits_out;    // optional copy (argmax fusion)
    unsigned long long *argmax_partial;  // optional per-tile (orderable value, index) keys
    int64_t *argmax_count;  // with argmax_partial: the launch stores how many keys it writes
                            //   (one per tile, or one per workgroup of a streaming kernel)
    int x_swiglu;         // x is f32 [m, 2k] (gate | up); the GEMV input is silu(gate) * up (m <= 2)
    int swiglu_out;       // Q4_K, m <= 2: rows come as 8 gate rows then the 8 matching up rows per
                          //   16-row tile; y [m, n / 2] gets silu(gate) * up (no bias, no argmax)
    int32_t *status;      // optional: status_mode 1 stores NNQ_OK (one thread), 2 stores
    int status_mode;      //   NNQ_ERR_NON_FINITE when an output is NaN or infinite
};

int launch_gemv(int fmt, const GemvArgs &a, void *stream);      // returns hipError_t
int launch_dequant(int fmt, const uint8_t *qs, const uint8_t *hdr, int64_t n, int64_t k, int64_t ntile,
                   int64_t nblk, float *out, void *stream);
int launch_argmax_reduce(const float *v, int64_t n, uint32_t *idx, int32_t *status, void *scratch,
                         size_t scratch_bytes, void *stream);
int launch_argmax_final(const unsigned long long *partial, int64_t count, uint32_t *idx, int32_t *status,
                        void *stream);
// MLP glue: h = silu(gate) * up from gu [m, 2 * inter] (gate | up halves, or with
// interleaved8 the 8-gate-rows / 8-up-rows order of each 16 columns; clears *status when
// given), and the non-finite output check (sets *status to NNQ_ERR_NON_FINITE)
int launch_swiglu(const float *gu, int64_t m, int64_t inter, float *h, int32_t *status, void *stream,
                  int interleaved8 = 0);
int launch_nonfinite_check(const void *y, int y_bf16, int64_t count, int32_t *status, void *stream);

// Token sampling over device logits[n] (k = min(top_k, n), 0: none): scratch bytes, whether
// the device path takes the shape (any k, n < 2^32), whether it fits the two-pass top-k
// (ceil(n / 2048) * min(k, 2048) <= 16384; else every key is sorted), and the launch
size_t sample_scratch_bytes(int64_t n, int64_t k);
bool sample_supported(int64_t n, int64_t k);
bool sample_two_pass(int64_t n, int64_t k);
// The fixed per-device scratch of nnq_linear_sample_noalloc: its size, and its device
// address on the current device (looked up once per device; returns a hipError_t).
constexpr size_t kSampleStaticScratchBytes = 384 * 1024;
int sample_static_scratch(void **out);
// keep_inf: top_k is None, so +inf logits are candidates too (k = n)
int launch_sample(const float *logits, int64_t n, const uint32_t *past, int64_t n_past, float temperature, int64_t k,
                  int keep_inf, int use_top_p, float top_p, float rep, int rep_on, float freq, int freq_on,
                  uint64_t seed, uint32_t *token, void *scratch, void *stream);

// GEMM (prefill) for Q4_K: x bf16/f32 [m, k] -> y [m, n].  `scratch` holds the
// staged activation and split-K partials (gemm_scratch_bytes(args) bytes, 256-byte
// aligned; every field but scratch set).
struct GemmArgs {
    const uint8_t *qs;
    const uint8_t *hdr;
    const uint8_t *aux;
    const void *x;
    int x_bf16;
    const float *bias;
    void *y;
    int y_bf16;
    int64_t n, k, m;
    int64_t ntile, nblk;
    void *scratch;
    int blk;  // 0: Q4_K; NNQ_FMT_Q8_0 / NNQ_FMT_Q6_K: the block-scaled GEMM (nnq_gemm_blk.hip)
};
int launch_gemm_q4k(const GemmArgs &a, void *stream);
// one-launch Q4_K GEMM for a few bf16 token rows (nnq_gemm_thin.hip): whether it takes
// the shape (R, W: tiles per workgroup and waves), and its launch; no scratch
int gemm_thin_plan(const GemmArgs &a, int *R, int *W);
int launch_gemm_thin(const GemmArgs &a, void *stream);
// Q8_0 / Q6_K prefill GEMM (M > 8): the activation staging below, then one kernel
int launch_gemm_blk(const GemmArgs &a, void *stream);
// its K split (and tile height and width, when bm / bn are given)
int gemm_blk_plan(const GemmArgs &a, int *bm, int *bn = nullptr);
size_t gemm_scratch_bytes(const GemmArgs &a);
// staged activation (gemm_prep_kernel): P = 1 (bf16 x) or 2 (f32 x, hi + lo planes)
struct GemmScratch {
    uint16_t *xh;      // [P][m][k] f16 of x * 2^s_row
    uint16_t *xs;      // [2][m][k / 32] f16 hi / lo of 2^-8 * sum(x * 2^s_row) per 32
    float *rowback;    // [m] 2^-s_row
    int ksplit;        // K split of the ring kernel (1: none)
    float *ysplit;     // [ksplit][m][n] f32 partial results when ksplit > 1
};
// ring kernel (nnq_gemm_ring.hip): its K split for a shape (0: the shape does not fit
// the kernel; bn and bm, when given, receive the tile width and height), and its launch
int gemm_ring_plan(const GemmArgs &a, int *bn, int *bm = nullptr);
int launch_gemm_ring(const GemmArgs &a, const GemmScratch &sc, void *stream);
// wide-wave-tile kernel (nnq_gemm_wide.hip; bf16 activations, more than 128 rows): its
// column tiles per workgroup (0: the shape does not fit) and K split, its scratch (the
// fragment-major staged activation in xh, min-term operands in xs, rowback, split slabs;
// s null: sizes only) and its launch (staging, kernel, and with a K split the slab sum)
int gemm_wide_plan(const GemmArgs &a, int *ks);
// the skinny kernel (same file and staging; bf16 activations, 17 to 32 rows): whether it
// takes the shape, with its tiles per workgroup R and waves W
int gemm_skinny_plan(const GemmArgs &a, int *R, int *W);
size_t gemm_wide_scratch(const GemmArgs &a, GemmScratch *s, uint8_t *base);
int launch_gemm_wide(const GemmArgs &a, const GemmScratch &sc, void *stream);
// the wide kernels' activation staging (bf16 x, K a multiple of 256 up to 12288): f16 of
// x * 2^s_row in fragment order, 2^-s_row per row, and (xs given) the Q4_K min-term operands
int launch_stage_wide(const uint16_t *x, int64_t m, int64_t k, void *xa, void *xs, float *rowback, void *stream);
// Q8_0 wide kernel (nnq_gemm_wide8.hip): column tiles per workgroup (0: not its shape) and
// K split; its scratch; the staging and the kernel (and the slab sum with a split)
int gemm_wide8_plan(const GemmArgs &a, int *ks);
size_t gemm_wide8_scratch(const GemmArgs &a, GemmScratch *s, uint8_t *base);
int launch_gemm_wide8(const GemmArgs &a, const GemmScratch &sc, void *stream);
// split-K result: ks f32 slabs [m][n] summed in order, plus the bias, to f32 or bf16 (n % 4 == 0)
int launch_gemm_finalize(const float *ys, int ks, const float *bias, void *y, int y_bf16, int64_t m, int64_t n,
                         void *stream);
// the staging scratch of a GEMM call (base null: sizes only) and the staging kernel
GemmScratch gemm_carve(void *base, const GemmArgs &a, size_t *bytes);
int launch_gemm_prep(const GemmArgs &a, const GemmScratch &sc, void *stream);

// MoE (GPT-OSS MXFP4).  Expert weights [E][K][N] with 32-element blocks along N
// (Mxfp4Tensor of the flat tensor) are repacked per (expert, 32-column block nb,
// 32-row block kb): codes [E][N/32][K/32][512] (lane l = 16p + c holds the 8 bytes
// of rows 32kb + 8p .. 8p + 7 at byte column c, i.e. columns 2c (high nibble) and
// 2c + 1 (low nibble)) and scales [E][N/32][K/32][32] (rows 32kb .. 32kb + 31).  A
// bijection on the bytes.
struct MoeDev {
    int64_t E, H, I;
    const uint8_t *gu_q;    // gate_up codes, K = H, N = 2I
    const uint8_t *gu_s;    // gate_up scales
    const float *gu_b;      // [E, 2I]
    const uint8_t *dn_q;    // down codes, K = I, N = H
    const uint8_t *dn_s;
    const float *dn_b;      // [E, H]
};
size_t moe_scratch_bytes(int64_t T, int64_t E, int64_t H, int64_t I, int top_k, int x_bf16);
// logits: nsplit slabs [T][E] summed in order, plus bias when given (nsplit 1, no bias: the logits);
// status (optional, cleared beforehand by the caller) flags a non-finite output
int launch_moe(const MoeDev &m, const void *x, int x_bf16, int64_t T, const float *logits, int nsplit,
               const float *bias, int top_k, float limit, float *y, uint32_t *topk_idx, float *topk_w,
               int32_t *status, void *scratch, void *stream);
int launch_moe_dequant(const MoeDev &m, int64_t e, float *gate_up, float *down, void *stream);
// nn-core OCP MXFP4 tensor decode: n values from 17-byte blocks (device pointers)
int launch_ocp_dequant(const uint8_t *blocks, int64_t n, float *out, void *stream);
// router Linear x[T, H] @ W[E, H]^T (+ bias), H a multiple of 16, over *nsplit K parts: with one
// part `partial` receives the logits (bias added), else nsplit slabs [T][E] of partial sums
// (router_partial_bytes; the bias is left to the consumer).  Clears *status when given.
size_t router_partial_bytes(int64_t T, int64_t H, int E);
int launch_router_logits(const void *x, int x_bf16, int64_t T, int64_t H, const float *W, const float *bias, int E,
                         float *partial, int *nsplit, int32_t *status, void *stream);
int launch_router_finalize(const float *partial, int ks, int64_t T, int E, const float *bias, float *logits,
                           void *stream);
// host repack of one weight (codes and scales of E experts, K rows, N columns); the device
// scale byte e means 2^(e - 127), so with gptoss_scales the GPT-OSS byte 0 (2^-126) is
// stored as 1
void moe_repack(const uint8_t *packed, const uint8_t *scales, int64_t E, int64_t K, int64_t N, uint8_t *dst_codes,
                uint8_t *dst_scales, bool gptoss_scales);
// nn-core OCP MXFP4 blocks (17 bytes: shared_exp, 16 packed with element 2i in the low
// nibble) -> GPT-OSS-ordered packed bytes (element 2i in the high nibble) and scale bytes
void ocp_split(const uint8_t *blocks, size_t nblocks, uint8_t *packed, uint8_t *scales);

}  // namespace nnq
