/*
 * CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's (alabsystems/nn, Rust) CPU arithmetic
 * for Q8_0 / Q4_K / Q6_K / GPT-OSS MXFP4 decode, encode and the matmul / MoE
 * computations that consume them.  Every function cites the reference file:line
 * it follows.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load this library, and only as the checker (or the timed CPU
 * baseline), never as the product path.
 *
 * Floating-point rules: compiled with -ffp-contract=off (Rust never contracts
 * a*b+c into an FMA), IEEE binary32 with round-to-nearest-even, no fast-math.
 *
 * Pinning (tests/test_oracle.py): decoders, the fused Q8_0 matmul, MXFP4 format
 * functions, argmax, softmax/top-k and the MoE forward are pinned by the reference's
 * known-answer tests, Kani invariants, closed forms and f64 brute force.  Parity
 * unpinned (stated where they are defined): the exact output bytes of
 * orc_quantize_q4_k (its tests only bound the round-trip error); orc_quantize_q8_0
 * and orc_quantize_q6_k_legacy, which are this build's own input generators because
 * the reference has no encoder for either (checked by round-trip bounds only); the
 * accumulation order of the f32 sinks (the reference's matrixmultiply order); the
 * order of exactly tied top-k values.  Parity of the GPU path is graded on decode and
 * compute over shared encoded bytes, so none of these enters a parity verdict.
 */
#ifndef NNQ_ORACLE_H
#define NNQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- half-precision helpers (the `half` crate's IEEE semantics) ---------- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
void orc_f16_to_f32_array(const uint16_t *in, size_t n, float *out);
void orc_f32_to_f16_array(const float *in, size_t n, uint16_t *out);
void orc_f32_to_bf16_array(const float *in, size_t n, uint16_t *out);

/* ---- Q8_0 ----------------------------------------------------------------- */
size_t orc_dequant_q8_0(const uint8_t *data, size_t nbytes, size_t num_elements, float *out);
int orc_q8_0_matmul(const float *x, size_t rows, size_t k, const uint8_t *w, size_t n, float *y);
void orc_quantize_q8_0(const float *v, size_t n, uint8_t *out);

/* ---- Q4_K (GGUF-spec layout: nn-core BlockQ4K) and nn-gguf legacy layout --- */
void orc_q4k_get_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m);
void orc_q4k_dequant_block(const uint8_t *blk, float *out);
size_t orc_dequant_q4_k_gguf(const uint8_t *data, size_t nbytes, size_t num_elements, float *out);
size_t orc_dequant_q4_k_legacy(const uint8_t *data, size_t nbytes, size_t num_elements, float *out);
int orc_q4k_nearest_int(float v, int32_t *out);
int orc_q4k_make_qkx1_quants(int nmax, int ntry, const float *x, size_t n, float *scale, float *neg_min);
int orc_quantize_q4_k_block(const float *v, uint8_t *blk);
int orc_quantize_q4_k(const float *v, size_t n_total, uint8_t *out);

/* ---- Q6_K (nn-gguf layout, the only reference decoder) --------------------- */
size_t orc_dequant_q6_k_legacy(const uint8_t *data, size_t nbytes, size_t num_elements, float *out);
void orc_quantize_q6_k_legacy(const float *v, size_t n, uint8_t *out);

/* ---- GPT-OSS MXFP4 ----------------------------------------------------------- */
float orc_mxfp4_lut(int code);
uint8_t orc_mxfp4_e8m0_from_max(float max_abs);
float orc_mxfp4_decode_e8m0(uint8_t e);
uint8_t orc_mxfp4_quantize_fp4(float v, float scale);
void orc_mxfp4_quantize(const float *data, size_t n, uint8_t *packed, uint8_t *scales);
void orc_mxfp4_dequantize(const uint8_t *packed, const uint8_t *scales, size_t nblocks, size_t total, float *out);

/* ---- f32 compute sinks ------------------------------------------------------- */
void orc_matmul_xwt(const float *x, size_t m, size_t k, const float *w, size_t n, float *y);
void orc_matmul_xw(const float *x, size_t m, size_t k, const float *w, size_t n, float *y);
int orc_argmax(const float *v, size_t n, uint32_t *idx);
int orc_softmax_rows(const float *x, size_t rows, size_t cols, float *out);
int orc_topk_rows(const float *x, size_t rows, size_t cols, size_t k, float *vals, uint32_t *idx);
int orc_q4k_linear(const float *x, size_t rows, size_t k, const uint8_t *w, size_t n, float *y);
int orc_q6k_linear(const float *x, size_t rows, size_t k, const uint8_t *w, size_t n, float *y);

/* ---- nn-core OCP MXFP4 (17-byte blocks [shared_exp][16 packed], low nibble first) */
float orc_ocp_block_scale(uint8_t shared_exp);
uint8_t orc_ocp_shared_exp(const float *v32);
uint8_t orc_ocp_encode(float v, float block_scale);
float orc_ocp_decode(uint8_t code, float block_scale);
int orc_ocp_quantize_tensor(const float *data, size_t n, uint8_t *blocks);
void orc_ocp_dequantize_tensor(const uint8_t *blocks, size_t n, float *out);

/* ---- GPT-OSS MXFP4 mixture-of-experts layer ---------------------------------- */
int orc_moe_forward_mxfp4(const float *x, size_t n_tokens, size_t hidden, const float *router_logits,
                          size_t num_experts, size_t top_k, const uint8_t *gu_packed, const uint8_t *gu_scales,
                          const float *gu_bias, const uint8_t *dn_packed, const uint8_t *dn_scales,
                          const float *dn_bias, size_t inter, float swiglu_limit, int faithful_full_dequant,
                          float *out, uint32_t *topk_idx_out, float *topk_w_out);

/* ---- build-independent splitmix64 (for known-answer checks of the generator) */
uint64_t orc_splitmix64(uint64_t z);

/* Qwen3 MLP glue: h = silu(g) * u elementwise; non-finite scan of an output */
void orc_silu_mul(const float *g, const float *u, size_t n, float *h);
int orc_any_nonfinite(const float *v, size_t n);

/* Token sampling: sample_token (crates/nn-gptoss/src/sampling.rs:136-185); top_k < 0 = None */
size_t orc_argmax_slice(const float *v, size_t n);
int orc_sample_token(const float *logits, size_t n, const uint32_t *past, size_t n_past, float temperature,
                     int64_t top_k, int use_top_p, float top_p, float rep_penalty, float freq_penalty, uint64_t seed,
                     uint32_t *token);

#ifdef __cplusplus
}
#endif
#endif
