/*
 * nnq — MI355X (gfx950) quantized-linear hot path: C ABI.
 *
 * Drop-in boundary for alabsystems/nn's dequant-fused matmul over GGUF block
 * formats (Q8_0, Q4_K, Q6_K) and the GPT-OSS MXFP4 mixture-of-experts layer.
 * A Rust backend crate binds these symbols with `extern "C"` the way nn-cuda
 * binds libamdhip64
 * (crates/nn-cuda/src/hip_runtime_ffi_linux.rs:17-47): plain pointers, sizes
 * and i32 status codes, no C++ or torch types.
 *
 * Conventions
 *  - Every call returns an nnq_status; on failure nnq_last_error() returns a
 *    thread-local message.
 *  - Device pointers (x, y, bias, logits, outputs) live on the current HIP
 *    device; `stream` is a hipStream_t (NULL = the null stream).  Compute calls
 *    are asynchronous on `stream` and never synchronize the host.
 *  - Weight handles are immutable after creation and may be shared across
 *    threads and streams.
 *  - Scratch memory: eager calls on a stream share that stream's workspace (grown
 *    and freed stream-ordered); calls captured into a HIP graph use a workspace of
 *    their capture sequence, so a graph may be replayed on any stream while eager
 *    calls run elsewhere.  Two replays of one graph that overlap in time share that
 *    graph's workspace and must be ordered by the caller.  A capture's workspace is
 *    kept until nnq_release_capture_workspaces; nnq_release_workspace frees a
 *    stream's eager one.
 *  - Several host threads may call on one stream: a call holds the stream's
 *    workspace from its first scratch request until its last enqueue, so their
 *    calls take it one at a time.  (nnq_linear_sample_noalloc's fixed scratch is
 *    the exception; see there.)
 *  - Weights are row-major W[n, k] (out_features x in_features) with blocks
 *    along k, as QuantizedStorage / QuantizedWeight store them
 *    (crates/nn-core/src/dyn_tensor/quantized.rs:109-172,
 *     crates/nn-core/src/layers/quantized/linear.rs:260-264).
 */
#ifndef NNQ_H
#define NNQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The quantized-matmul kinds mirror QuantizedMatmulError
 * (crates/nn-core/src/dyn_tensor/quantized_matmul.rs:30-82); the tensor and
 * backend kinds mirror TensorError / BackendErrorKind
 * (crates/nn-core/src/error.rs:48-93,171). */
typedef enum nnq_status {
    NNQ_OK = 0,
    NNQ_ERR_INVALID_ARGUMENT = 1,  /* null pointer, negative or zero size where not allowed */
    NNQ_ERR_SHAPE_MISMATCH = 2,    /* QuantizedMatmulError::ShapeMismatch (input K != weight K) */
    NNQ_ERR_WRONG_FORMAT = 3,      /* QuantizedMatmulError::WrongQuantType / unsupported layout */
    NNQ_ERR_NOT_QUANTIZED = 4,     /* QuantizedMatmulError::NotQuantized */
    NNQ_ERR_WEIGHT_RANK = 5,       /* QuantizedMatmulError::WeightRank */
    NNQ_ERR_BIAS_MISMATCH = 6,     /* QuantizedMatmulError::BiasMismatch */
    NNQ_ERR_DATA_LENGTH = 7,       /* TensorError::DataLengthMismatch */
    NNQ_ERR_INVALID_SHAPE = 8,     /* TensorError::InvalidShape (element count not a block multiple) */
    NNQ_ERR_NON_FINITE = 9,        /* TensorError::NonFiniteData / ValueOutOfRange */
    NNQ_ERR_NO_DEVICE = 10,        /* no HIP device */
    NNQ_ERR_OUT_OF_MEMORY = 11,    /* BackendErrorKind::OutOfMemory */
    NNQ_ERR_DISPATCH_FAILED = 12,  /* BackendErrorKind::DispatchFailed */
    NNQ_ERR_UNSUPPORTED = 13       /* TensorError::Unsupported */
} nnq_status;

/* Block formats; values are the GGUF type ids (GgufDType,
 * crates/nn-gguf/src/dequant.rs:14-45).  MXFP4 uses ggml's id 39. */
typedef enum nnq_format {
    NNQ_FMT_Q8_0 = 8,
    NNQ_FMT_Q4_K = 12,
    NNQ_FMT_Q6_K = 14,
    NNQ_FMT_MXFP4 = 39
} nnq_format;

/* Byte layouts.  The reference carries more than one decoder per format:
 *  NNQ_LAYOUT_GGUF    Q8_0 (crates/nn-core/src/dyn_tensor/quantized.rs:237-253) and
 *                     Q4_K as nn-core BlockQ4K (crates/nn-core/src/layers/quantized/linear.rs:49-92,166-176).
 *  NNQ_LAYOUT_NN_GGUF nn-gguf's own decoders: Q4_K (crates/nn-gguf/src/dequant.rs:335-398),
 *                     Q6_K (crates/nn-gguf/src/dequant.rs:415-459, the only Q6_K decoder), Q8_0 (:178-196).
 *  NNQ_LAYOUT_GPTOSS  GPT-OSS Mxfp4Tensor (crates/nn-gptoss/src/quantize.rs:122-188): packed bytes with
 *                     the HIGH nibble = even element, E8M0 scales in a separate array, byte 0 -> 2^-126.
 *  NNQ_LAYOUT_OCP     nn-core Mxfp4Block (crates/nn-core/src/layers/quantized/mxfp4.rs:70-84,177-244):
 *                     17-byte blocks [shared_exp][16 packed] along the flattened order, the LOW nibble =
 *                     even element, scale 2^(shared_exp - 127) with byte 0 -> 2^-127. */
typedef enum nnq_layout {
    NNQ_LAYOUT_GGUF = 0,
    NNQ_LAYOUT_NN_GGUF = 1,
    NNQ_LAYOUT_GPTOSS = 2,
    NNQ_LAYOUT_OCP = 3
} nnq_layout;

typedef enum nnq_dtype {
    NNQ_F32 = 0,
    NNQ_F16 = 1,
    NNQ_BF16 = 2
} nnq_dtype;

typedef struct nnq_weight nnq_weight;   /* opaque: device-resident, repacked block weight */
typedef struct nnq_moe nnq_moe;         /* opaque: device-resident MXFP4 expert weights + biases */
typedef struct nnq_mlp nnq_mlp;         /* opaque: device-resident SwiGLU MLP (gate | up, down) */
typedef struct nnq_router nnq_router;   /* opaque: device-resident f32 router Linear */
typedef struct nnq_gguf nnq_gguf;       /* opaque: a memory-mapped GGUF file */

/* ---- device ------------------------------------------------------------------- */

/* Count HIP devices (0 when none).  Replaces the device probe of nn-cuda's HIP
 * runtime (crates/nn-cuda/src/hip_runtime.rs:191). */
int nnq_device_count(int *count);

/* Make `device` current for this thread and initialise per-device state.
 * NNQ_ERR_NO_DEVICE when no HIP device exists.  Counterpart of
 * register_gpu_backend (crates/nn-core/src/dyn_tensor/gpu.rs:156-162). */
int nnq_init(int device);

/* Thread-local description of the last failure on this thread ("" if none). */
const char *nnq_last_error(void);

/* Free the scratch workspace that eager calls on `stream` (current device) hold, stream-
 * ordered on that stream; call it before destroying the stream.  No counterpart in the
 * reference (its CPU path allocates per call); the next call on the stream allocates
 * again. */
int nnq_release_workspace(void *stream);

/* Free the workspaces of every capture sequence on the current device (calls captured
 * into HIP graphs keep theirs, since a graph reads it on every replay).  Call it once
 * every graph that captured library calls on this device has been destroyed, or will
 * never be replayed again; a replay after it reads freed memory.  Graphs captured
 * afterwards allocate again.  No counterpart in the reference (it captures no graphs);
 * it is for callers that capture graphs repeatedly, e.g. one per shape bucket. */
int nnq_release_capture_workspaces(void);

/* ---- weights ------------------------------------------------------------------ */

/* Upload host block bytes for W[n, k] to the current device, repacked into the
 * device layout.  The caller keeps ownership of `bytes`.  Validation follows
 * QuantizedStorage::new (crates/nn-core/src/dyn_tensor/quantized.rs:121-140):
 * NNQ_ERR_INVALID_SHAPE when k is not a multiple of the block size (32 for Q8_0,
 * 256 for Q4_K/Q6_K), NNQ_ERR_DATA_LENGTH when nbytes != n*k/block*block_bytes.
 * Replaces DynTensor::from_quantized (:270-278) and QLinear::from_linear's
 * block storage (crates/nn-core/src/layers/quantized/linear.rs:309-346). */
int nnq_weight_create(nnq_format fmt, nnq_layout layout, const uint8_t *bytes, size_t nbytes, int64_t n,
                      int64_t k, nnq_weight **out);

int nnq_weight_destroy(nnq_weight *w);

/* Shape / format queries (QuantizedStorage::shape / quant_type, quantized.rs:142-152). */
int nnq_weight_info(const nnq_weight *w, int *fmt, int *layout, int64_t *n, int64_t *k, size_t *device_bytes);

/* Decode the whole weight to f32 W[n, k] at device pointer `out` — bit-exact with
 * QuantizedStorage::dequantize / BlockQ4K::dequantize / dequantize_q6_k
 * (crates/nn-core/src/dyn_tensor/quantized.rs:155-165,
 *  crates/nn-core/src/layers/quantized/linear.rs:268-281,
 *  crates/nn-gguf/src/dequant.rs:178-196,335-459). */
int nnq_dequant(const nnq_weight *w, float *out, void *stream);

/* ---- quantized linear ----------------------------------------------------------- */

/* y[m, n] = x[m, k] @ W^T (+ bias[n]).  `m` folds every leading batch dimension
 * (rank folding as in quantized_matmul_core, quantized_matmul.rs:232-272); m = 0
 * is a no-op.  `k` is the input's last dimension: k != weight k gives
 * NNQ_ERR_SHAPE_MISMATCH (validate_input, :121-145).  bias: f32 [bias_len] or
 * NULL; bias_len != n gives NNQ_ERR_BIAS_MISMATCH (:391-401).
 * x: NNQ_F32 or NNQ_BF16 (bf16 is widened exactly to f32, ops/matmul.rs:20-21);
 * y: NNQ_F32, or NNQ_BF16 (f32 accumulate, rounded to bf16 once, ops/matmul.rs:37-38).
 * Replaces quantized_linear / quantized_matmul_q8_0 (quantized_matmul.rs:335-406)
 * and QLinear::forward (crates/nn-core/src/layers/quantized/linear.rs:366-400). */
int nnq_linear(const nnq_weight *w, const void *x, nnq_dtype x_dtype, int64_t m, int64_t k, const float *bias,
               int64_t bias_len, void *y, nnq_dtype y_dtype, void *stream);

/* First index of the maximum of logits[n] (strict `>`), written as u32 to
 * `idx` (device).  NaN input -> *status_dev = NNQ_ERR_NON_FINITE (device int,
 * may be NULL).  Replaces DynTensor::argmax on the last dim
 * (crates/nn-core/src/dyn_tensor/ops_ext/argreduce.rs:19,94-118). */
int nnq_argmax_f32(const float *logits, int64_t n, uint32_t *idx, int32_t *status_dev, void *stream);

/* LM head: logits[n] = x[k] @ W^T (+bias) fused with the first-index argmax.
 * Replaces lm_head Linear + argmax (crates/nn-qwen3/src/lib.rs:124-133,
 * crates/nn-core/src/dyn_tensor/ops_ext/argreduce.rs:105-118). */
int nnq_linear_argmax(const nnq_weight *w, const float *x, int64_t k, const float *bias, int64_t bias_len,
                      float *logits, uint32_t *idx, int32_t *status_dev, void *stream);

/* ---- token sampling ------------------------------------------------------------- */

/* SamplingConfig (crates/nn-gptoss/src/sampling.rs:27-49) with the seed of sample_token.
 * The Option fields become flags: top_k < 0 is None, use_top_p = 0 is None. */
typedef struct nnq_sampling {
    float temperature;        /* > 0 and finite */
    int32_t top_k;            /* < 0: None (every logit > -inf, +inf included, is a candidate);
                                 0: no candidate (argmax fallback); >= n: the finite logits */
    int32_t use_top_p;        /* 0: top_p is None */
    float top_p;
    float repetition_penalty; /* 1.0: none */
    float frequency_penalty;  /* 0.0: none */
    uint64_t seed;            /* selector = (seed % 10000) / 10000 */
} nnq_sampling;

/* token (device u32) = sample_token(logits[n], cfg, past_tokens, seed) on the device:
 * repetition and frequency penalties per occurrence of past_tokens (device u32[n_past],
 * may be NULL when n_past = 0; indices >= n are ignored), temperature, top-k, top-p,
 * softmax and the seed's selector walk; with no candidate left, the last maximal index
 * of the original logits (argmax_slice).  logits is left unchanged.  Equal logits at the
 * k-th place keep the lower index (the reference's unstable sort leaves that open).
 * NNQ_ERR_INVALID_ARGUMENT for n = 0 or a temperature that is not positive and finite
 * (sample_token panics there).  Any top_k over any vocabulary below 2^32 logits: up to
 * ceil(n / 2048) * min(k, 2048) <= 16384 candidates (k = min(top_k, n), n with top_k
 * None) a two-pass top-k, beyond that every key sorted on the device (slower: the tail's
 * sums run in candidate order over all candidates, as the reference adds them).
 * Replaces sample_token (crates/nn-gptoss/src/sampling.rs:136-185). */
int nnq_sample_token(const float *logits, int64_t n, const uint32_t *past_tokens, int64_t n_past,
                     const nnq_sampling *cfg, uint32_t *token, void *stream);

/* LM head + sampling: logits[n] = x[k] @ W^T (+ bias), then nnq_sample_token on them,
 * with no host round trip.  Replaces lm_head Linear + sample_token (decode step). */
int nnq_linear_sample(const nnq_weight *w, const float *x, int64_t k, const float *bias, int64_t bias_len,
                      float *logits, const uint32_t *past_tokens, int64_t n_past, const nnq_sampling *cfg,
                      uint32_t *token, void *stream);

/* nnq_linear_sample without allocation.  It has no counterpart in the reference: it is
 * for callers that cannot call hipMalloc (code under HIP graph capture, serving loops,
 * harnesses that forbid allocation).  Arguments, results and errors as
 * nnq_linear_sample; the sampling scratch comes from a fixed device array of 384 KiB
 * that each GPU holds until the process ends (nnq_init looks up its address), so no
 * call allocates.  That bounds the top-k: ceil(n / 2048) * min(k, 2048) <= 16384, as for
 * nnq_linear_sample; beyond it NNQ_ERR_UNSUPPORTED.  Every call on one GPU uses that
 * GPU's one array: calls that overlap on one GPU (other streams, or graphs replayed
 * concurrently) race and must be serialized by the caller. */
int nnq_linear_sample_noalloc(const nnq_weight *w, const float *x, int64_t k, const float *bias, int64_t bias_len,
                              float *logits, const uint32_t *past_tokens, int64_t n_past, const nnq_sampling *cfg,
                              uint32_t *token, void *stream);

/* ---- Qwen3 SwiGLU MLP ----------------------------------------------------------- */

/* Upload one layer's MLP: gate_proj and up_proj W[inter, hidden] (block bytes of one
 * format / layout, gu_nbytes each) and down_proj W[hidden, inter].  gate and up are
 * stacked into one W[2 * inter, hidden] so that one GEMV computes both.  Validation
 * as nnq_weight_create.  Replaces Qwen3MLP::load (crates/nn-qwen3/src/layers.rs:26-38)
 * over quantized Linear weights. */
int nnq_mlp_create(nnq_format gu_fmt, nnq_layout gu_layout, const uint8_t *gate, const uint8_t *up,
                   size_t gu_nbytes, nnq_format down_fmt, nnq_layout down_layout, const uint8_t *down,
                   size_t down_nbytes, int64_t hidden, int64_t inter, nnq_mlp **out);

int nnq_mlp_destroy(nnq_mlp *mlp);

/* y[m, hidden] = down(silu(gate(x)) * up(x)) for x[m, k] (k = hidden; NNQ_F32 or
 * NNQ_BF16, 16-byte aligned); y NNQ_F32 or NNQ_BF16.  silu(v) = v / (1 + e^-v) and the
 * product in f32.  Decode (m <= 2): two launches, the gate | up GEMV, then the down GEMV
 * forming silu(gate) * up as it stages its input.  Larger m: gate | up linear, SwiGLU,
 * down linear.  status_dev (device int, may be NULL): NNQ_OK, or NNQ_ERR_NON_FINITE
 * when an output is NaN or infinite, as check_output_finite reports it
 * (crates/nn-core/src/layers/nan_check.rs:113-140).
 * Replaces Qwen3MLP::forward (crates/nn-qwen3/src/layers.rs:40-47). */
int nnq_mlp_forward(const nnq_mlp *mlp, const void *x, nnq_dtype x_dtype, int64_t m, int64_t k, void *y,
                    nnq_dtype y_dtype, int32_t *status_dev, void *stream);

/* ---- GPT-OSS MXFP4 mixture of experts ----------------------------------------- */

/* Upload one layer's expert weights in the GPT-OSS convention:
 *  gate_up: Mxfp4Tensor of the flat [E, hidden, 2*inter] f32 tensor
 *           (packed bytes E*hidden*2*inter/2, scales E*hidden*2*inter/32),
 *  down:    Mxfp4Tensor of the flat [E, inter, hidden] tensor,
 *  biases:  f32 [E, 2*inter] and [E, hidden] (host).
 * hidden and inter must be multiples of 32 (NNQ_ERR_INVALID_SHAPE), at most 32768 each and
 * at most 4096 experts (NNQ_ERR_UNSUPPORTED beyond; checked before any allocation).  The
 * codes are repacked on upload into per-(expert, 32-column block, 32-row block)
 * fragments in MFMA lane order (a permutation of the bytes).
 * Replaces QuantizedDecoderLayer::load's expert tensors
 * (crates/nn-gptoss/src/quantized_model.rs:70-78). */
int nnq_moe_create(int64_t num_experts, int64_t hidden, int64_t inter, const uint8_t *gu_packed,
                   const uint8_t *gu_scales, const float *gu_bias, const uint8_t *dn_packed,
                   const uint8_t *dn_scales, const float *dn_bias, nnq_moe **out);

/* The same upload from nn-core OCP MXFP4 tensors (NNQ_LAYOUT_OCP): gu_blocks holds the
 * quantize_tensor blocks of the flat [E, hidden, 2*inter] tensor (E*hidden*2*inter/32
 * blocks of 17 bytes), dn_blocks those of [E, inter, hidden]; biases and shape limits as
 * nnq_moe_create.
 * Both layouts decode to the same values on the device: every E8M0 byte e scales by
 * 2^(e - 127), GPT-OSS's byte 0 being stored as 1.  Replaces the expert tensors of an MoE
 * whose weights come from mxfp4_quantize_tensor
 * (crates/nn-core/src/layers/quantized/mxfp4.rs:293-315). */
int nnq_moe_create_ocp(int64_t num_experts, int64_t hidden, int64_t inter, const uint8_t *gu_blocks,
                       const float *gu_bias, const uint8_t *dn_blocks, const float *dn_bias, nnq_moe **out);

int nnq_moe_destroy(nnq_moe *moe);

/* y[t, hidden] (f32) = MoE(x[t, hidden]) with router logits [t, E] (f32):
 * softmax -> top_k -> renormalise -> per expert clamp(silu(x@Wg+bg), -limit, limit)
 * * (x@Wu+bu) -> @Wd + bd -> weighted sum.  x: NNQ_F32 or NNQ_BF16, 16-byte aligned;
 * any number of tokens (batches beyond 16384 token-expert assignments run as token
 * chunks of that size, one after another on the stream), top_k from 1 to the number of
 * experts (experts_per_token, crates/nn-gptoss/src/quantized_model.rs:92,141).  Routing,
 * permutation and combine run on the
 * device (no host synchronisation); the expert outputs are summed per token in
 * ascending expert order, as moe_forward's index_add does.
 * Optional outputs topk_idx [t, top_k] u32 and topk_w [t, top_k] f32 (device).
 * Replaces QuantizedDecoderLayer::moe_forward / expert_forward
 * (crates/nn-gptoss/src/quantized_model.rs:99-194). */
int nnq_moe_forward(const nnq_moe *moe, const void *x, nnq_dtype x_dtype, int64_t tokens,
                    const float *router_logits, int top_k, float swiglu_limit, float *y, uint32_t *topk_idx,
                    float *topk_w, void *stream);

/* Upload the GPT-OSS router Linear: weight f32 [num_experts, hidden], bias f32
 * [num_experts] or NULL (host).  hidden a multiple of 32, at most 4096 experts.
 * Replaces QuantizedDecoderLayer::load's router (crates/nn-gptoss/src/quantized_model.rs:63-67),
 * which keeps it at full precision. */
int nnq_router_create(int64_t num_experts, int64_t hidden, const float *weight, const float *bias, nnq_router **out);

int nnq_router_destroy(nnq_router *router);

/* logits[t, E] (f32) = x[t, hidden] @ W^T + bias, f32 products and sums; x NNQ_F32 or
 * NNQ_BF16 (16-byte aligned).  Replaces the router's Linear::forward
 * (crates/nn-core/src/layers/core_layers.rs:118-140, called at quantized_model.rs:138). */
int nnq_router_logits(const nnq_router *router, const void *x, nnq_dtype x_dtype, int64_t tokens, float *logits,
                      void *stream);

/* The whole MoE block of one layer: router logits on the device, then nnq_moe_forward's
 * routing, experts and combine, then the output check — QuantizedDecoderLayer::moe_forward
 * with its router (crates/nn-gptoss/src/quantized_model.rs:132-194).  Nothing returns to
 * the host between the steps.  status_dev (device int, may be NULL): NNQ_OK, or
 * NNQ_ERR_NON_FINITE when an output is NaN or infinite (check_output_finite,
 * crates/nn-core/src/layers/nan_check.rs:113-140).  Other arguments as nnq_moe_forward;
 * the router must match the MoE's experts and hidden size (NNQ_ERR_SHAPE_MISMATCH). */
int nnq_moe_block_forward(const nnq_moe *moe, const nnq_router *router, const void *x, nnq_dtype x_dtype,
                          int64_t tokens, int top_k, float swiglu_limit, float *y, uint32_t *topk_idx, float *topk_w,
                          int32_t *status_dev, void *stream);

/* Decode expert e's weights to f32 (device): gate_up [hidden, 2*inter] and down
 * [inter, hidden] — bit-exact with Mxfp4Tensor::dequantize
 * (crates/nn-gptoss/src/quantize.rs:167-188). Either output may be NULL. */
int nnq_moe_dequant_expert(const nnq_moe *moe, int64_t expert, float *gate_up, float *down, void *stream);

/* Decode the first n values of an nn-core OCP MXFP4 tensor (device blocks of 17 bytes,
 * ceil(n / 32) of them) to f32 at device `out` — bit-exact with dequantize_tensor
 * (crates/nn-core/src/layers/quantized/mxfp4.rs:226-244,320-333) for every shared_exp
 * 0..254 (255 scales by +inf: infinities, and NaN for zero codes). */
int nnq_dequant_mxfp4_ocp(const uint8_t *blocks, int64_t n, float *out, void *stream);

/* ---- GGUF ingest ------------------------------------------------------------------ */

/* Open a GGUF v3 file memory-mapped (no tensor bytes are read or copied): header,
 * metadata and tensor infos are parsed and every tensor's byte range is checked against
 * the file.  The data section starts at the next multiple of 32 bytes after the tensor
 * infos (fixed, as the reference does).  Errors: NNQ_ERR_WRONG_FORMAT (magic, version,
 * unknown metadata or tensor type), NNQ_ERR_INVALID_SHAPE (a reference limit exceeded:
 * 100000 tensors or metadata pairs, 16 MiB strings, 10^7 array elements, 8 dimensions,
 * a zero dimension, 8 GiB per tensor), NNQ_ERR_DATA_LENGTH (truncated file, tensor data
 * out of bounds), NNQ_ERR_INVALID_ARGUMENT (cannot open).  Host only; no device needed.
 * Replaces GgufFile::open (crates/nn-gguf/src/reader.rs:68-141). */
int nnq_gguf_open(const char *path, nnq_gguf **out);

int nnq_gguf_close(nnq_gguf *gguf);

int nnq_gguf_info(const nnq_gguf *gguf, uint32_t *version, int64_t *tensor_count, int64_t *metadata_count,
                  uint64_t *data_offset);

/* Tensor i (file order): name (valid until close), dimensions as stored (dims holds up to
 * 8), GGUF type id, offset in the data section and byte size (GgufTensorInfo,
 * crates/nn-gguf/src/tensor_info.rs:20-33).  Any output may be NULL. */
int nnq_gguf_tensor_info(const nnq_gguf *gguf, int64_t i, const char **name, int32_t *n_dims, uint64_t *dims,
                         uint32_t *dtype, uint64_t *offset, uint64_t *nbytes);

/* Zero-copy tensor bytes: a pointer into the mapping, valid until close
 * (GgufFile::tensor_data, reader.rs:287-344).  A repeated name resolves to its last entry. */
int nnq_gguf_tensor_data(const nnq_gguf *gguf, const char *name, const uint8_t **data, uint64_t *nbytes);

/* Metadata value of `key` (GgufMetadata::get, crates/nn-gguf/src/metadata.rs:98-130): its
 * GGUF type id and value (unsigned / bool in *u, signed in *i, floats in *f, strings in
 * *str (valid until close), arrays as element type and count).  Any output may be NULL. */
int nnq_gguf_metadata(const nnq_gguf *gguf, const char *key, uint32_t *type, uint64_t *u, int64_t *i, double *f,
                      const char **str, uint32_t *arr_type, uint64_t *arr_count);

/* A device weight straight from a Q8_0 / Q4_K / Q6_K tensor's mapped bytes (repacked on
 * upload, as nnq_weight_create; no f32 expansion).  The 2-D shape is read as stored,
 * [out, in], or with ggml_order != 0 as [in, out] (ggml's ne0 first).  layout selects the
 * block decoder the bytes follow (NNQ_LAYOUT_NN_GGUF: nn-gguf's, which its reader uses).
 * Replaces the read_tensor_f32 + Linear path of weight loading
 * (crates/nn-gguf/src/reader.rs:192-281). */
int nnq_gguf_weight_create(const nnq_gguf *gguf, const char *name, nnq_layout layout, int ggml_order,
                           nnq_weight **out);

/* ---- host encoders (CPU, no device needed) --------------------------------------- */

/* BlockQ4K::quantize over a flat f32 buffer, zero-padded to 256 as
 * QLinear::from_linear does (crates/nn-core/src/layers/quantized/linear.rs:95-162,
 * 309-346).  `out` holds ceil(n/256)*144 bytes.  NNQ_ERR_NON_FINITE on NaN/inf. */
int nnq_quantize_q4_k(const float *v, size_t n, uint8_t *out);

/* Mxfp4Tensor::quantize (crates/nn-gptoss/src/quantize.rs:122-163): `packed`
 * holds ceil(n/32)*16 bytes, `scales` ceil(n/32) bytes. */
int nnq_quantize_mxfp4(const float *v, size_t n, uint8_t *packed, uint8_t *scales);

/* nn-core OCP MXFP4 quantize_tensor (crates/nn-core/src/layers/quantized/mxfp4.rs:142-220,
 * 293-315): `blocks` holds ceil(n/32)*17 bytes; NNQ_ERR_NON_FINITE on NaN/inf
 * (ValueOutOfRange). */
int nnq_quantize_mxfp4_ocp(const float *v, size_t n, uint8_t *blocks);

/* Q8_0 and nn-gguf-layout Q6_K encoders.  The reference ships no encoder for
 * either (its tests hand-build blocks, quantized_matmul_tests.rs:37-46); these
 * are this library's own input generators.  n must be a block multiple. */
int nnq_quantize_q8_0(const float *v, size_t n, uint8_t *out);
int nnq_quantize_q6_k(const float *v, size_t n, uint8_t *out);

/* Seeded N(0, sigma) f32 generator: splitmix64 (crates/nn-core/src/test_prng.rs:18-22)
 * keyed by (seed, tensor_id, index), uniform from the top 53 bits (:31-33),
 * Box-Muller in f64, cast to f32. */
int nnq_synth_normal(uint64_t seed, uint64_t tensor_id, size_t n, double sigma, float *out);

#ifdef __cplusplus
}
#endif
#endif /* NNQ_H */
