"""nn_amd — MI355X (gfx950) quantized-linear hot path for alabsystems/nn.

Hand-written HIP kernels behind a C ABI (``include/nnq.h``, ``libnnq.so``) for
the dequant-fused matmul over GGUF Q8_0 / Q4_K / Q6_K blocks and the GPT-OSS
MXFP4 mixture-of-experts layer (GPT-OSS and nn-core OCP MXFP4 layouts); ``nn_amd.quantized`` mirrors the reference's
operator surface in Python.
"""
from .quantized import (  # noqa: F401
    BiasMismatch, DataLengthMismatch, InvalidShape, Layout, NonFiniteData, NotQuantized, QuantizedMatmulError,
    QuantizedMLP, QuantizedMoE, QuantizedWeight, QuantType, RankMismatch, ShapeMismatch, TensorError, Unsupported, WeightRank,
    WrongQuantType, argmax, dequantize_mxfp4_ocp, device_count, init, linear_argmax, linear_sample, sample_token,
    quantize_mxfp4, quantize_mxfp4_ocp, quantize_q4_k, quantize_q6_k, quantize_q8_0, quantized_linear, quantized_matmul_q4_k, quantized_matmul_q6_k, quantized_matmul_q8_0,
    synth_normal)
