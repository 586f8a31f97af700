"""ctypes wrapper over the C oracle (``liboracle.so``) — TEST INFRASTRUCTURE ONLY.

The oracle is a CPU restatement of the reference's (alabsystems/nn) arithmetic for
the quantized-linear path; see ``nnq_oracle.c`` for the per-function citations.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker or the timed CPU baseline.

``compare`` mirrors nn-reftest's metric semantics
(crates/nn-reftest/src/compare.rs:22-120): max_abs, max_rel with a near-zero
skip below ``abs_tol``, and cosine similarity accumulated in f64.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_sz = ctypes.c_size_t


def build() -> str:
    """Compile liboracle.so from nnq_oracle.c (gcc, via oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32_array": (None, [_u16p, _sz, _f32p]),
            "orc_f32_to_f16_array": (None, [_f32p, _sz, _u16p]),
            "orc_f32_to_bf16_array": (None, [_f32p, _sz, _u16p]),
            "orc_dequant_q8_0": (_sz, [_u8p, _sz, _sz, _f32p]),
            "orc_q8_0_matmul": (ctypes.c_int, [_f32p, _sz, _sz, _u8p, _sz, _f32p]),
            "orc_quantize_q8_0": (None, [_f32p, _sz, _u8p]),
            "orc_q4k_get_scale_min": (None, [ctypes.c_int, _u8p, _u8p, _u8p]),
            "orc_q4k_dequant_block": (None, [_u8p, _f32p]),
            "orc_dequant_q4_k_gguf": (_sz, [_u8p, _sz, _sz, _f32p]),
            "orc_dequant_q4_k_legacy": (_sz, [_u8p, _sz, _sz, _f32p]),
            "orc_q4k_nearest_int": (ctypes.c_int, [ctypes.c_float, _i32p]),
            "orc_q4k_make_qkx1_quants": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _f32p, _sz, _f32p, _f32p]),
            "orc_quantize_q4_k_block": (ctypes.c_int, [_f32p, _u8p]),
            "orc_quantize_q4_k": (ctypes.c_int, [_f32p, _sz, _u8p]),
            "orc_dequant_q6_k_legacy": (_sz, [_u8p, _sz, _sz, _f32p]),
            "orc_quantize_q6_k_legacy": (None, [_f32p, _sz, _u8p]),
            "orc_mxfp4_lut": (ctypes.c_float, [ctypes.c_int]),
            "orc_mxfp4_e8m0_from_max": (ctypes.c_uint8, [ctypes.c_float]),
            "orc_mxfp4_decode_e8m0": (ctypes.c_float, [ctypes.c_uint8]),
            "orc_mxfp4_quantize_fp4": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_float]),
            "orc_mxfp4_quantize": (None, [_f32p, _sz, _u8p, _u8p]),
            "orc_mxfp4_dequantize": (None, [_u8p, _u8p, _sz, _sz, _f32p]),
            "orc_ocp_block_scale": (ctypes.c_float, [ctypes.c_uint8]),
            "orc_ocp_shared_exp": (ctypes.c_uint8, [_f32p]),
            "orc_ocp_encode": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_float]),
            "orc_ocp_decode": (ctypes.c_float, [ctypes.c_uint8, ctypes.c_float]),
            "orc_ocp_quantize_tensor": (ctypes.c_int, [_f32p, _sz, _u8p]),
            "orc_ocp_dequantize_tensor": (None, [_u8p, _sz, _f32p]),
            "orc_matmul_xwt": (None, [_f32p, _sz, _sz, _f32p, _sz, _f32p]),
            "orc_matmul_xw": (None, [_f32p, _sz, _sz, _f32p, _sz, _f32p]),
            "orc_argmax": (ctypes.c_int, [_f32p, _sz, _u32p]),
            "orc_softmax_rows": (ctypes.c_int, [_f32p, _sz, _sz, _f32p]),
            "orc_topk_rows": (ctypes.c_int, [_f32p, _sz, _sz, _sz, _f32p, _u32p]),
            "orc_q4k_linear": (ctypes.c_int, [_f32p, _sz, _sz, _u8p, _sz, _f32p]),
            "orc_q6k_linear": (ctypes.c_int, [_f32p, _sz, _sz, _u8p, _sz, _f32p]),
            "orc_moe_forward_mxfp4": (
                ctypes.c_int,
                [_f32p, _sz, _sz, _f32p, _sz, _sz, _u8p, _u8p, _f32p, _u8p, _u8p, _f32p, _sz, ctypes.c_float,
                 ctypes.c_int, _f32p, _u32p, _f32p],
            ),
            "orc_splitmix64": (ctypes.c_uint64, [ctypes.c_uint64]),
            "orc_silu_mul": (None, [_f32p, _f32p, _sz, _f32p]),
            "orc_argmax_slice": (_sz, [_f32p, _sz]),
            "orc_sample_token": (ctypes.c_int, [_f32p, _sz, _u32p, _sz, ctypes.c_float, ctypes.c_int64, ctypes.c_int,
                                                ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_uint64,
                                                _u32p]),
            "orc_any_nonfinite": (ctypes.c_int, [_f32p, _sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(np.frombuffer(bytes(a), dtype=np.uint8) if isinstance(a, (bytes, bytearray)) else a,
                                dtype=np.uint8)


class OracleError(RuntimeError):
    pass


# ---- conversions -----------------------------------------------------------
def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(bits, _u16p), bits.size, _p(out, _f32p))
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x, _f32p), x.size, _p(out, _u16p))
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_array(_p(x, _f32p), x.size, _p(out, _u16p))
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- decoders ----------------------------------------------------------------
def _dequant(fn, data, num_elements):
    data = _u8(data)
    out = np.zeros(num_elements, np.float32)
    n = fn(_p(data, _u8p), data.size, num_elements, _p(out, _f32p))
    return out[:n]


def dequant_q8_0(data, num_elements):
    return _dequant(lib().orc_dequant_q8_0, data, num_elements)


def dequant_q4_k(data, num_elements):
    """GGUF-spec layout (nn-core BlockQ4K)."""
    return _dequant(lib().orc_dequant_q4_k_gguf, data, num_elements)


def dequant_q4_k_legacy(data, num_elements):
    """nn-gguf's own Q4_K layout."""
    return _dequant(lib().orc_dequant_q4_k_legacy, data, num_elements)


def dequant_q6_k(data, num_elements):
    """nn-gguf Q6_K layout (the reference's only Q6_K decoder)."""
    return _dequant(lib().orc_dequant_q6_k_legacy, data, num_elements)


def q4k_get_scale_min(j, scales12):
    q = _u8(scales12)
    sc = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().orc_q4k_get_scale_min(j, _p(q, _u8p), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def q4k_nearest_int(v: float):
    out = ctypes.c_int32()
    rc = lib().orc_q4k_nearest_int(ctypes.c_float(v), ctypes.byref(out))
    if rc:
        raise OracleError("nearest_int: non-finite value or out of range")
    return out.value


# ---- encoders ------------------------------------------------------------------
def quantize_q8_0(v):
    v = _f32(v).ravel()
    out = np.zeros(v.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0(_p(v, _f32p), v.size, _p(out, _u8p))
    return out


def quantize_q4_k(v):
    v = _f32(v).ravel()
    out = np.zeros((v.size + 255) // 256 * 144, np.uint8)
    if lib().orc_quantize_q4_k(_p(v, _f32p), v.size, _p(out, _u8p)):
        raise OracleError("BlockQ4K::quantize: non-finite value")
    return out


def quantize_q6_k(v):
    v = _f32(v).ravel()
    out = np.zeros(v.size // 256 * 210, np.uint8)
    lib().orc_quantize_q6_k_legacy(_p(v, _f32p), v.size, _p(out, _u8p))
    return out


def mxfp4_quantize(v):
    v = _f32(v).ravel()
    nb = (v.size + 31) // 32
    packed = np.zeros(nb * 16, np.uint8)
    scales = np.zeros(nb, np.uint8)
    lib().orc_mxfp4_quantize(_p(v, _f32p), v.size, _p(packed, _u8p), _p(scales, _u8p))
    return packed, scales


def mxfp4_dequantize(packed, scales, total):
    packed = _u8(packed)
    scales = _u8(scales)
    out = np.zeros(total, np.float32)
    lib().orc_mxfp4_dequantize(_p(packed, _u8p), _p(scales, _u8p), scales.size, total, _p(out, _f32p))
    return out


def ocp_block_scale(e):
    """block_scale_from_exp (crates/nn-core/src/layers/quantized/mxfp4.rs:177-186)."""
    return float(lib().orc_ocp_block_scale(int(e)))


def ocp_shared_exp(v32):
    v = _f32(v32).ravel()
    assert v.size == 32
    return int(lib().orc_ocp_shared_exp(_p(v, _f32p)))


def ocp_encode(v, scale):
    return int(lib().orc_ocp_encode(ctypes.c_float(v), ctypes.c_float(scale)))


def ocp_decode(code, scale):
    return float(np.float32(lib().orc_ocp_decode(int(code), ctypes.c_float(scale))))


def ocp_quantize(v):
    """nn-core mxfp4 quantize_tensor (mxfp4.rs:293-315): ceil(n / 32) 17-byte blocks
    [shared_exp][16 packed, low nibble first]; OracleError on a non-finite value."""
    v = _f32(v).ravel()
    out = np.zeros(((v.size + 31) // 32) * 17, np.uint8)
    if lib().orc_ocp_quantize_tensor(_p(v, _f32p), v.size, _p(out, _u8p)) != 0:
        raise OracleError("mxfp4 quantize: non-finite input value")
    return out


def ocp_dequantize(blocks, n):
    """nn-core mxfp4 dequantize_tensor (mxfp4.rs:320-333): the first n values."""
    blocks = _u8(blocks)
    assert blocks.size >= ((n + 31) // 32) * 17
    out = np.zeros(n, np.float32)
    lib().orc_ocp_dequantize_tensor(_p(blocks, _u8p), n, _p(out, _f32p))
    return out


# ---- compute -------------------------------------------------------------------
def q8_0_matmul(x, w_bytes, n):
    x = _f32(x)
    k = x.shape[-1]
    rows = x.size // k
    w = _u8(w_bytes)
    y = np.zeros(x.shape[:-1] + (n,), np.float32)
    if lib().orc_q8_0_matmul(_p(x, _f32p), rows, k, _p(w, _u8p), n, _p(y, _f32p)):
        raise OracleError("q8_0 matmul: K not a multiple of 32")
    return y


def q4k_linear(x, w_bytes, n):
    x = _f32(x)
    k = x.shape[-1]
    w = _u8(w_bytes)
    y = np.zeros(x.shape[:-1] + (n,), np.float32)
    if lib().orc_q4k_linear(_p(x, _f32p), x.size // k, k, _p(w, _u8p), n, _p(y, _f32p)):
        raise OracleError("q4k linear failed")
    return y


def q6k_linear(x, w_bytes, n):
    x = _f32(x)
    k = x.shape[-1]
    w = _u8(w_bytes)
    y = np.zeros(x.shape[:-1] + (n,), np.float32)
    if lib().orc_q6k_linear(_p(x, _f32p), x.size // k, k, _p(w, _u8p), n, _p(y, _f32p)):
        raise OracleError("q6k linear failed")
    return y


def matmul_xwt(x, w):
    x = _f32(x)
    w = _f32(w)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), np.float32)
    lib().orc_matmul_xwt(_p(x, _f32p), m, k, _p(w, _f32p), n, _p(y, _f32p))
    return y


def argmax(v):
    v = _f32(v).ravel()
    idx = ctypes.c_uint32()
    rc = lib().orc_argmax(_p(v, _f32p), v.size, ctypes.byref(idx))
    if rc == -1:
        raise OracleError("argmax: NaN input")
    if rc:
        raise OracleError("argmax: zero-length")
    return idx.value


def softmax_rows(x):
    x = _f32(x)
    out = np.empty_like(x)
    if lib().orc_softmax_rows(_p(x, _f32p), x.shape[0], x.shape[1], _p(out, _f32p)):
        raise OracleError("softmax: NaN input")
    return out


def topk_rows(x, k):
    x = _f32(x)
    vals = np.empty((x.shape[0], k), np.float32)
    idx = np.empty((x.shape[0], k), np.uint32)
    rc = lib().orc_topk_rows(_p(x, _f32p), x.shape[0], x.shape[1], k, _p(vals, _f32p), _p(idx, _u32p))
    if rc:
        raise OracleError("topk failed")
    return vals, idx


def moe_forward(x, router_logits, top_k, gu_packed, gu_scales, gu_bias, dn_packed, dn_scales, dn_bias, inter,
                swiglu_limit=7.0, faithful=False):
    x = _f32(x)
    T, H = x.shape
    logits = _f32(router_logits)
    E = logits.shape[1]
    out = np.zeros((T, H), np.float32)
    ti = np.zeros((T, top_k), np.uint32)
    tw = np.zeros((T, top_k), np.float32)
    gp, gs, dp, ds = _u8(gu_packed), _u8(gu_scales), _u8(dn_packed), _u8(dn_scales)
    gb, db = _f32(gu_bias), _f32(dn_bias)
    rc = lib().orc_moe_forward_mxfp4(_p(x, _f32p), T, H, _p(logits, _f32p), E, top_k, _p(gp, _u8p), _p(gs, _u8p),
                                     _p(gb, _f32p), _p(dp, _u8p), _p(ds, _u8p), _p(db, _f32p), inter,
                                     ctypes.c_float(swiglu_limit), 1 if faithful else 0, _p(out, _f32p),
                                     _p(ti, _u32p), _p(tw, _f32p))
    if rc:
        raise OracleError(f"moe_forward failed ({rc})")
    return out, ti, tw


def router_logits(x, weight, bias=None):
    """The router Linear (crates/nn-core/src/layers/core_layers.rs:118-140): x @ W^T,
    then + bias, in f32."""
    y = matmul_xwt(x, weight)
    if bias is not None:
        y = (y + _f32(bias)[None, :]).astype(np.float32)
    return y


def silu_mul(g, u):
    g, u = _f32(g), _f32(u)
    h = np.empty_like(g)
    lib().orc_silu_mul(_p(g, _f32p), _p(u, _f32p), g.size, _p(h, _f32p))
    return h


_LINEAR = {8: lambda x, b, n: q8_0_matmul(x, b, n), 12: lambda x, b, n: q4k_linear(x, b, n),
           14: lambda x, b, n: q6k_linear(x, b, n)}


def mlp_forward(x, gate, up, down, hidden, inter):
    """Qwen3MLP::forward (crates/nn-qwen3/src/layers.rs:40-47) over quantized weights:
    each of gate / up / down is (format id, block bytes) with W[out, in] rows, the
    linear layers as QLinear::forward / quantized_matmul restate them.  Returns the
    output and whether check_output_finite would fail."""
    x = _f32(x)
    g = _LINEAR[gate[0]](x, gate[1], inter)
    u = _LINEAR[up[0]](x, up[1], inter)
    h = silu_mul(g, u)
    y = _LINEAR[down[0]](h, down[1], hidden)
    return y, bool(lib().orc_any_nonfinite(_p(y, _f32p), y.size))


def argmax_slice(v):
    v = _f32(v).ravel()
    return int(lib().orc_argmax_slice(_p(v, _f32p), v.size))


def sample_token(logits, temperature=0.7, top_k=50, top_p=0.9, repetition_penalty=1.0, frequency_penalty=0.0,
                 past_tokens=(), seed=0):
    """sample_token (crates/nn-gptoss/src/sampling.rs:136-185); top_k / top_p None disable
    the step, as the reference's Option fields do."""
    lg = _f32(logits).ravel()
    past = np.ascontiguousarray(np.asarray(() if past_tokens is None else past_tokens, np.uint32).ravel())
    out = ctypes.c_uint32()
    rc = lib().orc_sample_token(_p(lg, _f32p), lg.size, _p(past, _u32p) if past.size else None, past.size,
                                ctypes.c_float(temperature), -1 if top_k is None else int(top_k),
                                0 if top_p is None else 1, ctypes.c_float(0.0 if top_p is None else top_p),
                                ctypes.c_float(repetition_penalty), ctypes.c_float(frequency_penalty),
                                ctypes.c_uint64(seed), ctypes.byref(out))
    if rc:
        raise OracleError("sample_token: empty logits or temperature not positive and finite")
    return out.value


def splitmix64(z: int) -> int:
    return lib().orc_splitmix64(ctypes.c_uint64(z & 0xFFFFFFFFFFFFFFFF))


# ---- nn-reftest comparison semantics ----------------------------------------------
def compare(ref, cand, abs_tol=1e-5):
    """Metrics as in crates/nn-reftest/src/compare.rs:22-120.

    Returns dict(max_abs, max_rel, cosine, normwise) where max_rel skips pairs with
    both |r| and |c| below ``abs_tol`` and ``normwise`` = max|c-r| / max|r|.
    """
    r = np.asarray(ref, np.float32).ravel()
    c = np.asarray(cand, np.float32).ravel()
    assert r.shape == c.shape and r.size > 0
    if not (np.isfinite(r).all() and np.isfinite(c).all()):
        return dict(max_abs=np.inf, max_rel=np.inf, cosine=float("nan"), normwise=np.inf)
    d = np.abs(r - c)
    keep = (np.abs(r) >= abs_tol) | (np.abs(c) >= abs_tol)
    denom = np.maximum(np.maximum(np.abs(r), np.abs(c)), 1e-8)
    max_rel = float((d[keep] / denom[keep]).max()) if keep.any() else 0.0
    r64, c64 = r.astype(np.float64), c.astype(np.float64)
    nr, nc = float(np.dot(r64, r64)), float(np.dot(c64, c64))
    if nr == 0.0 and nc == 0.0:
        cos = 1.0
    elif nr == 0.0 or nc == 0.0:
        cos = 0.0
    else:
        cos = float(np.dot(r64, c64) / (np.sqrt(nr) * np.sqrt(nc)))
    mr = float(np.abs(r).max())
    return dict(max_abs=float(d.max()), max_rel=max_rel, cosine=cos, normwise=float(d.max()) / mr if mr else float(d.max()))


def row_cosines(ref, cand):
    """Per-row cosine similarity in f64 (rows along the first axis)."""
    r = np.asarray(ref, np.float64).reshape(ref.shape[0], -1)
    c = np.asarray(cand, np.float64).reshape(cand.shape[0], -1)
    num = (r * c).sum(1)
    den = np.sqrt((r * r).sum(1)) * np.sqrt((c * c).sum(1))
    out = np.ones(r.shape[0])
    nz = den > 0
    out[nz] = num[nz] / den[nz]
    return out
