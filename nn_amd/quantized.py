"""Host-side mirror of nn's quantized-linear operator surface over the nnq C ABI.

The names, argument meaning and errors follow the reference's op layer:
``QuantType`` / ``DynTensor::from_quantized`` (crates/nn-core/src/dyn_tensor/quantized.rs:26-140,270-278),
``quantized_linear`` / ``quantized_matmul_q8_0`` and ``QuantizedMatmulError``
(crates/nn-core/src/dyn_tensor/quantized_matmul.rs:30-406), ``BlockQ4K`` / ``QLinear``
(crates/nn-core/src/layers/quantized/linear.rs:49-400), argmax
(crates/nn-core/src/dyn_tensor/ops_ext/argreduce.rs:19-118) and the GPT-OSS MXFP4 MoE
(crates/nn-gptoss/src/quantize.rs:122-188, crates/nn-gptoss/src/quantized_model.rs:99-194).

Tensors are torch tensors used as device-memory handles; every compute call runs a
hand-written HIP kernel through ``libnnq.so`` on torch's current stream.  There is
no CPU fallback: without the library or a GPU these functions raise.
"""
from __future__ import annotations

import ctypes
import enum
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib

# ---------------------------------------------------------------------------------
# errors (TensorError / QuantizedMatmulError kinds)
# ---------------------------------------------------------------------------------


class TensorError(RuntimeError):
    """Base error (crates/nn-core/src/error.rs)."""


class QuantizedMatmulError(TensorError):
    """crates/nn-core/src/dyn_tensor/quantized_matmul.rs:30-82"""


class NotQuantized(QuantizedMatmulError):
    pass


class WrongQuantType(QuantizedMatmulError):
    pass


class ShapeMismatch(QuantizedMatmulError):
    pass


class WeightRank(QuantizedMatmulError):
    pass


class BiasMismatch(QuantizedMatmulError):
    pass


class DataLengthMismatch(TensorError):
    pass


class InvalidShape(TensorError):
    pass


class RankMismatch(TensorError):
    pass


class NonFiniteData(TensorError):
    pass


class Unsupported(TensorError):
    pass


class BackendFailure(TensorError):
    pass


_CODE_TO_EXC = {
    _lib.ERR_INVALID_ARGUMENT: TensorError,
    _lib.ERR_SHAPE_MISMATCH: ShapeMismatch,
    _lib.ERR_WRONG_FORMAT: WrongQuantType,
    _lib.ERR_NOT_QUANTIZED: NotQuantized,
    _lib.ERR_WEIGHT_RANK: WeightRank,
    _lib.ERR_BIAS_MISMATCH: BiasMismatch,
    _lib.ERR_DATA_LENGTH: DataLengthMismatch,
    _lib.ERR_INVALID_SHAPE: InvalidShape,
    _lib.ERR_NON_FINITE: NonFiniteData,
    _lib.ERR_NO_DEVICE: BackendFailure,
    _lib.ERR_OUT_OF_MEMORY: BackendFailure,
    _lib.ERR_DISPATCH_FAILED: BackendFailure,
    _lib.ERR_UNSUPPORTED: Unsupported,
}


def _check(rc: int):
    if rc != _lib.OK:
        raise _CODE_TO_EXC.get(rc, TensorError)(f"[nnq status {rc}] {_lib.last_error()}")


# ---------------------------------------------------------------------------------
# formats
# ---------------------------------------------------------------------------------


class QuantType(enum.IntEnum):
    """Block formats (GGUF type ids, crates/nn-gguf/src/dequant.rs:14-45)."""
    Q8_0 = 8
    Q4_K = 12
    Q6_K = 14
    MXFP4 = 39

    def block_size(self) -> int:
        return 32 if self in (QuantType.Q8_0, QuantType.MXFP4) else 256

    def block_bytes(self) -> int:
        return {QuantType.Q8_0: 34, QuantType.Q4_K: 144, QuantType.Q6_K: 210, QuantType.MXFP4: 17}[self]

    def expected_bytes(self, num_elements: int) -> Optional[int]:
        """QuantType::expected_bytes (quantized.rs:79-89)."""
        if num_elements == 0:
            return 0
        if num_elements % self.block_size():
            return None
        return num_elements // self.block_size() * self.block_bytes()


class Layout(enum.IntEnum):
    GGUF = 0       # GGUF spec: Q8_0, nn-core BlockQ4K
    NN_GGUF = 1    # nn-gguf's own Q4_K / Q6_K decoders
    GPTOSS = 2     # GPT-OSS Mxfp4Tensor
    OCP = 3        # nn-core Mxfp4Block / Mxfp4Tensor (17-byte blocks, low nibble first)


_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_initialised = set()


def init(device: int = 0):
    """nnq_init for `device` (idempotent per process)."""
    if device not in _initialised:
        _check(_lib.load().nnq_init(device))
        _initialised.add(device)


def device_count() -> int:
    c = ctypes.c_int(0)
    _check(_lib.load().nnq_device_count(ctypes.byref(c)))
    return c.value


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _device_input(t: torch.Tensor, what: str, device: Optional[int] = None) -> torch.Tensor:
    """Reject a tensor the kernels cannot read: the C ABI takes device pointers and
    cannot tell a host address from a device one, so a CPU tensor (or one on another
    device than the weights') is refused here, before any launch."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise Unsupported(f"{what} must be a device tensor")
    if device is not None and t.device.index != device:
        raise Unsupported(f"{what} is on cuda:{t.device.index}, the weights on cuda:{device}")
    return t


def _side_input(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """A secondary operand (bias, router logits) as contiguous f32 on the device of `like`."""
    return t.to(device=like.device, dtype=torch.float32).contiguous()


def _as_u8(data) -> np.ndarray:
    if isinstance(data, (bytes, bytearray, memoryview)):
        return np.frombuffer(bytes(data), dtype=np.uint8)
    if isinstance(data, torch.Tensor):
        return data.detach().cpu().contiguous().view(torch.uint8).numpy()
    return np.ascontiguousarray(data, dtype=np.uint8)


# ---------------------------------------------------------------------------------
# quantized weight (DynTensor::from_quantized on the GPU)
# ---------------------------------------------------------------------------------


class QuantizedWeight:
    """Device-resident block-quantized weight W[out_features, in_features].

    Mirrors ``DynTensor::from_quantized(data, quant_type, shape)`` with the
    validation of ``QuantizedStorage::new`` (quantized.rs:121-140): the element
    count must be a block multiple and the byte length must match.
    """

    def __init__(self, handle, quant_type: QuantType, layout: Layout, shape, device: int):
        self._h = handle
        self.quant_type = QuantType(quant_type)
        self.layout = Layout(layout)
        self.shape = tuple(int(s) for s in shape)
        self.device = device

    @classmethod
    def from_quantized(cls, data, quant_type: QuantType, shape: Sequence[int], layout: Layout = Layout.GGUF,
                       device: int = 0) -> "QuantizedWeight":
        quant_type = QuantType(quant_type)
        shape = tuple(int(s) for s in shape)
        if len(shape) != 2:
            raise WeightRank(f"quantized weight must be 2-D [out_features, in_features], got rank {len(shape)}")
        n, k = shape
        num = n * k
        exp = quant_type.expected_bytes(num)
        if exp is None:
            raise InvalidShape(f"element count {num} is not a multiple of {quant_type.name} block size "
                               f"{quant_type.block_size()}")
        buf = _as_u8(data)
        if buf.size != exp:
            raise DataLengthMismatch(f"expected {exp} bytes, got {buf.size}")
        init(device)
        with torch.cuda.device(device):
            h = ctypes.c_void_p()
            _check(_lib.load().nnq_weight_create(int(quant_type), int(layout), buf.ctypes.data_as(ctypes.c_void_p),
                                                 buf.size, n, k, ctypes.byref(h)))
        return cls(h, quant_type, layout, shape, device)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib.load().nnq_weight_destroy(h)
            except Exception:
                pass
            self._h = None

    @property
    def handle(self):
        return self._h

    def device_bytes(self) -> int:
        nb = ctypes.c_size_t()
        _check(_lib.load().nnq_weight_info(self._h, None, None, None, None, ctypes.byref(nb)))
        return nb.value

    def dequantize(self) -> torch.Tensor:
        """Bit-exact f32 decode on the device (QuantizedStorage::dequantize)."""
        out = torch.empty(self.shape, dtype=torch.float32, device=f"cuda:{self.device}")
        _check(_lib.load().nnq_dequant(self._h, _ptr(out), _stream(out)))
        return out


def _validate_input(input: torch.Tensor, in_features: int, device: Optional[int] = None):
    """validate_input (quantized_matmul.rs:121-145)."""
    if input.dim() < 2:
        raise RankMismatch(f"expected rank >= 2, got {input.dim()}")
    k = input.shape[-1]
    if k != in_features:
        raise ShapeMismatch(f"quantized matmul shape mismatch: input last dim {k} != weight in_features {in_features}")
    _device_input(input, "input", device)
    if input.dtype not in (torch.float32, torch.bfloat16):
        input = input.float()
    return input.contiguous()


def quantized_linear(input: torch.Tensor, weight: QuantizedWeight, bias: Optional[torch.Tensor] = None,
                     out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``y = input @ weight^T + bias`` (quantized_matmul.rs:367-406 / QLinear::forward).

    Output dtype is f32 (the fused ops' convention) unless ``out_dtype`` is given
    (bf16 rounds the f32 accumulator once, as the f32 sink does for a bf16 lhs).
    """
    if not isinstance(weight, QuantizedWeight):
        raise NotQuantized("quantized_linear: weight is not quantized")
    n, k = weight.shape
    x = _validate_input(input, k, weight.device)
    if bias is not None:
        if bias.dim() != 1 or bias.shape[0] != n:
            raise BiasMismatch(f"bias shape mismatch: expected [{n}], got {list(bias.shape)}")
        bias = _side_input(bias, x)
    out_dtype = out_dtype or torch.float32
    y = torch.empty(tuple(x.shape[:-1]) + (n,), dtype=out_dtype, device=x.device)
    m = x.numel() // k
    _check(_lib.load().nnq_linear(weight.handle, _ptr(x), _DTYPE[x.dtype], m, k, _ptr(bias),
                                  n if bias is not None else 0, _ptr(y), _DTYPE[out_dtype], _stream(x)))
    return y


def _typed_matmul(expected: QuantType):
    def fn(input: torch.Tensor, weight: QuantizedWeight) -> torch.Tensor:
        if not isinstance(weight, QuantizedWeight):
            raise NotQuantized(f"weight tensor is not quantized (expected {expected.name})")
        if weight.quant_type != expected:
            raise WrongQuantType(f"weight quantization type mismatch: expected {expected.name}, got "
                                 f"{weight.quant_type.name}")
        return quantized_linear(input, weight)
    fn.__name__ = f"quantized_matmul_{expected.name.lower()}"
    return fn


quantized_matmul_q8_0 = _typed_matmul(QuantType.Q8_0)   # quantized_matmul.rs:335-350
quantized_matmul_q4_k = _typed_matmul(QuantType.Q4_K)
quantized_matmul_q6_k = _typed_matmul(QuantType.Q6_K)


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """First-index argmax over a 1-D device f32 tensor; NaN raises NonFiniteData
    (argreduce.rs:94-118).  Synchronizes to read the status."""
    if logits.dim() != 1:
        raise Unsupported("argmax: 1-D input expected")
    if logits.numel() == 0:
        raise InvalidShape("argmax over a zero-length dimension")
    v = _device_input(logits, "logits").float().contiguous()
    idx = torch.empty(1, dtype=torch.int32, device=v.device)
    st = torch.zeros(1, dtype=torch.int32, device=v.device)
    _check(_lib.load().nnq_argmax_f32(_ptr(v), v.numel(), _ptr(idx), _ptr(st), _stream(v)))
    if int(st.item()) != 0:
        raise NonFiniteData("argmax/argmin input contains NaN")
    return idx.view(torch.int32)[0].to(torch.int64)


def linear_argmax(x: torch.Tensor, weight: QuantizedWeight, bias: Optional[torch.Tensor] = None,
                  check: bool = True):
    """LM head: logits = x @ W^T (+bias) and their first-index argmax, fused."""
    n, k = weight.shape
    xv = _device_input(x, "x", weight.device).reshape(-1).float().contiguous()
    if xv.numel() != k:
        raise ShapeMismatch(f"input has {xv.numel()} elements, weight in_features {k}")
    if bias is not None:
        if bias.dim() != 1 or bias.shape[0] != n:
            raise BiasMismatch(f"bias shape mismatch: expected [{n}], got {list(bias.shape)}")
        bias = _side_input(bias, xv)
    logits = torch.empty(n, dtype=torch.float32, device=xv.device)
    idx = torch.empty(1, dtype=torch.int32, device=xv.device)
    st = torch.zeros(1, dtype=torch.int32, device=xv.device)
    _check(_lib.load().nnq_linear_argmax(weight.handle, _ptr(xv), k, _ptr(bias), n if bias is not None else 0,
                                         _ptr(logits), _ptr(idx), _ptr(st), _stream(xv)))
    if check and int(st.item()) != 0:
        raise NonFiniteData("argmax input contains NaN")
    return logits, idx[0].to(torch.int64)


# ---------------------------------------------------------------------------------
# token sampling (crates/nn-gptoss/src/sampling.rs)
# ---------------------------------------------------------------------------------


def _sampling(temperature, top_k, top_p, repetition_penalty, frequency_penalty, seed):
    return _lib.Sampling(float(temperature), -1 if top_k is None else int(top_k), 0 if top_p is None else 1,
                         0.0 if top_p is None else float(top_p), float(repetition_penalty), float(frequency_penalty),
                         int(seed) & 0xFFFFFFFFFFFFFFFF)


def _past(past_tokens, device):
    if past_tokens is None or len(past_tokens) == 0:
        return None, 0
    if isinstance(past_tokens, torch.Tensor):
        p = past_tokens.to(device=device, dtype=torch.int32).contiguous()
    else:
        p = torch.tensor(np.asarray(past_tokens, np.int64).astype(np.uint32).view(np.int32), device=device)
    return p, p.numel()


def sample_token(logits: torch.Tensor, temperature: float = 0.7, top_k: Optional[int] = 50,
                 top_p: Optional[float] = 0.9, repetition_penalty: float = 1.0, frequency_penalty: float = 0.0,
                 past_tokens=None, seed: int = 0) -> torch.Tensor:
    """sample_token (sampling.rs:136-185) over a 1-D device f32 logits tensor; returns the
    token as a device int64 scalar tensor (no host synchronisation)."""
    v = _device_input(logits, "logits").reshape(-1).float().contiguous()
    if v.numel() == 0:
        raise InvalidShape("logits must be non-empty")
    past, n_past = _past(past_tokens, v.device)
    tok = torch.empty(1, dtype=torch.int32, device=v.device)
    cfg = _sampling(temperature, top_k, top_p, repetition_penalty, frequency_penalty, seed)
    _check(_lib.load().nnq_sample_token(_ptr(v), v.numel(), _ptr(past), n_past, ctypes.byref(cfg), _ptr(tok),
                                        _stream(v)))
    return tok.view(torch.int32)[0].to(torch.int64)


def linear_sample(x: torch.Tensor, weight: QuantizedWeight, bias: Optional[torch.Tensor] = None,
                  temperature: float = 0.7, top_k: Optional[int] = 50, top_p: Optional[float] = 0.9,
                  repetition_penalty: float = 1.0, frequency_penalty: float = 0.0, past_tokens=None, seed: int = 0):
    """LM head + sampling: logits = x @ W^T (+bias), then sample_token on the device."""
    n, k = weight.shape
    xv = _device_input(x, "x", weight.device).reshape(-1).float().contiguous()
    if xv.numel() != k:
        raise ShapeMismatch(f"input has {xv.numel()} elements, weight in_features {k}")
    if bias is not None:
        if bias.dim() != 1 or bias.shape[0] != n:
            raise BiasMismatch(f"bias shape mismatch: expected [{n}], got {list(bias.shape)}")
        bias = _side_input(bias, xv)
    logits = torch.empty(n, dtype=torch.float32, device=xv.device)
    past, n_past = _past(past_tokens, xv.device)
    tok = torch.empty(1, dtype=torch.int32, device=xv.device)
    cfg = _sampling(temperature, top_k, top_p, repetition_penalty, frequency_penalty, seed)
    _check(_lib.load().nnq_linear_sample(weight.handle, _ptr(xv), k, _ptr(bias), n if bias is not None else 0,
                                         _ptr(logits), _ptr(past), n_past, ctypes.byref(cfg), _ptr(tok), _stream(xv)))
    return logits, tok.view(torch.int32)[0].to(torch.int64)


# ---------------------------------------------------------------------------------
# Qwen3 SwiGLU MLP
# ---------------------------------------------------------------------------------


class QuantizedMLP:
    """Device-resident Qwen3 MLP over quantized weights: gate_proj and up_proj
    W[inter, hidden] in one format / layout, down_proj W[hidden, inter]
    (crates/nn-qwen3/src/layers.rs:19-48).  ``forward`` raises NonFiniteData when an
    output is NaN or infinite, as check_output_finite does (it synchronizes to read
    the status; ``check=False`` skips that)."""

    def __init__(self, gate, up, down, quant_type: QuantType, hidden: int, inter: int,
                 down_type: Optional[QuantType] = None, layout: Layout = Layout.GGUF,
                 down_layout: Optional[Layout] = None, device: int = 0):
        qt = QuantType(quant_type)
        dt = QuantType(down_type if down_type is not None else quant_type)
        dl = Layout(down_layout if down_layout is not None else layout)
        g, u, d = _as_u8(gate), _as_u8(up), _as_u8(down)
        if g.size != u.size:
            raise DataLengthMismatch(f"gate ({g.size} bytes) and up ({u.size} bytes) differ")
        init(device)
        h = ctypes.c_void_p()
        vp = ctypes.c_void_p
        with torch.cuda.device(device):
            _check(_lib.load().nnq_mlp_create(int(qt), int(layout), g.ctypes.data_as(vp), u.ctypes.data_as(vp), g.size,
                                              int(dt), int(dl), d.ctypes.data_as(vp), d.size, int(hidden), int(inter),
                                              ctypes.byref(h)))
        self._h = h
        self.hidden, self.inter, self.device = int(hidden), int(inter), device

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib.load().nnq_mlp_destroy(h)
            except Exception:
                pass
            self._h = None

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None, check: bool = True) -> torch.Tensor:
        """down(silu(gate(x)) * up(x)) over the last dimension of x (Qwen3MLP::forward)."""
        _validate_input(x, self.hidden, self.device)
        xx = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
        xx = xx.reshape(-1, self.hidden).contiguous()
        m = xx.shape[0]
        od = out_dtype if out_dtype is not None else torch.float32
        y = torch.empty((m, self.hidden), dtype=od, device=xx.device)
        st = torch.zeros(1, dtype=torch.int32, device=xx.device)
        _check(_lib.load().nnq_mlp_forward(self._h, _ptr(xx), _DTYPE[xx.dtype], m, self.hidden, _ptr(y), _DTYPE[od],
                                           _ptr(st), _stream(xx)))
        if check and m > 0 and int(st.item()) != 0:
            raise NonFiniteData("Qwen3MLP output contains NaN or Inf")
        return y.reshape(*x.shape[:-1], self.hidden)

    __call__ = forward


# ---------------------------------------------------------------------------------
# GPT-OSS MXFP4 mixture of experts
# ---------------------------------------------------------------------------------


class QuantizedMoE:
    """Device-resident GPT-OSS MXFP4 expert weights of one layer.

    gate_up: Mxfp4Tensor (packed, scales) of the flat [E, hidden, 2*inter] tensor;
    down: of the flat [E, inter, hidden] tensor; biases f32 [E, 2*inter], [E, hidden]
    (crates/nn-gptoss/src/quantized_model.rs:44-97).
    """

    def __init__(self, num_experts, hidden, inter, gu_packed, gu_scales, gu_bias, dn_packed, dn_scales, dn_bias,
                 device: int = 0, router_weight=None, router_bias=None):
        E, H, I = int(num_experts), int(hidden), int(inter)
        gp, gs, dp, ds = (_as_u8(a) for a in (gu_packed, gu_scales, dn_packed, dn_scales))
        if gp.size != E * H * 2 * I // 2 or gs.size != E * H * 2 * I // 32:
            raise DataLengthMismatch("gate_up MXFP4 byte count does not match [E, hidden, 2*inter]")
        if dp.size != E * I * H // 2 or ds.size != E * I * H // 32:
            raise DataLengthMismatch("down MXFP4 byte count does not match [E, inter, hidden]")
        gb = np.ascontiguousarray(np.asarray(gu_bias, np.float32).reshape(E, 2 * I))
        db = np.ascontiguousarray(np.asarray(dn_bias, np.float32).reshape(E, H))
        init(device)
        h = ctypes.c_void_p()
        vp = ctypes.c_void_p
        with torch.cuda.device(device):
            _check(_lib.load().nnq_moe_create(E, H, I, gp.ctypes.data_as(vp), gs.ctypes.data_as(vp),
                                              gb.ctypes.data_as(vp), dp.ctypes.data_as(vp), ds.ctypes.data_as(vp),
                                              db.ctypes.data_as(vp), ctypes.byref(h)))
        self._h = h
        self._router = None
        self.num_experts, self.hidden, self.inter, self.device = E, H, I, device
        self._attach_router(router_weight, router_bias)

    @classmethod
    def from_ocp(cls, num_experts, hidden, inter, gu_blocks, gu_bias, dn_blocks, dn_bias, device: int = 0,
                 router_weight=None, router_bias=None) -> "QuantizedMoE":
        """The same layer from nn-core OCP MXFP4 tensors (mxfp4.rs quantize_tensor of the
        flat [E, hidden, 2*inter] and [E, inter, hidden] weights: 17-byte blocks)."""
        E, H, I = int(num_experts), int(hidden), int(inter)
        gb_, db_ = _as_u8(gu_blocks), _as_u8(dn_blocks)
        if gb_.size != E * H * 2 * I // 32 * 17:
            raise DataLengthMismatch("gate_up OCP MXFP4 byte count does not match [E, hidden, 2*inter]")
        if db_.size != E * I * H // 32 * 17:
            raise DataLengthMismatch("down OCP MXFP4 byte count does not match [E, inter, hidden]")
        gb = np.ascontiguousarray(np.asarray(gu_bias, np.float32).reshape(E, 2 * I))
        db = np.ascontiguousarray(np.asarray(dn_bias, np.float32).reshape(E, H))
        init(device)
        h = ctypes.c_void_p()
        vp = ctypes.c_void_p
        with torch.cuda.device(device):
            _check(_lib.load().nnq_moe_create_ocp(E, H, I, gb_.ctypes.data_as(vp), gb.ctypes.data_as(vp),
                                                  db_.ctypes.data_as(vp), db.ctypes.data_as(vp), ctypes.byref(h)))
        self = object.__new__(cls)
        self._h = h
        self._router = None
        self.num_experts, self.hidden, self.inter, self.device = E, H, I, device
        self._attach_router(router_weight, router_bias)
        return self

    def _attach_router(self, router_weight, router_bias):
        E, H, device = self.num_experts, self.hidden, self.device
        vp = ctypes.c_void_p
        if router_weight is not None:
            rw = np.ascontiguousarray(np.asarray(router_weight, np.float32))
            if rw.shape != (E, H):
                raise ShapeMismatch(f"router weight must be [{E}, {H}], got {list(rw.shape)}")
            rb = None if router_bias is None else np.ascontiguousarray(np.asarray(router_bias, np.float32))
            if rb is not None and rb.shape != (E,):
                raise BiasMismatch(f"router bias must be [{E}], got {list(rb.shape)}")
            r = ctypes.c_void_p()
            with torch.cuda.device(device):
                _check(_lib.load().nnq_router_create(E, H, rw.ctypes.data_as(vp),
                                                     None if rb is None else rb.ctypes.data_as(vp), ctypes.byref(r)))
            self._router = r

    def __del__(self):
        for name, fn in (("_router", "nnq_router_destroy"), ("_h", "nnq_moe_destroy")):
            h = getattr(self, name, None)
            if h is not None and h.value:
                try:
                    getattr(_lib.load(), fn)(h)
                except Exception:
                    pass
                setattr(self, name, None)

    def _input(self, x):
        _device_input(x, "x", self.device)
        if x.dim() != 2 or x.shape[1] != self.hidden:
            raise ShapeMismatch(f"x must be [tokens, {self.hidden}]")
        return x.contiguous() if x.dtype in (torch.float32, torch.bfloat16) else x.float().contiguous()

    def router_logits(self, x: torch.Tensor) -> torch.Tensor:
        """The router Linear alone: x @ W^T + b in f32 (quantized_model.rs:138)."""
        if self._router is None:
            raise Unsupported("this MoE was created without a router")
        xx = self._input(x)
        lg = torch.empty((xx.shape[0], self.num_experts), dtype=torch.float32, device=xx.device)
        _check(_lib.load().nnq_router_logits(self._router, _ptr(xx), _DTYPE[xx.dtype], xx.shape[0], _ptr(lg),
                                             _stream(xx)))
        return lg

    def block_forward(self, x: torch.Tensor, top_k: int = 4, swiglu_limit: float = 7.0,
                      return_routing: bool = False, check: bool = True):
        """moe_forward with its router (quantized_model.rs:132-194): logits, routing,
        experts and combine on the device; NonFiniteData when an output is NaN or
        infinite (check_output_finite; synchronizes to read the status unless check=False)."""
        if self._router is None:
            raise Unsupported("this MoE was created without a router")
        xx = self._input(x)
        T = xx.shape[0]
        if top_k <= 0 or top_k > self.num_experts:
            raise InvalidShape(f"topk k={top_k} out of range for dim 1 (size {self.num_experts})")
        y = torch.empty((T, self.hidden), dtype=torch.float32, device=xx.device)
        ti = torch.empty((T, top_k), dtype=torch.int32, device=xx.device) if return_routing else None
        tw = torch.empty((T, top_k), dtype=torch.float32, device=xx.device) if return_routing else None
        st = torch.zeros(1, dtype=torch.int32, device=xx.device)
        _check(_lib.load().nnq_moe_block_forward(self._h, self._router, _ptr(xx), _DTYPE[xx.dtype], T, int(top_k),
                                                 float(swiglu_limit), _ptr(y), _ptr(ti), _ptr(tw), _ptr(st),
                                                 _stream(xx)))
        if check and T > 0 and int(st.item()) != 0:
            raise NonFiniteData("QuantizedMoeBlock output contains NaN or Inf")
        if return_routing:
            return y, ti, tw
        return y

    def forward(self, x: torch.Tensor, router_logits: torch.Tensor, top_k: int = 4, swiglu_limit: float = 7.0,
                return_routing: bool = False):
        """moe_forward (quantized_model.rs:132-194) with router logits given."""
        xx = self._input(x)
        T = xx.shape[0]
        if router_logits.shape != (T, self.num_experts):
            raise ShapeMismatch(f"router logits must be [{T}, {self.num_experts}]")
        if top_k <= 0 or top_k > self.num_experts:
            raise InvalidShape(f"topk k={top_k} out of range for dim 1 (size {self.num_experts})")
        lg = _side_input(router_logits, xx)
        y = torch.empty((T, self.hidden), dtype=torch.float32, device=xx.device)
        ti = torch.empty((T, top_k), dtype=torch.int32, device=xx.device) if return_routing else None
        tw = torch.empty((T, top_k), dtype=torch.float32, device=xx.device) if return_routing else None
        _check(_lib.load().nnq_moe_forward(self._h, _ptr(xx), _DTYPE[xx.dtype], T, _ptr(lg), int(top_k),
                                           float(swiglu_limit), _ptr(y), _ptr(ti), _ptr(tw), _stream(xx)))
        if return_routing:
            return y, ti, tw
        return y

    __call__ = forward

    def dequant_expert(self, e: int):
        gu = torch.empty((self.hidden, 2 * self.inter), dtype=torch.float32, device=f"cuda:{self.device}")
        dn = torch.empty((self.inter, self.hidden), dtype=torch.float32, device=f"cuda:{self.device}")
        _check(_lib.load().nnq_moe_dequant_expert(self._h, int(e), _ptr(gu), _ptr(dn), _stream(gu)))
        return gu, dn


# ---------------------------------------------------------------------------------
# host encoders and the seeded generator (CPU; no device needed)
# ---------------------------------------------------------------------------------


def _f32c(v) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(v, dtype=np.float32).ravel())


def quantize_q4_k(values) -> np.ndarray:
    """BlockQ4K::quantize over the flat values, zero-padded to 256 (QLinear::from_linear)."""
    v = _f32c(values)
    out = np.zeros((v.size + 255) // 256 * 144, np.uint8)
    _check(_lib.load().nnq_quantize_q4_k(v.ctypes.data_as(ctypes.c_void_p), v.size,
                                         out.ctypes.data_as(ctypes.c_void_p)))
    return out


def quantize_q8_0(values) -> np.ndarray:
    v = _f32c(values)
    out = np.zeros(v.size // 32 * 34, np.uint8)
    _check(_lib.load().nnq_quantize_q8_0(v.ctypes.data_as(ctypes.c_void_p), v.size,
                                         out.ctypes.data_as(ctypes.c_void_p)))
    return out


def quantize_q6_k(values) -> np.ndarray:
    v = _f32c(values)
    out = np.zeros(v.size // 256 * 210, np.uint8)
    _check(_lib.load().nnq_quantize_q6_k(v.ctypes.data_as(ctypes.c_void_p), v.size,
                                         out.ctypes.data_as(ctypes.c_void_p)))
    return out


def quantize_mxfp4(values):
    """Mxfp4Tensor::quantize -> (packed, scales)."""
    v = _f32c(values)
    nb = (v.size + 31) // 32
    packed = np.zeros(nb * 16, np.uint8)
    scales = np.zeros(nb, np.uint8)
    _check(_lib.load().nnq_quantize_mxfp4(v.ctypes.data_as(ctypes.c_void_p), v.size,
                                          packed.ctypes.data_as(ctypes.c_void_p),
                                          scales.ctypes.data_as(ctypes.c_void_p)))
    return packed, scales


def quantize_mxfp4_ocp(values) -> np.ndarray:
    """nn-core mxfp4 quantize_tensor (crates/nn-core/src/layers/quantized/mxfp4.rs:293-315)
    of the flattened values: ceil(n / 32) 17-byte blocks; NonFiniteData on NaN / inf."""
    v = _f32c(values)
    out = np.zeros(((v.size + 31) // 32) * 17, np.uint8)
    _check(_lib.load().nnq_quantize_mxfp4_ocp(v.ctypes.data_as(ctypes.c_void_p), v.size,
                                              out.ctypes.data_as(ctypes.c_void_p)))
    return out


def dequantize_mxfp4_ocp(blocks, n: int, device: int = 0) -> torch.Tensor:
    """nn-core mxfp4 dequantize_tensor on the device (bit-exact): the first n values of
    the 17-byte blocks (a host array or a device uint8 tensor), as a device f32 tensor."""
    if isinstance(blocks, torch.Tensor) and blocks.is_cuda:
        b = blocks.contiguous().view(torch.uint8)
    else:
        b = torch.from_numpy(_as_u8(blocks).copy()).to(f"cuda:{device}")
    if b.numel() < ((int(n) + 31) // 32) * 17:
        raise DataLengthMismatch(f"{b.numel()} bytes hold fewer than {n} values")
    out = torch.empty(int(n), dtype=torch.float32, device=b.device)
    _check(_lib.load().nnq_dequant_mxfp4_ocp(_ptr(b), int(n), _ptr(out), _stream(out)))
    return out


def synth_normal(seed: int, tensor_id: int, shape, sigma: float = 1.0) -> np.ndarray:
    """Seeded N(0, sigma) f32 values (splitmix64 + Box-Muller)."""
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    _check(_lib.load().nnq_synth_normal(int(seed) & (2**64 - 1), int(tensor_id) & (2**64 - 1), n, float(sigma),
                                        out.ctypes.data_as(ctypes.c_void_p)))
    return out.reshape(shape)
