"""GGUF ingest over the C ABI (nnq_gguf_*): a memory-mapped GGUF v3 file whose
quantized tensors become device weights straight from the mapped bytes.

Mirrors nn-gguf's GgufFile (crates/nn-gguf/src/reader.rs): ``tensors`` (name -> info,
shape as stored), ``metadata(key)``, ``tensor_data(name)`` (the raw bytes) and, in place
of read_tensor_f32 + Linear, ``weight(name)`` -> QuantizedWeight.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, Tuple

import numpy as np
import torch

from . import _lib
from .quantized import Layout, QuantizedWeight, QuantType, _check, init

# GGUF metadata value type ids (metadata.rs:139-222)
_U, _I, _F = {0, 2, 4, 7, 10}, {1, 3, 5, 11}, {6, 12}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: Tuple[int, ...]
    dtype: int          # GGUF type id (GgufDType)
    offset: int         # from the start of the data section
    nbytes: int


class GgufFile:
    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _check(_lib.load().nnq_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        ver, nt, nm, off = ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_uint64()
        _check(_lib.load().nnq_gguf_info(h, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nm), ctypes.byref(off)))
        self.version, self.data_offset, self.metadata_count = ver.value, off.value, nm.value
        self.tensors: Dict[str, TensorInfo] = {}
        self.tensor_order = []
        dims = (ctypes.c_uint64 * 8)()
        for i in range(nt.value):
            name, nd, dt, to, nb = ctypes.c_char_p(), ctypes.c_int32(), ctypes.c_uint32(), ctypes.c_uint64(), \
                ctypes.c_uint64()
            _check(_lib.load().nnq_gguf_tensor_info(h, i, ctypes.byref(name), ctypes.byref(nd), dims,
                                                    ctypes.byref(dt), ctypes.byref(to), ctypes.byref(nb)))
            info = TensorInfo(name.value.decode(), tuple(int(dims[d]) for d in range(nd.value)), dt.value, to.value,
                              nb.value)
            self.tensors[info.name] = info  # a repeated name keeps its last entry
            self.tensor_order.append(info)

    def close(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _lib.load().nnq_gguf_close(h)
            self._h = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def metadata(self, key: str):
        """The value of `key`: int / float / bool / str, or (element type, count) for arrays."""
        t, u, i, f = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_int64(), ctypes.c_double()
        s, at, ac = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint64()
        _check(_lib.load().nnq_gguf_metadata(self._h, key.encode(), ctypes.byref(t), ctypes.byref(u), ctypes.byref(i),
                                             ctypes.byref(f), ctypes.byref(s), ctypes.byref(at), ctypes.byref(ac)))
        if t.value == 7:
            return bool(u.value)
        if t.value in _U:
            return int(u.value)
        if t.value in _I:
            return int(i.value)
        if t.value in _F:
            return float(f.value)
        if t.value == 8:
            return s.value.decode()
        return ("array", int(at.value), int(ac.value))

    def tensor_data(self, name: str) -> np.ndarray:
        """The tensor's bytes (a copy of the mapped range, read-only use)."""
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(_lib.load().nnq_gguf_tensor_data(self._h, name.encode(), ctypes.byref(p), ctypes.byref(n)))
        return np.frombuffer(ctypes.string_at(p.value, n.value), np.uint8)

    def weight(self, name: str, layout: Layout = Layout.NN_GGUF, ggml_order: bool = False,
               device: int = 0) -> QuantizedWeight:
        """A device weight from a 2-D Q8_0 / Q4_K / Q6_K tensor, with no f32 expansion."""
        info = self.tensors[name]
        init(device)
        h = ctypes.c_void_p()
        with torch.cuda.device(device):
            _check(_lib.load().nnq_gguf_weight_create(self._h, name.encode(), int(layout), 1 if ggml_order else 0,
                                                      ctypes.byref(h)))
        n, k = (info.shape[1], info.shape[0]) if ggml_order else (info.shape[0], info.shape[1])
        return QuantizedWeight(h, QuantType(info.dtype), Layout(layout), (n, k), device)
