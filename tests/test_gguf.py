"""GGUF ingest (nnq_gguf_*): the reader against files written per the GGUF v3 layout
(tests/gguf_writer.py), the reference's header and limit cases
(crates/nn-gguf/src/header.rs:133-168, tensor_info.rs, metadata.rs, reader.rs:68-141),
and, on the GPU, weights uploaded straight from the mapped bytes against weights built
from the same bytes in memory (identical device images, bit-identical outputs) and
against the oracle."""
import struct

import numpy as np
import pytest

import gguf_writer as GW


def open_gguf(tmp_path, blob, name="t.gguf"):
    from nn_amd.gguf import GgufFile
    p = tmp_path / name
    p.write_bytes(blob)
    return GgufFile(str(p))


def qwen_like(O):
    """Q4_K gate/up/down and a Q6_K LM head of a tiny Qwen-style model, plus f32 norms."""
    import nn_amd
    H, I, V = 256, 512, 1000
    wg = O.quantize_q4_k(nn_amd.synth_normal(1, 1, (I, H), 0.05))
    wu = O.quantize_q4_k(nn_amd.synth_normal(1, 2, (I, H), 0.05))
    wd = O.quantize_q4_k(nn_amd.synth_normal(1, 3, (H, I), 0.05))
    wo = O.quantize_q6_k(nn_amd.synth_normal(1, 4, (V, H), 0.05))
    w8 = O.quantize_q8_0(nn_amd.synth_normal(1, 5, (96, 64), 0.05))
    norm = np.arange(H, dtype=np.float32) * 0.01
    meta = [("general.architecture", GW.STRING, "qwen2"), ("qwen2.embedding_length", GW.U32, H),
            ("qwen2.feed_forward_length", GW.U32, I), ("qwen2.attention.layer_norm_rms_epsilon", GW.F32, 1e-6),
            ("qwen2.rope.freq_base", GW.F64, 1e6), ("general.flag", GW.BOOL, True), ("neg", GW.I64, -5),
            ("tokenizer.ggml.tokens", GW.ARRAY, (GW.STRING, ["a", "bb", "ccc"])),
            ("nested", GW.ARRAY, (GW.ARRAY, [(GW.U8, [1, 2]), (GW.U8, [3])]))]
    tensors = [("blk.0.ffn_gate.weight", [I, H], 12, wg.tobytes()), ("blk.0.ffn_up.weight", [I, H], 12, wu.tobytes()),
               ("blk.0.ffn_down.weight", [H, I], 12, wd.tobytes()), ("output_norm.weight", [H], 0, norm.tobytes()),
               ("output.weight", [V, H], 14, wo.tobytes()), ("small.q8", [96, 64], 8, w8.tobytes())]
    return meta, tensors


def test_gguf_parse_round_trip(O, tmp_path):
    meta, tensors = qwen_like(O)
    blob, base = GW.build(meta, tensors)
    g = open_gguf(tmp_path, blob)
    assert g.version == 3 and g.data_offset == base and base % 32 == 0
    assert g.metadata_count == len(meta)
    assert g.metadata("general.architecture") == "qwen2"
    assert g.metadata("qwen2.embedding_length") == 256
    assert abs(g.metadata("qwen2.attention.layer_norm_rms_epsilon") - 1e-6) < 1e-12
    assert g.metadata("qwen2.rope.freq_base") == 1e6
    assert g.metadata("general.flag") is True and g.metadata("neg") == -5
    assert g.metadata("tokenizer.ggml.tokens") == ("array", GW.STRING, 3)
    assert g.metadata("nested") == ("array", GW.ARRAY, 2)
    assert [t.name for t in g.tensor_order] == [t[0] for t in tensors]
    off = 0
    for name, dims, dtype, data in tensors:
        info = g.tensors[name]
        assert info.shape == tuple(dims) and info.dtype == dtype and info.offset == off and info.nbytes == len(data)
        assert g.tensor_data(name).tobytes() == data
        off += len(data)
    g.close()


def test_gguf_header_cases(O, tmp_path):
    """The reference's header tests (header.rs:133-168): valid header, magic 0xDEADBEEF,
    version 2; and a truncated header."""
    import nn_amd
    from nn_amd.gguf import GgufFile
    ok = struct.pack("<IIQQ", GW.MAGIC, 3, 0, 0)
    g = open_gguf(tmp_path, ok)
    assert g.version == 3 and len(g.tensors) == 0 and g.data_offset == 32
    with pytest.raises(nn_amd.WrongQuantType):
        open_gguf(tmp_path, struct.pack("<I", 0xDEADBEEF) + ok[4:], "m.gguf")
    with pytest.raises(nn_amd.WrongQuantType):
        open_gguf(tmp_path, struct.pack("<IIQQ", GW.MAGIC, 2, 0, 0), "v.gguf")
    with pytest.raises(nn_amd.DataLengthMismatch):
        open_gguf(tmp_path, ok[:12], "s.gguf")
    with pytest.raises(nn_amd.TensorError):
        GgufFile(str(tmp_path / "missing.gguf"))


def test_gguf_limits_and_bounds(O, tmp_path):
    import nn_amd
    d = np.zeros(64, np.float32).tobytes()
    cases = {
        "zero_dim": (GW.build([], [("z", [0, 4], 0, b"")])[0], nn_amd.InvalidShape),
        "nine_dims": (GW.build([], [("n", [1] * 9, 0, d[:4])])[0], nn_amd.InvalidShape),
        "unknown_dtype": (GW.build([], [("u", [4], 99, d[:16])])[0], nn_amd.WrongQuantType),
        "out_of_bounds": (GW.build([], [("o", [64], 0, d)], offsets=[0])[0][:-4], nn_amd.DataLengthMismatch),
        "tensor_count": (struct.pack("<IIQQ", GW.MAGIC, 3, 100001, 0), nn_amd.InvalidShape),
        "kv_count": (struct.pack("<IIQQ", GW.MAGIC, 3, 0, 100001), nn_amd.InvalidShape),
        "long_string": (struct.pack("<IIQQ", GW.MAGIC, 3, 0, 1) + struct.pack("<Q", (16 << 20) + 1),
                        nn_amd.InvalidShape),
        "long_array": (struct.pack("<IIQQ", GW.MAGIC, 3, 0, 1) + GW.gguf_string("a") +
                       struct.pack("<IIQ", GW.ARRAY, GW.U8, 10000001), nn_amd.InvalidShape),
        "bad_value_type": (struct.pack("<IIQQ", GW.MAGIC, 3, 0, 1) + GW.gguf_string("a") + struct.pack("<I", 13),
                           nn_amd.WrongQuantType),
    }
    for name, (blob, exc) in cases.items():
        with pytest.raises(exc):
            open_gguf(tmp_path, blob, name + ".gguf")
    # a tensor past 8 GiB is refused from its declared shape alone
    with pytest.raises(nn_amd.InvalidShape):
        open_gguf(tmp_path, GW.build([], [("big", [1 << 31, 2], 0, b"")])[0], "big.gguf")
    # data-offset alignment: 32 after the infos, whatever their length
    for nm in ["a", "ab" * 7, "x" * 33]:
        blob, base = GW.build([], [(nm, [8], 0, d[:32])])
        g = open_gguf(tmp_path, blob, "al.gguf")
        assert g.data_offset == base and base % 32 == 0
        assert g.tensor_data(nm).tobytes() == d[:32]
        g.close()


def test_gguf_duplicate_names_last_wins(O, tmp_path):
    a, b = np.ones(8, np.float32).tobytes(), np.full(8, 2.0, np.float32).tobytes()
    g = open_gguf(tmp_path, GW.build([], [("w", [8], 0, a), ("w", [8], 0, b)])[0])
    assert len(g.tensor_order) == 2 and g.tensor_data("w").tobytes() == b


@pytest.mark.gpu
def test_gguf_weights_on_device(O, tmp_path):
    """Weights uploaded from the mapped file equal weights built from the same bytes in
    memory (device images byte-identical, outputs bit-identical), and the GEMV over them
    meets the linear bars against the oracle."""
    import torch

    import nn_amd
    from test_gpu_linear import check_close
    nn_amd.init(0)
    dev = torch.device("cuda:0")
    meta, tensors = qwen_like(O)
    g = open_gguf(tmp_path, GW.build(meta, tensors)[0])
    fmt_layout = {12: nn_amd.Layout.GGUF, 14: nn_amd.Layout.NN_GGUF, 8: nn_amd.Layout.GGUF}
    for name, dims, dtype, data in tensors:
        if dtype == 0:
            continue
        n, k = dims
        lay = fmt_layout[dtype]
        wf = g.weight(name, layout=lay)
        wm = nn_amd.QuantizedWeight.from_quantized(np.frombuffer(data, np.uint8), dtype, (n, k), layout=lay)
        assert wf.shape == (n, k) and wf.device_bytes() == wm.device_bytes()
        assert torch.equal(wf.dequantize(), wm.dequantize())
        x = torch.from_numpy(nn_amd.synth_normal(n, 9, (2, k), 1.0)).to(dev)
        y = nn_amd.quantized_linear(x, wf)
        assert torch.equal(y, nn_amd.quantized_linear(x, wm))
        xb = x.cpu().numpy()
        ref = {12: O.q4k_linear, 14: O.q6k_linear, 8: O.q8_0_matmul}[dtype](xb, np.frombuffer(data, np.uint8), n)
        check_close(ref, y.cpu().numpy(), f"gguf {name}")
    # ggml order: dims stored [in, out]
    blob = GW.build([], [("t", [256, 48], 12, tensors[0][3][:48 * 144])])[0]
    g2 = open_gguf(tmp_path, blob, "ggml.gguf")
    w = g2.weight("t", layout=nn_amd.Layout.GGUF, ggml_order=True)
    assert w.shape == (48, 256)
    with pytest.raises(nn_amd.WrongQuantType):
        g.weight("output_norm.weight")
