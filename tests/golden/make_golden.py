"""Generate the committed golden fixtures of the quantized-linear path.

The fixtures are produced by the CPU oracle (oracle/nnq_oracle.c, the restatement of
the reference's decoders, fused Q8_0 matmul, QLinear::forward and the GPT-OSS MXFP4
MoE layer) on small seeded inputs, and stored as .npz data (inputs + expected outputs):

  decode_blocks.npz  block bytes of every format / layout (random bytes with finite f16
                     scales, plus encoder output) and their decoded f32 bit patterns
  linear_small.npz   tiny y = x W^T cases per format (f32 x, m = 1, 3, 16)
  moe_small.npz      an MXFP4 MoE layer (E = 4, top-2, hidden = intermediate = 64,
                     12 tokens): inputs, top-k experts / weights and the output

The reference itself is Rust with no toolchain in this image, so it cannot produce the
vectors; the oracle is pinned to the reference's own known-answer tests, invariants
and closed forms in tests/test_oracle.py.  Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def rand_blocks(fmt, nblocks, rng):
    """Random block bytes with finite f16 scales (every other bit random)."""
    if fmt == "q8_0":
        b = rng.integers(0, 256, (nblocks, 34), dtype=np.uint8)
        b[:, 0:2] = (b[:, 0:2].copy().view(np.uint16) & 0x7BFF).view(np.uint8)
    elif fmt == "q4_k":
        b = rng.integers(0, 256, (nblocks, 144), dtype=np.uint8)
        b[:, 0:4] = (b[:, 0:4].copy().view(np.uint16) & 0x7BFF).view(np.uint8)
    else:  # q6_k (nn-gguf layout, f16 d at byte 208)
        b = rng.integers(0, 256, (nblocks, 210), dtype=np.uint8)
        b[:, 208:210] = (b[:, 208:210].copy().view(np.uint16) & 0x7BFF).view(np.uint8)
    return b.ravel()


def decode_blocks(rng):
    out = {}
    w = (rng.standard_normal(8 * 256) * 0.02).astype(np.float32)
    for name, fmt, dec, per in [("q8_0", "q8_0", O.dequant_q8_0, 32), ("q4_k", "q4_k", O.dequant_q4_k, 256),
                                ("q4_k_legacy", "q4_k", O.dequant_q4_k_legacy, 256),
                                ("q6_k", "q6_k", O.dequant_q6_k, 256)]:
        b = rand_blocks(fmt, 8, rng)
        out[f"{name}_random_bytes"] = b
        out[f"{name}_random_f32bits"] = dec(b, 8 * per).view(np.uint32)
        enc = {"q8_0": O.quantize_q8_0, "q4_k": O.quantize_q4_k, "q6_k": O.quantize_q6_k}[fmt](w[:8 * per])
        out[f"{name}_encoded_bytes"] = enc
        out[f"{name}_encoded_f32bits"] = dec(enc, 8 * per).view(np.uint32)
    # MXFP4 (GPT-OSS Mxfp4Tensor): random codes, scales across the E8M0 range incl. 0 and 255
    packed = rng.integers(0, 256, 16 * 16, dtype=np.uint8)
    scales = np.array([0, 1, 2, 100, 120, 125, 126, 127, 128, 129, 140, 200, 253, 254, 127, 130], np.uint8)
    out["mxfp4_packed"] = packed
    out["mxfp4_scales"] = scales
    out["mxfp4_f32bits"] = O.mxfp4_dequantize(packed, scales, 16 * 32).view(np.uint32)
    return out


def linear_small(rng):
    out = {}
    for name, fmt, k in [("q8_0", "q8_0", 320), ("q4_k", "q4_k", 512), ("q4_k_legacy", "q4_k", 512),
                         ("q6_k", "q6_k", 512)]:
        n = 48
        w = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
        b = {"q8_0": O.quantize_q8_0, "q4_k": O.quantize_q4_k, "q6_k": O.quantize_q6_k}[fmt](w)
        if name == "q4_k_legacy":  # the legacy layout decodes random bytes (its own packing)
            b = rand_blocks("q4_k", n * k // 256, rng)
        out[f"{name}_bytes"] = b
        out[f"{name}_shape"] = np.array([n, k], np.int64)
        for m in (1, 3, 16):
            x = rng.standard_normal((m, k)).astype(np.float32)
            if fmt == "q8_0":
                y = O.q8_0_matmul(x, b, n)
            else:
                dec = {"q4_k": O.dequant_q4_k, "q4_k_legacy": O.dequant_q4_k_legacy, "q6_k": O.dequant_q6_k}[name]
                y = O.matmul_xwt(x, dec(b, n * k).reshape(n, k))
            out[f"{name}_x_m{m}"] = x
            out[f"{name}_y_m{m}"] = y
    return out


def moe_small(rng):
    E, K, T, H, I = 4, 2, 12, 64, 64
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    gu = (rng.standard_normal(E * H * 2 * I) * 0.1).astype(np.float32)
    dn = (rng.standard_normal(E * I * H) * 0.1).astype(np.float32)
    gb = (rng.standard_normal(E * 2 * I) * 0.1).astype(np.float32)
    db = (rng.standard_normal(E * H) * 0.1).astype(np.float32)
    gp, gs = O.mxfp4_quantize(gu)
    dp, ds = O.mxfp4_quantize(dn)
    y, ti, tw = O.moe_forward(x, logits, K, gp, gs, gb, dp, ds, db, I, 7.0)
    return dict(dims=np.array([E, K, T, H, I], np.int64), x=x, logits=logits, gu_packed=gp, gu_scales=gs,
                gu_bias=gb, dn_packed=dp, dn_scales=ds, dn_bias=db, y=y, topk_idx=ti, topk_w=tw, limit=np.float32(7.0))


def main():
    O.build()
    rng = np.random.default_rng(20261201)
    np.savez_compressed(os.path.join(HERE, "decode_blocks.npz"), **decode_blocks(rng))
    np.savez_compressed(os.path.join(HERE, "linear_small.npz"), **linear_small(rng))
    np.savez_compressed(os.path.join(HERE, "moe_small.npz"), **moe_small(rng))
    for f in ("decode_blocks.npz", "linear_small.npz", "moe_small.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
