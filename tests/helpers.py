"""Shared comparison helpers for the parity tests."""
from __future__ import annotations

import numpy as np

from peregrine_amd.synth import bf16_to_f32

# Tolerance stated by the north star for bf16 outputs with fp32 accumulation.
BF16_RTOL = 1e-2


def assert_bf16_close(got_bits, ref_bits, rtol: float = BF16_RTOL, atol_frac: float = 1e-2,
                      min_exact: float | None = None, what: str = "") -> dict:
    """|got - ref| <= rtol*|ref| + atol_frac*rms(ref), elementwise.

    bf16 keeps 8 significant bits, so one output ulp is ~0.4-0.8% relative;
    rtol 1e-2 admits a one-ulp rounding flip caused by a different fp32
    summation order and nothing larger. The absolute floor (1% of the RMS of
    the reference) covers outputs that cancel to near zero.
    """
    g = bf16_to_f32(np.asarray(got_bits)).astype(np.float64)
    r = bf16_to_f32(np.asarray(ref_bits)).astype(np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    rms = float(np.sqrt(np.mean(r * r))) if r.size else 0.0
    err = np.abs(g - r)
    bound = rtol * np.abs(r) + atol_frac * rms
    bad = err > bound
    exact = float(np.mean(np.asarray(got_bits) == np.asarray(ref_bits)))
    stats = {"max_abs": float(err.max(initial=0)), "exact_frac": exact, "rms": rms, "bad": int(bad.sum())}
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; {stats}"
    if min_exact is not None:
        assert exact >= min_exact, f"{what}: bit-exact fraction {exact:.4f} < {min_exact}; {stats}"
    return stats


# ------------------------------------------------------------ checkpoints ---
# A safetensors writer from the published format: u64 little-endian header
# length, a JSON header {name: {dtype, shape, data_offsets}} padded with spaces
# to a multiple of 8, then the tensor bytes. Cross-checked against the
# `safetensors` package in tests/test_checkpoint.py.
def write_safetensors(path, tensors: dict, metadata: dict | None = None) -> None:
    """tensors: {name: (dtype_string, shape, array_or_bytes)}."""
    import json
    import struct

    header, blobs, off = {}, [], 0
    for name, (dtype, shape, data) in tensors.items():
        b = data if isinstance(data, (bytes, bytearray)) else np.ascontiguousarray(data).tobytes()
        header[name] = {"dtype": dtype, "shape": [int(d) for d in shape], "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata is not None:
        header["__metadata__"] = metadata
    hj = json.dumps(header).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def write_checkpoint(directory, tensors: dict, n_shards: int = 2, config: dict | None = None,
                     prefix: str = "model") -> dict:
    """Write tensors over n_shards files plus model.safetensors.index.json (and
    config.json when given). Returns {name: shard file name}."""
    import json
    from pathlib import Path

    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    names = sorted(tensors)
    where, shards = {}, []
    for s in range(n_shards):
        fname = f"{prefix}-{s + 1:05d}-of-{n_shards:05d}.safetensors"
        part = {n: tensors[n] for n in names[s::n_shards]}
        write_safetensors(d / fname, part, metadata={"format": "mlx"})
        where.update({n: fname for n in part})
        shards.append(fname)
    total = sum(len(np.ascontiguousarray(t[2]).tobytes()) if not isinstance(t[2], (bytes, bytearray))
                else len(t[2]) for t in tensors.values())
    (d / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": total}, "weight_map": where}, indent=2))
    if config is not None:
        (d / "config.json").write_text(json.dumps(config, indent=2))
    return where


def qwen35_config(hidden=4096, intermediate=12288, layers=32, vocab=248320, bits=4, group=64, mode="affine",
                  **text_overrides) -> dict:
    """config.json of an MLX Qwen3.5 text checkpoint with the fields
    config.zig:6-31 reads (values of the 9B model unless overridden)."""
    tc = {"model_type": "qwen3_5_text", "hidden_size": hidden, "intermediate_size": intermediate,
          "num_hidden_layers": layers, "num_attention_heads": 16, "num_key_value_heads": 4, "head_dim": 256,
          "full_attention_interval": 4, "linear_num_key_heads": 16, "linear_num_value_heads": 32,
          "linear_key_head_dim": 128, "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
          "vocab_size": vocab, "rms_norm_eps": 1e-6,
          "rope_parameters": {"partial_rotary_factor": 0.25, "rope_theta": 10000000}}
    tc.update(text_overrides)
    return {"model_type": "qwen3_5", "text_config": tc,
            "quantization": {"group_size": group, "bits": bits, "mode": mode}}
