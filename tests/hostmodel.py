"""TEST INFRASTRUCTURE: a seeded Qwen3.5-shaped Q4 model held in host memory.

It exposes the two things oracle.model.OracleModel reads from a model (`cfg`
and `read(name, dtype)`), so the oracle's composition can run on the CPU
without a GPU, and it lists its tensors in checkpoint form (`tensors()`), so a
GPU test can write it as an MLX safetensors checkpoint and upload it with
prg_model_load. The same weights then reach the oracle, the HIP model and the
transformers float reference written by tests/golden/make_hf_golden.py.

Tensor names, dtypes and shapes are those of the reference's upload code
(src/model/decoder_layer.zig:376-412, block_linear.zig:155-173,
block_attn.zig:235-248, block_mlp.zig:116-122, mtp.zig:86-116). The value
distributions follow the random-init model of the HIP library: Q4 scales
U(0.002, 0.02) and biases -7.5*s + N(0, 0.01) (zero-mean dequantised weights),
norm weights N(1, 0.1), conv taps N(0, 0.5), A_log and dt_bias N(0, 0.5).
"""
from __future__ import annotations

import hashlib

import numpy as np

from peregrine_amd.model import ModelConfig
from peregrine_amd.synth import bf16_to_f32, f32_to_bf16

ROOT = "language_model.model"


def tensor_specs(cfg: ModelConfig) -> list[tuple[str, str, tuple[int, ...]]]:
    """(name, checkpoint dtype, checkpoint shape) in upload order."""
    out = []

    def q4(base, n, k):
        out.extend([(base + ".weight", "U32", (n, k // 8)), (base + ".scales", "BF16", (n, k // 64)),
                    (base + ".biases", "BF16", (n, k // 64))])

    def norms(p):
        out.extend([(p + ".input_layernorm.weight", "BF16", (cfg.hidden,)),
                    (p + ".post_attention_layernorm.weight", "BF16", (cfg.hidden,))])

    def full(p):
        a = p + ".self_attn"
        q4(a + ".q_proj", 2 * 16 * 256, cfg.hidden)
        q4(a + ".k_proj", 4 * 256, cfg.hidden)
        q4(a + ".v_proj", 4 * 256, cfg.hidden)
        q4(a + ".o_proj", cfg.hidden, 16 * 256)
        out.extend([(a + ".q_norm.weight", "BF16", (256,)), (a + ".k_norm.weight", "BF16", (256,))])

    def mlp(p):
        q4(p + ".mlp.gate_proj", cfg.intermediate, cfg.hidden)
        q4(p + ".mlp.up_proj", cfg.intermediate, cfg.hidden)
        q4(p + ".mlp.down_proj", cfg.hidden, cfg.intermediate)

    q4(ROOT + ".embed_tokens", cfg.vocab, cfg.hidden)
    for i in range(cfg.num_layers):
        p = f"{ROOT}.layers.{i}"
        norms(p)
        if cfg.is_linear(i):
            a = p + ".linear_attn"
            q4(a + ".in_proj_qkv", 8192, cfg.hidden)
            q4(a + ".in_proj_z", 4096, cfg.hidden)
            q4(a + ".in_proj_a", 32, cfg.hidden)
            q4(a + ".in_proj_b", 32, cfg.hidden)
            q4(a + ".out_proj", cfg.hidden, 4096)
            out.extend([(a + ".conv1d.weight", "BF16", (8192, 4, 1)), (a + ".A_log", "F32", (32,)),
                        (a + ".dt_bias", "BF16", (32,)), (a + ".norm.weight", "BF16", (128,))])
        else:
            full(p)
        mlp(p)
    out.append((ROOT + ".norm.weight", "BF16", (cfg.hidden,)))
    q4("language_model.lm_head", cfg.vocab, cfg.hidden)
    if cfg.mtp_layers:
        out.extend([("mtp.pre_fc_norm_embedding.weight", "BF16", (cfg.hidden,)),
                    ("mtp.pre_fc_norm_hidden.weight", "BF16", (cfg.hidden,))])
        q4("mtp.fc", cfg.hidden, 2 * cfg.hidden)
        norms("mtp.layers.0")
        full("mtp.layers.0")
        mlp("mtp.layers.0")
        out.append(("mtp.norm.weight", "BF16", (cfg.hidden,)))
    return out


class HostModel:
    """Seeded random weights in host memory, addressed by checkpoint name."""

    def __init__(self, cfg: ModelConfig, seed: int = 0) -> None:
        self.cfg = cfg
        rng = np.random.default_rng(seed)
        self.data: dict[str, tuple[str, tuple[int, ...], np.ndarray]] = {}
        last_scales = None
        for name, dtype, shape in tensor_specs(cfg):
            n = int(np.prod(shape))
            if dtype == "U32":
                a = np.frombuffer(rng.bytes(4 * n), np.uint32).copy()
            elif name.endswith(".scales"):
                a = f32_to_bf16(rng.uniform(0.002, 0.02, n).astype(np.float32))
                last_scales = a
            elif name.endswith(".biases"):
                b = -7.5 * bf16_to_f32(last_scales) + rng.normal(0.0, 0.01, n).astype(np.float32)
                a = f32_to_bf16(b.astype(np.float32))
            elif name.endswith("A_log"):
                a = rng.normal(0.0, 0.5, n).astype(np.float32)
            elif name.endswith("conv1d.weight") or name.endswith("dt_bias"):
                a = f32_to_bf16(rng.normal(0.0, 0.5, n).astype(np.float32))
            else:  # RMSNorm / gated-norm weights
                a = f32_to_bf16(rng.normal(1.0, 0.1, n).astype(np.float32))
            self.data[name] = (dtype, shape, a)

    def read(self, name: str, dtype) -> np.ndarray:
        return self.data[name][2].view(dtype).ravel().copy()

    def tensors(self) -> dict:
        """{name: (dtype, shape, array)} for helpers.write_checkpoint."""
        return {n: (d, s, a.reshape(s)) for n, (d, s, a) in self.data.items()}

    def digest(self) -> str:
        """sha256 over every tensor's name and bytes, in upload order: pins the
        generator, so a fixture made from these weights is only ever compared
        with the same weights."""
        h = hashlib.sha256()
        for name, (_, _, a) in self.data.items():
            h.update(name.encode())
            h.update(np.ascontiguousarray(a).tobytes())
        return h.hexdigest()
