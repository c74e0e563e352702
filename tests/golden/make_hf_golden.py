"""Write tests/golden/hf_v1.npz: float reference logits for the model
composition, from Hugging Face transformers' Qwen3.5 text model.

CPU only, run in the build container (transformers is not needed anywhere
else; no GPU test imports this script):

    python tests/golden/make_hf_golden.py

transformers 5.15 implements the same architecture as the reference's Zig
host code (src/model/decoder_layer.zig:461-566,644-819,
block_linear.zig:199-469, block_attn.zig:261-631, block_mlp.zig:155-311,
model.zig:686-717) independently: its own GatedDeltaNet (chunked delta rule
for a prompt, recurrent rule per token), causal conv1d, gated attention
with partial NeoX RoPE, SwiGLU MLP and RMSNorms. The weights are the seeded
host model of tests/hostmodel.py, dequantised exactly (s*q + b in float64),
loaded into a float64 model. Differences from the reference's conventions,
bridged here and nowhere else:

- Qwen3_5RMSNorm scales by (1 + w); the reference multiplies by the stored
  w (rmsnorm.metal:80-116), so those modules get w - 1 (exact in float64).
  Qwen3_5RMSNormGated multiplies by w, as the reference's gated norm does.
- conv1d weight [C, 4] becomes the torch Conv1d weight [C, 1, 4] (tap 0 is
  the oldest input in both).

The MTP drafter (src/model/mtp.zig:188-280) has no transformers module; it is
assembled from transformers parts: Qwen3_5RMSNorm for the two pre-fc norms and
the final norm, a bias-free Linear for fc over [norm(embed) | norm(hidden)],
one full-attention Qwen3_5DecoderLayer with its own causal attention over the
drafter positions, and the shared lm_head. Drafter slot j reads the token at
position j + 1 and the target's final-normed hidden row j
(src/server/decode_loop.zig:181-196).

Stored: the prompt, float32 target logits per position (one causal forward
pass; the script asserts that token-by-token decoding with transformers'
cache gives the same logits), the float32 final-normed hidden rows, float32
drafter logits per slot, and the host model's weight digest.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (str(ROOT), str(HERE.parent)):
    if p not in sys.path:
        sys.path.insert(0, p)

from hostmodel import HostModel  # noqa: E402
from peregrine_amd.model import ModelConfig  # noqa: E402
from peregrine_amd.synth import Q4Weight, bf16_to_f32  # noqa: E402

CFG = ModelConfig(num_layers=4, hidden=1024, intermediate=2048, vocab=4096, mtp_layers=1)
SEED = 21
PROMPT_SEED = 22
PROMPT_LEN = 24
OUT = HERE / "hf_v1.npz"


def hf_config(cfg: ModelConfig, num_layers: int | None = None, layer_types=None):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    n = cfg.num_layers if num_layers is None else num_layers
    kw = dict(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
              num_hidden_layers=n, num_attention_heads=16, num_key_value_heads=4, head_dim=256,
              rms_norm_eps=cfg.rms_eps, hidden_act="silu", tie_word_embeddings=False,
              linear_conv_kernel_dim=4, linear_key_head_dim=128, linear_value_head_dim=128,
              linear_num_key_heads=16, linear_num_value_heads=32, max_position_embeddings=4096,
              rope_parameters={"rope_type": "default", "rope_theta": 1e7, "partial_rotary_factor": 0.25})
    if layer_types is not None:
        kw["layer_types"] = layer_types
    c = Qwen3_5TextConfig(**kw)
    c._attn_implementation = "eager"
    return c


class Loader:
    def __init__(self, hm: HostModel) -> None:
        self.hm = hm

    def dense(self, base: str, n: int, k: int):
        import torch

        q = Q4Weight(self.hm.read(base + ".weight", np.uint32).reshape(n, k // 8),
                     self.hm.read(base + ".scales", np.uint16).reshape(n, k // 64),
                     self.hm.read(base + ".biases", np.uint16).reshape(n, k // 64))
        return torch.from_numpy(q.dequant_f64())

    def vec(self, name: str, shift: float = 0.0):
        import torch

        dt = self.hm.data[name][0]
        a = self.hm.read(name, np.float32 if dt == "F32" else np.uint16)
        v = a.astype(np.float64) if dt == "F32" else bf16_to_f32(a).astype(np.float64)
        return torch.from_numpy(v + shift)

    def set_(self, param, value) -> None:
        assert tuple(param.shape) == tuple(value.shape), (param.shape, value.shape)
        with __import__("torch").no_grad():
            param.copy_(value)

    def decoder_layer(self, layer, p: str, linear: bool) -> None:
        c, H = CFG, CFG.hidden
        self.set_(layer.input_layernorm.weight, self.vec(p + ".input_layernorm.weight", -1.0))
        self.set_(layer.post_attention_layernorm.weight, self.vec(p + ".post_attention_layernorm.weight", -1.0))
        if linear:
            la, a = layer.linear_attn, p + ".linear_attn"
            self.set_(la.in_proj_qkv.weight, self.dense(a + ".in_proj_qkv", 8192, H))
            self.set_(la.in_proj_z.weight, self.dense(a + ".in_proj_z", 4096, H))
            self.set_(la.in_proj_a.weight, self.dense(a + ".in_proj_a", 32, H))
            self.set_(la.in_proj_b.weight, self.dense(a + ".in_proj_b", 32, H))
            self.set_(la.out_proj.weight, self.dense(a + ".out_proj", H, 4096))
            self.set_(la.conv1d.weight, self.vec(a + ".conv1d.weight").reshape(8192, 1, 4))
            self.set_(la.A_log, self.vec(a + ".A_log"))
            self.set_(la.dt_bias, self.vec(a + ".dt_bias"))
            self.set_(la.norm.weight, self.vec(a + ".norm.weight"))  # gated norm: plain w
        else:
            sa, a = layer.self_attn, p + ".self_attn"
            self.set_(sa.q_proj.weight, self.dense(a + ".q_proj", 8192, H))
            self.set_(sa.k_proj.weight, self.dense(a + ".k_proj", 1024, H))
            self.set_(sa.v_proj.weight, self.dense(a + ".v_proj", 1024, H))
            self.set_(sa.o_proj.weight, self.dense(a + ".o_proj", H, 4096))
            self.set_(sa.q_norm.weight, self.vec(a + ".q_norm.weight", -1.0))
            self.set_(sa.k_norm.weight, self.vec(a + ".k_norm.weight", -1.0))
        self.set_(layer.mlp.gate_proj.weight, self.dense(p + ".mlp.gate_proj", c.intermediate, H))
        self.set_(layer.mlp.up_proj.weight, self.dense(p + ".mlp.up_proj", c.intermediate, H))
        self.set_(layer.mlp.down_proj.weight, self.dense(p + ".mlp.down_proj", H, c.intermediate))


def main() -> None:
    import torch
    from transformers.models.qwen3_5.modeling_qwen3_5 import (Qwen3_5DecoderLayer, Qwen3_5ForCausalLM,
                                                              Qwen3_5RMSNorm, Qwen3_5TextRotaryEmbedding)

    torch.manual_seed(0)
    hm = HostModel(CFG, SEED)
    ld = Loader(hm)
    root = "language_model.model"
    model = Qwen3_5ForCausalLM(hf_config(CFG)).to(torch.float64).eval()
    tm = model.model
    ld.set_(tm.embed_tokens.weight, ld.dense(root + ".embed_tokens", CFG.vocab, CFG.hidden))
    for i, layer in enumerate(tm.layers):
        assert (layer.layer_type if hasattr(layer, "layer_type") else layer.block_type) == (
            "linear_attention" if CFG.is_linear(i) else "full_attention")
        ld.decoder_layer(layer, f"{root}.layers.{i}", CFG.is_linear(i))
    ld.set_(tm.norm.weight, ld.vec(root + ".norm.weight", -1.0))
    ld.set_(model.lm_head.weight, ld.dense("language_model.lm_head", CFG.vocab, CFG.hidden))

    prompt = np.random.default_rng(PROMPT_SEED).integers(0, CFG.vocab, size=PROMPT_LEN).astype(np.int64)
    ids = torch.from_numpy(prompt)[None]
    with torch.no_grad():
        out = tm(input_ids=ids, use_cache=False)
        hidden = out.last_hidden_state[0]                       # final-normed rows
        logits = model.lm_head(hidden)
        # transformers' per-token route (recurrent delta rule, conv update,
        # KV cache) must agree with its one-pass route
        step_logits = []
        past = None
        for t in range(PROMPT_LEN):
            o = model(input_ids=ids[:, t:t + 1], past_key_values=past, use_cache=True)
            past = o.past_key_values
            step_logits.append(o.logits[0, -1])
        step_logits = torch.stack(step_logits)
    d = float((step_logits - logits).abs().max() / logits.abs().max())
    print(f"transformers one-pass vs per-token logits: max rel diff {d:.2e}")
    assert d < 1e-5, d

    # MTP drafter from transformers parts (mtp.zig:188-280)
    H = CFG.hidden
    dcfg = hf_config(CFG, num_layers=1, layer_types=["full_attention"])
    layer = Qwen3_5DecoderLayer(dcfg, 0).to(torch.float64).eval()
    ld.decoder_layer(layer, "mtp.layers.0", linear=False)
    norm_e, norm_h, norm_f = (Qwen3_5RMSNorm(H, eps=CFG.rms_eps).to(torch.float64) for _ in range(3))
    ld.set_(norm_e.weight, ld.vec("mtp.pre_fc_norm_embedding.weight", -1.0))
    ld.set_(norm_h.weight, ld.vec("mtp.pre_fc_norm_hidden.weight", -1.0))
    ld.set_(norm_f.weight, ld.vec("mtp.norm.weight", -1.0))
    fc = ld.dense("mtp.fc", H, 2 * H)
    rope = Qwen3_5TextRotaryEmbedding(dcfg)
    S = PROMPT_LEN - 1
    with torch.no_grad():
        emb = tm.embed_tokens(ids[0, 1:])                      # token at position j + 1
        fused = torch.cat([norm_e(emb), norm_h(hidden[:S])], dim=-1) @ fc.T
        pos = torch.arange(S)[None]
        cos, sin = rope(fused[None], pos)
        mask = torch.full((S, S), float("-inf"), dtype=torch.float64).triu(1)[None, None]
        h = layer(fused[None], position_embeddings=(cos, sin), attention_mask=mask, position_ids=pos)
        h = h[0] if isinstance(h, tuple) else h
        draft_logits = model.lm_head(norm_f(h[0]))

    np.savez_compressed(
        OUT, prompt=prompt.astype(np.uint32), logits=logits.numpy().astype(np.float32),
        hidden=hidden.numpy().astype(np.float32), draft_logits=draft_logits.numpy().astype(np.float32),
        digest=np.array(hm.digest()), seed=np.array(SEED),
        config=np.array([CFG.num_layers, CFG.hidden, CFG.intermediate, CFG.vocab, CFG.mtp_layers]),
        transformers_version=np.array(__import__("transformers").__version__))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
