"""TEST INFRASTRUCTURE: CPU restatement of the reference's decode and prompt
(prefill) compositions.

Orchestrates the C oracle primitives exactly as the reference's Zig host code
dispatches its kernels, without any of the GPU build's fusions. One token:
  DecoderLayer.decodeStepBf16          src/model/decoder_layer.zig:461-566, 756-781
  LinearAttentionBlock.decodeStepBf16  src/model/block_linear.zig:199-263
  FullAttentionBlock.decodeStepBf16    src/model/block_attn.zig:261-359
  MlpBlock.decodeResidualBf16          src/model/block_mlp.zig:260-277
  encodeStackBf16 + argmax tail        src/model/model.zig:686-717, 1346-1388
  decodeFromPrefixCache (no prefix)    src/server/decode_loop.zig:96-160
A prompt of T tokens at once (layer-major, one chunk):
  DecoderLayer.prefillStepBf16         src/model/decoder_layer.zig:644-760
  LinearAttentionBlock prefill         src/model/block_linear.zig:265-469
  FullAttentionBlock prefill           src/model/block_attn.zig:361-631
  MlpBlock prefill (gate/up, down)     src/model/block_mlp.zig:155-258
  encodePrefillArgmaxTailBf16          src/model/model.zig:1307-1324
Weights are read back from the GPU model (same bits on both sides).
"""
from __future__ import annotations

import numpy as np

from peregrine_amd.synth import Q4Weight, bf16_to_f32

from .binding import oracle

ROOT = "language_model.model"


def decisive_margin(logits) -> tuple[int, int, float, float]:
    """(top-1 index, runner-up index, top-1 minus top-2 logit, guard) of one
    step's bf16 logits. The guard is four bf16 ulps of the top logit: bf16
    keeps 8 significant bits, and every projection output on both sides is
    rounded to bf16, so one-ulp rounding flips from a different fp32
    summation order propagate through the residual stream. A step is
    decisive when the margin exceeds the guard; below it, a different winner
    is a legitimate tie-break."""
    lg = np.asarray(logits, np.float64)
    i1 = int(np.argmax(lg))
    rest = lg.copy()
    rest[i1] = -np.inf
    i2 = int(np.argmax(rest))
    top1, top2 = float(lg[i1]), float(lg[i2])
    ulp = 2.0 ** (np.floor(np.log2(max(abs(top1), 1e-30))) - 7)
    return i1, i2, top1 - top2, 4.0 * ulp


def _q4(model, base: str, out_dim: int, in_dim: int) -> Q4Weight:
    w = model.read(base + ".weight", np.uint32).reshape(out_dim, in_dim // 8)
    s = model.read(base + ".scales", np.uint16).reshape(out_dim, in_dim // 64)
    b = model.read(base + ".biases", np.uint16).reshape(out_dim, in_dim // 64)
    return Q4Weight(w, s, b)


class OracleModel:
    def __init__(self, model, max_seq: int) -> None:
        """model: peregrine_amd.model.DeviceModel (weights are copied to host)."""
        c = model.cfg
        self.cfg = c
        self.o = oracle()
        self.embed = _q4(model, ROOT + ".embed_tokens", c.vocab, c.hidden)
        self.layers = []
        for i in range(c.num_layers):
            p = f"{ROOT}.layers.{i}"
            L = {"linear": c.is_linear(i),
                 "input_norm": model.read(p + ".input_layernorm.weight", np.uint16),
                 "post_norm": model.read(p + ".post_attention_layernorm.weight", np.uint16),
                 "gate": _q4(model, p + ".mlp.gate_proj", c.intermediate, c.hidden),
                 "up": _q4(model, p + ".mlp.up_proj", c.intermediate, c.hidden),
                 "down": _q4(model, p + ".mlp.down_proj", c.hidden, c.intermediate)}
            if L["linear"]:
                a = p + ".linear_attn"
                L.update(qkv=_q4(model, a + ".in_proj_qkv", 8192, c.hidden),
                         z=_q4(model, a + ".in_proj_z", 4096, c.hidden),
                         a=_q4(model, a + ".in_proj_a", 32, c.hidden),
                         b=_q4(model, a + ".in_proj_b", 32, c.hidden),
                         out=_q4(model, a + ".out_proj", c.hidden, 4096),
                         conv_w=model.read(a + ".conv1d.weight", np.uint16).reshape(8192, 4),
                         A_log=model.read(a + ".A_log", np.float32),
                         dt_bias=model.read(a + ".dt_bias", np.uint16),
                         norm_w=model.read(a + ".norm.weight", np.uint16))
            else:
                a = p + ".self_attn"
                L.update(q=_q4(model, a + ".q_proj", 8192, c.hidden),
                         k=_q4(model, a + ".k_proj", 1024, c.hidden),
                         v=_q4(model, a + ".v_proj", 1024, c.hidden),
                         o=_q4(model, a + ".o_proj", c.hidden, 4096),
                         q_norm=model.read(a + ".q_norm.weight", np.uint16),
                         k_norm=model.read(a + ".k_norm.weight", np.uint16))
            self.layers.append(L)
        self.final_norm = model.read(ROOT + ".norm.weight", np.uint16)
        self.lm_head = _q4(model, "language_model.lm_head", c.vocab, c.hidden)
        self.mtp = None
        if getattr(c, "mtp_layers", 0):                              # mtp.zig:86-116
            p = "mtp.layers.0"
            a = p + ".self_attn"
            self.mtp = {"linear": False,
                        "pre_e": model.read("mtp.pre_fc_norm_embedding.weight", np.uint16),
                        "pre_h": model.read("mtp.pre_fc_norm_hidden.weight", np.uint16),
                        "fc": _q4(model, "mtp.fc", c.hidden, 2 * c.hidden),
                        "norm": model.read("mtp.norm.weight", np.uint16),
                        "input_norm": model.read(p + ".input_layernorm.weight", np.uint16),
                        "post_norm": model.read(p + ".post_attention_layernorm.weight", np.uint16),
                        "gate": _q4(model, p + ".mlp.gate_proj", c.intermediate, c.hidden),
                        "up": _q4(model, p + ".mlp.up_proj", c.intermediate, c.hidden),
                        "down": _q4(model, p + ".mlp.down_proj", c.hidden, c.intermediate),
                        "q": _q4(model, a + ".q_proj", 8192, c.hidden),
                        "k": _q4(model, a + ".k_proj", 1024, c.hidden),
                        "v": _q4(model, a + ".v_proj", 1024, c.hidden),
                        "o": _q4(model, a + ".o_proj", c.hidden, 4096),
                        "q_norm": model.read(a + ".q_norm.weight", np.uint16),
                        "k_norm": model.read(a + ".k_norm.weight", np.uint16)}
        a = 64 if max_seq >= 16000 else 256
        self.stride = (max_seq + a - 1) // a * a  # state.zig:25-32
        self.reset()

    def reset(self) -> None:  # state.zig:52-90 (zeroed), resetForNewSequence
        self.state = []
        for L in self.layers:
            if L["linear"]:
                self.state.append({"conv": np.zeros((3, 8192), np.float32),
                                   "recur": np.zeros((32, 128, 128), np.float32)})
            else:
                self.state.append({"k": np.zeros((4, self.stride, 256), np.uint16),
                                   "v": np.zeros((4, 256, self.stride), np.uint16)})
        self.mtp_state = {"k": np.zeros((4, self.stride, 256), np.uint16),
                          "v": np.zeros((4, 256, self.stride), np.uint16)}

    def load_state(self, snap: dict) -> None:
        """Take over a device state: host copies of its GDN conv / recurrent
        states and KV caches keyed "layers.<i>.conv|recur|cache_k|cache_v"
        (f32 for the GDN states, bf16 bits for the caches), with the same
        cache stride."""
        assert snap["stride"] == self.stride, (snap["stride"], self.stride)
        for i, L in enumerate(self.layers):
            if L["linear"]:
                self.state[i]["conv"] = np.asarray(snap[f"layers.{i}.conv"], np.float32).reshape(3, 8192).copy()
                self.state[i]["recur"] = np.asarray(snap[f"layers.{i}.recur"], np.float32).reshape(32, 128, 128).copy()
            else:
                self.state[i]["k"] = np.asarray(snap[f"layers.{i}.cache_k"], np.uint16).reshape(4, self.stride, 256).copy()
                self.state[i]["v"] = np.asarray(snap[f"layers.{i}.cache_v"], np.uint16).reshape(4, 256, self.stride).copy()

    def _layer(self, i: int, h: np.ndarray, pos: int) -> np.ndarray:
        return self._decode_layer(self.layers[i], self.state[i], h, pos)

    def _decode_layer(self, L, S, h: np.ndarray, pos: int) -> np.ndarray:
        o, eps = self.o, self.cfg.rms_eps
        normed = o.rmsnorm(h, L["input_norm"], eps)[0]            # decoder_layer.zig:531
        if L["linear"]:                                            # block_linear.zig:222-262
            qkv = o.q4_gemv(normed, L["qkv"])[0]
            z = o.q4_gemv(normed, L["z"])[0]
            a = o.q4_gemv(normed, L["a"])[0]
            b = o.q4_gemv(normed, L["b"])[0]
            conv_out, S["conv"] = o.conv1d_decode(S["conv"], qkv, L["conv_w"])
            y, S["recur"] = o.gated_delta_decode(S["recur"], conv_out, a, b, L["A_log"], L["dt_bias"],
                                                 has_prev=pos != 0)  # decoder_layer.zig:564
            gated = o.rmsnorm_gated(y, L["norm_w"], z, 128, eps)
            attn = o.q4_gemv(gated, L["out"])[0]
        else:                                                      # block_attn.zig:312-358
            qp = o.q4_gemv(normed, L["q"])[0]
            k = o.q4_gemv(normed, L["k"])[0]
            v = o.q4_gemv(normed, L["v"])[0]
            q, gate, S["k"], S["v"] = o.attn_prepare(qp, L["q_norm"], k, v, L["k_norm"], S["k"], S["v"],
                                                     self.stride, dst=pos, pos=pos)
            ctx = o.attn_decode(q, S["k"], S["v"], gate, self.stride, pos + 1)
            attn = o.q4_gemv(ctx, L["o"])[0]
        r, normed2 = o.add_rmsnorm(h, attn, L["post_norm"], eps)   # decoder_layer.zig:772
        inter = o.q4_gemv_silu_gate(normed2, L["gate"], L["up"])   # block_mlp.zig:272
        return o.q4_gemv_residual_add(inter, L["down"], r)[0]      # block_mlp.zig:276

    def step(self, token: int, pos: int, want_logits: bool = False, want_hidden: bool = False):
        """One decode step at position pos; returns (next_token, logits|None)
        (and the final-normed hidden when want_hidden)."""
        o = self.o
        h = o.embedding(self.embed, token)                          # model.zig:700
        for i in range(len(self.layers)):
            h = self._layer(i, h, pos)
        normed = o.rmsnorm(h, self.final_norm, self.cfg.rms_eps)[0]  # model.zig:1355
        tok, logits = self._head(normed, want_logits)
        return (tok, logits, normed) if want_hidden else (tok, logits)

    def verify2(self, t0: int, t1: int, pos: int, want_logits: bool = False):
        """forwardTwoTokenDecodeVerifierBf16 (model.zig:1627-1659): rows t0 at
        pos and t1 at pos + 1 through encodeStack2Bf16 / decodeStep2Bf16
        (model.zig:719-760, decoder_layer.zig:485-516). The reference runs
        the attention-side projections once per row and the M = 2 GEMVs
        (linear_decode.metal:76-159, 233-309, 484-580) with per-row
        arithmetic identical to M = 1, so each row is one decode step.
        Returns (verify, bonus, logits0|None, logits1|None, hidden rows)."""
        v, lg0, h0 = self.step(t0, pos, want_logits, want_hidden=True)
        b, lg1, h1 = self.step(t1, pos + 1, want_logits, want_hidden=True)
        return v, b, lg0, lg1, np.stack([h0, h1])

    def _head(self, normed, want_logits: bool):
        o = self.o
        pv, pi = o.q4_argmax_partial(normed, self.lm_head)          # model.zig:1386
        tok = o.argmax_pairs(pv[0], pi[0])                          # model.zig:1387
        logits = bf16_to_f32(o.q4_gemv(normed, self.lm_head)[0]) if want_logits else None
        return tok, logits

    # ------------------------------------------------------- MTP drafter ---
    def _pre_fc(self, tokens, hidden_rows):                       # mtp.zig:244-280
        o, t, eps = self.o, self.mtp, self.cfg.rms_eps
        e = o.embedding_many(self.embed, np.atleast_1d(np.asarray(tokens, np.uint32)))
        ne = o.rmsnorm(e, t["pre_e"], eps)
        nh = o.rmsnorm(np.atleast_2d(hidden_rows), t["pre_h"], eps)
        return np.ascontiguousarray(np.concatenate([ne, nh], axis=1))

    def mtp_step(self, token: int, hidden, pos: int, want_logits: bool = False):
        """Drafter.forwardDraftTokenProfiled (mtp.zig:187-242) at drafter slot pos."""
        o, t = self.o, self.mtp
        fused = o.q4_gemv(self._pre_fc([token], hidden)[0], t["fc"])[0]
        out = self._decode_layer(t, self.mtp_state, fused, pos)
        normed = o.rmsnorm(out, t["norm"], self.cfg.rms_eps)[0]
        return self._head(normed, want_logits)

    def mtp_prefill(self, tokens, hidden_rows, start: int) -> None:
        """Drafter.forwardPrefill (mtp.zig:137-185)."""
        fused = self.o.q4_qmm(self._pre_fc(tokens, hidden_rows), self.mtp["fc"])
        self._prefill_layer_impl(self.mtp, self.mtp_state, fused, start)

    def _prefill_layer(self, i: int, h: np.ndarray, start: int) -> np.ndarray:
        return self._prefill_layer_impl(self.layers[i], self.state[i], h, start)

    def _prefill_layer_impl(self, L, S, h: np.ndarray, start: int) -> np.ndarray:
        o, eps = self.o, self.cfg.rms_eps
        T = h.shape[0]
        normed = o.rmsnorm(h, L["input_norm"], eps)                # decoder_layer.zig:666
        if L["linear"]:                                            # block_linear.zig:265-361
            qkv = o.q4_qmm(normed, L["qkv"])
            z = o.q4_qmm(normed, L["z"])
            a = o.q4_qmm(normed, L["a"])
            b = o.q4_qmm(normed, L["b"])
            has_prev = start != 0                                  # decoder_layer.zig:635
            conv_out, S["conv"] = o.conv1d_prefill(S["conv"], qkv, L["conv_w"], has_prev)
            qn, kn = o.qk_l2norm_prefill(conv_out)
            g, beta = o.gating_many(L["A_log"], a, L["dt_bias"], b)
            y, S["recur"] = o.gated_delta_prefill(S["recur"], qn, kn, conv_out, g, beta, has_prev)
            gated = o.rmsnorm_gated(y, L["norm_w"], z, 128, eps)
            attn = o.q4_qmm(gated.reshape(T, 4096), L["out"])
        else:                                                      # block_attn.zig:361-498
            qp = o.q4_qmm(normed, L["q"])
            k = o.q4_qmm(normed, L["k"])
            v = o.q4_qmm(normed, L["v"])
            q, gate = o.split_qg_many(qp)
            q, S["k"], S["v"] = o.qk_norm_rope_append_many(q, L["q_norm"], k, L["k_norm"], v, S["k"], S["v"],
                                                           start, start, self.stride)
            ctx = o.attn_prefill(q, S["k"], S["v"], T, start, self.stride)
            ctx = o.sigmoid_mul_pair(ctx, gate)
            attn = o.q4_qmm(ctx, L["o"])
        r, normed2 = o.add_rmsnorm(h, attn, L["post_norm"], eps)   # decoder_layer.zig:752
        inter = o.silu_mul_pair(o.q4_qmm(normed2, L["gate"]), o.q4_qmm(normed2, L["up"]))
        return o.q4_qmm(inter, L["down"], residual=r)              # block_mlp.zig:216-258

    def prefill(self, tokens, start: int = 0, want_logits: bool = False, want_hidden: bool = False):
        """Ingest tokens at positions start.. (state kept from earlier calls);
        returns (next_token, logits|None) from the last row (and all rows'
        final-normed hiddens when want_hidden)."""
        o = self.o
        tok = np.asarray(tokens, np.uint32)
        h = o.embedding_many(self.embed, tok)                     # embedding.metal:73-96
        for i in range(len(self.layers)):
            h = self._prefill_layer(i, h, start)
        normed = o.rmsnorm(h, self.final_norm, self.cfg.rms_eps)
        nxt, logits = self._head(normed[-1], want_logits)
        return (nxt, logits, normed) if want_hidden else (nxt, logits)

    def teacher_forced(self, tokens, want_logits: bool = False):
        self.reset()
        preds, logits = [], []
        for pos, t in enumerate(tokens):
            tok, lg = self.step(int(t), pos, want_logits)
            preds.append(tok)
            logits.append(lg)
        return np.array(preds, np.uint32), logits
