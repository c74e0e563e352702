"""The oracle's model composition (oracle/model.py) against an independent
float reference: transformers' Qwen3.5 text model and a drafter assembled
from transformers modules, both in float64 with the same (dequantised)
weights. Fixture: tests/golden/hf_v1.npz, written by
tests/golden/make_hf_golden.py.

What this pins: the wiring of src/model/decoder_layer.zig:461-566,644-819,
block_linear.zig:199-469, block_attn.zig:261-631, block_mlp.zig:155-311,
model.zig:686-717 and mtp.zig:188-280 as restated by OracleModel (which
weights feed which op, norm placement, the q | gate split, the conv tap
order, the GDN gates and state carry, the residual stream, the drafter's
concat order and positions). The kernel-level arithmetic and rounding points
are pinned elsewhere (tests/test_oracle_*.py, tests/test_golden.py).

Tolerance. The oracle rounds to bf16 at every stage the reference does; the
fixture never rounds. The logits' relative RMS difference is 1.4-3.2% per
position for the target (growing ~0.5-0.8% per layer through the residual
stream) and ~0.8% for the drafter, so the bound is 5% (target) and 3%
(drafter). Every planted wiring mistake tested below moves it to >= 10%.
Top-1 must agree wherever the fixture's top-2 margin exceeds 4 bf16 ulps of
its top logit (23 of the 24 target positions and every drafter slot here).

One wiring mistake is invisible by construction: exchanging q_norm and
k_norm leaves q.k unchanged outside the 64 rotary dims (each score term is
q_i w_qi k_i w_ki), so no logit comparison can see it.
"""
from __future__ import annotations

import copy
from pathlib import Path

import numpy as np
import pytest

from hostmodel import HostModel
from peregrine_amd.model import ModelConfig
from peregrine_amd.synth import bf16_to_f32, f32_to_bf16

FIXTURE = Path(__file__).resolve().parent / "golden" / "hf_v1.npz"
TARGET_RTOL = 0.05
DRAFT_RTOL = 0.03


@pytest.fixture(scope="module")
def fx():
    z = np.load(FIXTURE, allow_pickle=False)
    c = [int(v) for v in z["config"]]
    cfg = ModelConfig(num_layers=c[0], hidden=c[1], intermediate=c[2], vocab=c[3], mtp_layers=c[4])
    hm = HostModel(cfg, int(z["seed"]))
    assert hm.digest() == str(z["digest"]), "host model generator changed: regenerate the fixture"
    return {"z": z, "hm": hm, "cfg": cfg}


def _oracle(fx):
    from oracle.model import OracleModel

    om = OracleModel(fx["hm"], 64)
    om.o.set_threads(8)
    return om


def relrms(g, r) -> float:
    g, r = np.asarray(g, np.float64), np.asarray(r, np.float64)
    return float(np.sqrt(np.mean((g - r) ** 2)) / np.sqrt(np.mean(r * r)))


def decisive(ref_logits) -> bool:
    s = np.sort(np.asarray(ref_logits, np.float64))
    guard = 4 * 2.0 ** (np.floor(np.log2(max(abs(s[-1]), 1e-30))) - 7)
    return bool(s[-1] - s[-2] > guard)


def target_report(om, z):
    preds, logits = om.teacher_forced(z["prompt"], want_logits=True)
    ref = z["logits"]
    errs = [relrms(logits[n], ref[n]) for n in range(len(ref))]
    dec = [n for n in range(len(ref)) if decisive(ref[n])]
    agree = [n for n in dec if int(preds[n]) == int(np.argmax(ref[n]))]
    return errs, dec, agree, preds


def draft_report(om, z, split: int = 12):
    """Drafter prefill over slots [0, split) then one draft step per slot
    after it; slot j reads token j + 1 and the fixture's hidden row j."""
    p, hid, ref = z["prompt"], f32_to_bf16(z["hidden"]), z["draft_logits"]
    om.mtp_prefill(p[1:split + 1], hid[:split], 0)
    out = []
    for j in range(split, len(p) - 1):
        tok, lg = om.mtp_step(int(p[j + 1]), hid[j], j, want_logits=True)
        out.append((j, relrms(lg, ref[j]), decisive(ref[j]), int(tok) == int(np.argmax(ref[j]))))
    return out


def test_fixture_is_self_consistent(fx):
    z = fx["z"]
    assert z["logits"].shape == (len(z["prompt"]), fx["cfg"].vocab)
    assert z["draft_logits"].shape == (len(z["prompt"]) - 1, fx["cfg"].vocab)
    assert np.isfinite(z["logits"]).all() and np.isfinite(z["draft_logits"]).all()


def test_decode_route_matches_transformers(fx):
    errs, dec, agree, _ = target_report(_oracle(fx), fx["z"])
    print("relrms per position:", [round(e, 4) for e in errs])
    assert max(errs) <= TARGET_RTOL, errs
    assert len(dec) >= 20, f"only {len(dec)} decisive positions"
    assert agree == dec, f"top-1 differs at {sorted(set(dec) - set(agree))}"


def test_prefill_route_matches_transformers_and_decode_route(fx):
    """One 24-token layer-major prefill: the final-normed rows against the
    fixture's, every row's logits against the fixture's, and the per-row
    tokens against the decode route on decisive rows."""
    z = fx["z"]
    om = _oracle(fx)
    nxt, last_logits, normed = om.prefill(z["prompt"], want_logits=True, want_hidden=True)
    assert relrms(bf16_to_f32(normed), z["hidden"]) <= TARGET_RTOL
    assert relrms(last_logits, z["logits"][-1]) <= TARGET_RTOL
    row_logits = bf16_to_f32(om.o.q4_gemv(normed, om.lm_head))
    _, _, _, dec_preds = target_report(_oracle(fx), z)
    for n in range(len(z["prompt"])):
        assert relrms(row_logits[n], z["logits"][n]) <= TARGET_RTOL, n
        if decisive(z["logits"][n]):
            assert int(np.argmax(row_logits[n])) == int(np.argmax(z["logits"][n])) == int(dec_preds[n]), n
    assert nxt == dec_preds[-1]


def test_drafter_matches_transformers_parts(fx):
    rows = draft_report(_oracle(fx), fx["z"])
    print("drafter relrms:", [round(r[1], 4) for r in rows])
    assert all(r[1] <= DRAFT_RTOL for r in rows), rows
    assert sum(r[2] for r in rows) >= 8
    assert all(r[3] for r in rows if r[2]), rows


# ---- planted mistakes: each must be rejected by the same bounds -----------
def _swap_norms(om):
    for L in om.layers:
        L["input_norm"], L["post_norm"] = L["post_norm"], L["input_norm"]


def _swap_gate_up(om):
    for L in om.layers:
        L["gate"], L["up"] = L["up"], L["gate"]


def _swap_q_gate(om):
    for L in om.layers:
        if not L["linear"]:
            L["q"] = copy.deepcopy(L["q"])
            for arr in (L["q"].w, L["q"].s, L["q"].b):
                a = arr.reshape(16, 2, 256, -1)
                a[:] = a[:, ::-1].copy()


def _conv_reversed(om):
    for L in om.layers:
        if L["linear"]:
            L["conv_w"] = np.ascontiguousarray(L["conv_w"][:, ::-1])


def _unit_final_norm(om):
    om.final_norm = np.full_like(om.final_norm, 0x3F80)


def _unit_gated_norm(om):
    for L in om.layers:
        if L["linear"]:
            L["norm_w"] = np.full_like(L["norm_w"], 0x3F80)


def _no_dt_bias(om):
    for L in om.layers:
        if L["linear"]:
            L["dt_bias"] = np.zeros_like(L["dt_bias"])


@pytest.mark.parametrize("plant", [_swap_norms, _swap_gate_up, _swap_q_gate, _conv_reversed, _unit_final_norm,
                                   _unit_gated_norm, _no_dt_bias], ids=lambda f: f.__name__.strip("_"))
def test_planted_wiring_mistake_is_rejected(fx, plant):
    om = _oracle(fx)
    plant(om)
    errs, dec, agree, _ = target_report(om, fx["z"])
    assert max(errs) > 2 * TARGET_RTOL, f"{plant.__name__}: relrms {max(errs):.4f} not caught"


def test_planted_gdn_state_carry_mistake_is_rejected(fx, monkeypatch):
    """GDN layers that ignore the carried state (has_previous_state = 0 at
    every position, decoder_layer.zig:564)."""
    from oracle.model import OracleModel

    orig = OracleModel._decode_layer
    monkeypatch.setattr(OracleModel, "_decode_layer",
                        lambda self, L, S, h, pos: orig(self, L, S, h, 0 if L["linear"] else pos))
    errs, _, _, _ = target_report(_oracle(fx), fx["z"])
    assert max(errs) > 2 * TARGET_RTOL


def test_planted_drafter_concat_order_is_rejected(fx, monkeypatch):
    """[norm(hidden) | norm(embed)] instead of the reference's
    [norm(embed) | norm(hidden)] (mtp.zig:262-270)."""
    from oracle.model import OracleModel

    orig = OracleModel._pre_fc

    def swapped(self, tokens, hidden_rows):
        x = orig(self, tokens, hidden_rows)
        H = x.shape[1] // 2
        return np.ascontiguousarray(np.concatenate([x[:, H:], x[:, :H]], axis=1))

    monkeypatch.setattr(OracleModel, "_pre_fc", swapped)
    rows = draft_report(_oracle(fx), fx["z"])
    assert max(r[1] for r in rows) > 2 * DRAFT_RTOL
