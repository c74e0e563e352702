"""The oracle against the committed known-answer vectors (tests/golden).

The vectors were computed by tests/golden/make_golden.py from the mathematics
alone (float64 dense products, the textbook delta rule, softmax attention, and
a plain-Python step-by-step run of argmax_pairs_f32_u32's thread scan and
halving tree), not by the oracle, so these tests pin the oracle's restatements
of linear_decode.metal / argmax.metal / gated_delta.metal /
attention_decode.metal to an independent answer on fixed inputs.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

from peregrine_amd.synth import Q4Weight, bf16_to_f32

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

from make_golden import GDN_SAMPLE, argmax_sim, bf16_rne_from_f64, gdn_state  # noqa: E402


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN / "golden_v1.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _wt(g) -> Q4Weight:
    return Q4Weight(w=g["gemv_w"], s=g["gemv_s"], b=g["gemv_b"])


def test_golden_gemv_vectors_are_consistent(gold):
    """The stored bf16 answer is the RNE rounding of the stored float64 dot,
    which is the dense product of the stored inputs."""
    wt = _wt(gold)
    y64 = wt.dequant_f64() @ bf16_to_f32(gold["gemv_x"]).astype(np.float64)
    np.testing.assert_allclose(y64, gold["gemv_y_f64"], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(bf16_rne_from_f64(gold["gemv_y_f64"]), gold["gemv_y_bf16"])


def test_golden_gemv_oracle(gold, orc):
    """fp32 accumulation may only move a result across a bf16 rounding
    boundary when the float64 value lies within the fp32 error bound of it."""
    wt = _wt(gold)
    got = orc.q4_gemv(gold["gemv_x"][None, :], wt)[0]
    ref = gold["gemv_y_bf16"]
    y64 = gold["gemv_y_f64"]
    # fp32 error bound of a K-term sum: K * eps32 * sum |x_k w_k|
    dense = np.abs(wt.dequant_f64()) @ np.abs(bf16_to_f32(gold["gemv_x"]).astype(np.float64))
    bound = 1024 * 2.0 ** -24 * dense
    mismatch = got != ref
    for i in np.nonzero(mismatch)[0]:
        g = float(bf16_to_f32(got[i]))
        r = float(bf16_to_f32(ref[i]))
        mid = 0.5 * (g + r)
        assert abs(y64[i] - mid) <= bound[i], (i, g, r, y64[i])
    assert mismatch.mean() <= 0.05


def test_golden_argmax_oracle(gold, orc):
    assert orc.argmax_pairs(gold["argmax_values"], gold["argmax_indices"]) == int(gold["argmax_winner"][0])


def test_golden_argmax_simulation_is_stored_winner(gold):
    # the plain-Python run of the reference's scan and tree reproduces the stored winner
    assert argmax_sim(gold["argmax_values"], gold["argmax_indices"]) == int(gold["argmax_winner"][0])


def test_golden_gdn_oracle(gold, orc):
    """y within 1 bf16 ulp (rel 1e-2) of the float64 delta rule; the new state
    within rel 1e-4 on the stored sample."""
    S = gdn_state()
    y, S_new = orc.gated_delta_decode(S, gold["gdn_conv"], gold["gdn_a"], gold["gdn_b"], gold["gdn_A_log"],
                                      gold["gdn_dt_bias"], True)
    y64 = gold["gdn_y_f64"]
    yg = bf16_to_f32(y).astype(np.float64)
    rms = float(np.sqrt(np.mean(y64 * y64)))
    assert np.all(np.abs(yg - y64) <= 1e-2 * np.abs(y64) + 1e-3 * rms)
    samp = S_new.reshape(-1)[::GDN_SAMPLE].astype(np.float64)
    ref = gold["gdn_S_new_sample_f64"]
    srms = float(np.sqrt(np.mean(ref * ref)))
    np.testing.assert_allclose(samp, ref, rtol=1e-4, atol=1e-5 * srms)


def test_golden_attn_oracle(gold, orc):
    out = orc.attn_decode(gold["attn_q"], gold["attn_k"], gold["attn_v"], gold["attn_gate"], 64, 64)
    ref = gold["attn_out_f64"]
    got = bf16_to_f32(out).astype(np.float64)
    rms = float(np.sqrt(np.mean(ref * ref)))
    assert np.all(np.abs(got - ref) <= 1e-2 * np.abs(ref) + 1e-3 * rms)
