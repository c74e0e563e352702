"""The HIP kernels against the committed known-answer vectors (tests/golden),
through the C ABI: the Q4 GEMV, the lm_head argmax pair reduction, one Gated
DeltaNet decode step and GQA decode attention. The expected values were
computed from the mathematics (float64) by tests/golden/make_golden.py, so
these checks do not go through the oracle at all.

Bars: the argmax winner is exact; bf16 outputs within rel 1e-2 of the
float64 value (one bf16 ulp) with an RMS floor; the GDN state within rel 1e-3
(the north star's state tolerance).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

from peregrine_amd.synth import Q4Weight, bf16_to_f32

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

from make_golden import GDN_SAMPLE, gdn_state  # noqa: E402


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN / "golden_v1.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _d(a):
    from peregrine_amd.device import DeviceArray

    return DeviceArray.from_numpy(np.ascontiguousarray(a))


def _e(shape, dtype=np.uint16):
    from peregrine_amd.device import DeviceArray

    return DeviceArray(shape, dtype)


def _close(got: np.ndarray, ref: np.ndarray, rtol: float = 1e-2, floor: float = 1e-3) -> None:
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = np.abs(got - ref)
    bad = err > rtol * np.abs(ref) + floor * rms
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} outside tolerance; max err {err.max():.3g}, rms {rms:.3g}"


def test_golden_gemv_gpu(gpu, gold):
    from peregrine_amd.ops import Q4Linear

    wt = Q4Weight(w=gold["gemv_w"], s=gold["gemv_s"], b=gold["gemv_b"])
    y = _e((1, 64))
    Q4Linear.upload(wt).encode_bf16_fast(_d(gold["gemv_x"][None, :]), y)
    got = bf16_to_f32(y.numpy()[0]).astype(np.float64)
    _close(got, gold["gemv_y_f64"])
    assert np.mean(y.numpy()[0] == gold["gemv_y_bf16"]) >= 0.9


def test_golden_argmax_gpu(gpu, gold):
    from peregrine_amd.ops import argmax_pairs

    vals, idx = gold["argmax_values"], gold["argmax_indices"]
    out = _e((1,), np.uint32)
    argmax_pairs(_d(vals), _d(idx), out, vals.size)
    assert int(out.numpy()[0]) == int(gold["argmax_winner"][0])


def test_golden_gdn_gpu(gpu, gold):
    from peregrine_amd import ops

    dS = _d(gdn_state())
    y = _e((4096,))
    ops.gated_delta_decode(dS, _d(gold["gdn_conv"]), _d(gold["gdn_a"]), _d(gold["gdn_b"]), _d(gold["gdn_A_log"]),
                           _d(gold["gdn_dt_bias"]), y, True)
    _close(bf16_to_f32(y.numpy()).astype(np.float64), gold["gdn_y_f64"])
    samp = dS.numpy().reshape(-1)[::GDN_SAMPLE].astype(np.float64)
    _close(samp, gold["gdn_S_new_sample_f64"], rtol=1e-3, floor=1e-4)


def test_golden_attn_gpu(gpu, gold):
    from peregrine_amd import ops

    out = _e((16 * 256,))
    part = _e((ops.attn_partials_bytes(64) // 4,), np.float32)
    ops.attn_decode(_d(gold["attn_q"]), _d(gold["attn_k"]), _d(gold["attn_v"]), _d(gold["attn_gate"]), out, part,
                    64, 64)
    _close(bf16_to_f32(out.numpy()).astype(np.float64), gold["attn_out_f64"])
