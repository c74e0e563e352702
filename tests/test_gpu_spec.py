"""GPU checks of the multi-token-prediction path: the two-token verify
(src/model/model.zig:1627-1659, decoder_layer.zig:485-516), the MTP drafter
(src/model/mtp.zig:137-280) against the oracle's restatement, and the
device-resident speculative loop (src/server/decode_loop.zig:163-311).

The speculative loop must emit exactly the plain greedy tokens: every
per-token kernel of the verify is the single-token kernel (the M = 2 GEMVs do
the same per-row arithmetic), and a rejected draft's GDN update is undone
from the row-0 snapshot. Drafters with random weights are almost never
accepted, so one test rewrites the drafter into a "copy" drafter whose draft
is the current token (fc selects the target hidden, o_proj and down_proj are
zero): it is accepted exactly where the greedy sequence repeats a token, which
exercises the accept path and the state swap.
"""
import ctypes as C

import numpy as np
import pytest

from peregrine_amd.synth import f32_to_bf16, random_bf16

pytestmark = pytest.mark.gpu

SMALL = dict(num_layers=4, hidden=1024, intermediate=2048, vocab=4096, mtp_layers=1)


def _write(m, name, arr):
    from peregrine_amd._lib import call

    p, n = m.tensor_ptr(name)
    arr = np.ascontiguousarray(arr)
    assert arr.nbytes == n, (name, arr.nbytes, n)
    call("prg_hip_memcpy", C.c_void_p(p), arr.ctypes.data_as(C.c_void_p), C.c_size_t(n), 0, None, 1)


def _make_copy_drafter(m, H):
    """fc = [0 | I] (draft input = the target hidden), attention and MLP
    outputs zero, unit norms: draft = argmax lm_head(h) = the current token."""
    q = np.zeros((H, 2 * H), np.uint32)
    q[np.arange(H), H + np.arange(H)] = 1
    words = np.zeros((H, 2 * H // 8), np.uint32)
    for j in range(8):
        words |= q[:, j::8] << np.uint32(4 * j)
    _write(m, "mtp.fc.weight", words)
    one = f32_to_bf16(np.float32(1.0))
    _write(m, "mtp.fc.scales", np.full((H, 2 * H // 64), one, np.uint16))
    _write(m, "mtp.fc.biases", np.zeros((H, 2 * H // 64), np.uint16))
    for t in ["mtp.layers.0.self_attn.o_proj", "mtp.layers.0.mlp.down_proj"]:
        _, n = m.tensor_ptr(t + ".scales")
        _write(m, t + ".scales", np.zeros(n // 2, np.uint16))
        _write(m, t + ".biases", np.zeros(n // 2, np.uint16))
    _write(m, "mtp.pre_fc_norm_hidden.weight", np.full(H, one, np.uint16))
    _write(m, "mtp.norm.weight", np.full(H, one, np.uint16))


@pytest.fixture(scope="module")
def model(gpu):
    from peregrine_amd.model import DeviceModel, ModelConfig

    m = DeviceModel(ModelConfig(**SMALL), seed=11)
    yield m
    m.close()


def _greedy(m, prompt, n):
    from peregrine_amd.model import ModelState

    st = ModelState(m, max_seq=128)
    first = st.prefill(prompt)
    rest, _ = st.decode(n - 1)
    st.close()
    return np.concatenate([[first], rest]).astype(np.uint32)


def test_two_token_verify_equals_two_single_steps(model):
    """forward_two_tokens == forward_next_token twice: same tokens and the
    same GDN states / KV caches, bit for bit."""
    from peregrine_amd.model import ModelConfig, ModelState

    rng = np.random.default_rng(0)
    prompt = rng.integers(0, SMALL["vocab"], size=12).astype(np.uint32)
    a, b = ModelState(model, max_seq=64), ModelState(model, max_seq=64)
    a.prefill(prompt)
    b.prefill(prompt)
    t0, t1 = 17, 4000
    v, bonus = a.forward_two_tokens(t0, t1, 12)
    n0 = b.forward_next_token(t0, 12)
    n1 = b.forward_next_token(t1, 13)
    assert (v, bonus) == (n0, n1)
    cfg = ModelConfig(**SMALL)
    for i in range(SMALL["num_layers"]):
        names = ["recur", "conv"] if cfg.is_linear(i) else ["cache_k", "cache_v"]
        for nm in names:
            np.testing.assert_array_equal(a.read(f"layers.{i}.{nm}", np.uint16), b.read(f"layers.{i}.{nm}", np.uint16),
                                          err_msg=f"layer {i} {nm}")
    a.close()
    b.close()


def test_mtp_drafter_matches_oracle(model):
    """Drafter prefill over 6 rows, then 3 draft steps, against the oracle's
    restatement of mtp.zig (same bf16 inputs: random normalised-scale hidden
    rows standing in for the target's). Draft tokens must agree wherever the
    oracle's top-2 logit margin exceeds 4 bf16 ulps of the top logit."""
    from oracle.model import OracleModel
    from peregrine_amd.device import DeviceArray
    from peregrine_amd.model import ModelState

    rng = np.random.default_rng(1)
    H = SMALL["hidden"]
    st = ModelState(model, max_seq=64)
    om = OracleModel(model, 64)
    toks = rng.integers(0, SMALL["vocab"], size=9).astype(np.uint32)
    hid = random_bf16(rng, (9, H), std=1.0)
    st.mtp_prefill(toks[:6], DeviceArray.from_numpy(hid[:6]), 0)
    om.mtp_prefill(toks[:6], hid[:6], 0)
    checked = 0
    for j in range(6, 9):
        d = st.mtp_draft(int(toks[j]), DeviceArray.from_numpy(hid[j]), j)
        ref, logits = om.mtp_step(int(toks[j]), hid[j], j, want_logits=True)
        srt = np.sort(logits)
        guard = 4 * 2.0 ** (np.floor(np.log2(max(abs(srt[-1]), 1e-30))) - 7)
        print(f"draft step {j}: gpu {d} oracle {ref} margin {srt[-1] - srt[-2]:.4f} guard {guard:.4f}")
        if srt[-1] - srt[-2] > guard:
            checked += 1
            assert d == ref
    assert checked >= 1
    # the drafter's K cache after the steps
    gk = st.read("layers.3.cache_k", np.uint16)  # target layer untouched by the drafter
    assert not gk.any()
    st.close()


def test_speculative_equals_greedy_random_drafter(model):
    from peregrine_amd.model import ModelState

    rng = np.random.default_rng(2)
    prompt = rng.integers(0, SMALL["vocab"], size=16).astype(np.uint32)
    ref = _greedy(model, prompt, 24)
    st = ModelState(model, max_seq=128)
    toks, acc, att, ms = st.generate_speculative(prompt, 24)
    print(f"random drafter: accepted {acc}/{att}, {ms:.2f} ms")
    np.testing.assert_array_equal(toks, ref)
    assert att >= 12 and ms > 0
    st.close()


def test_speculative_equals_greedy_copy_drafter(gpu):
    """With the copy drafter every immediate repeat in the greedy sequence is
    an accepted draft; the emitted tokens still equal greedy decoding."""
    from peregrine_amd.model import DeviceModel, ModelConfig, ModelState

    m = DeviceModel(ModelConfig(**SMALL), seed=13)
    _make_copy_drafter(m, SMALL["hidden"])
    # Final norm weight e_0: the logits become w[:, 0] * h_0 / rms, so greedy
    # output is one of two tokens (by the sign of h_0) and repeats often.
    e0 = np.zeros(SMALL["hidden"], np.uint16)
    e0[0] = int(f32_to_bf16(np.float32(1.0)))
    _write(m, "language_model.model.norm.weight", e0)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, SMALL["vocab"], size=20).astype(np.uint32)
    n = 48
    ref = _greedy(m, prompt, n)
    repeats = int(np.sum(ref[1:] == ref[:-1]))
    st = ModelState(m, max_seq=128)
    toks, acc, att, ms = st.generate_speculative(prompt, n)
    print(f"copy drafter: greedy repeats {repeats}, accepted {acc}/{att}")
    np.testing.assert_array_equal(toks, ref)
    assert acc <= repeats
    assert repeats >= 4, "the two-token target should repeat"
    assert acc >= 2, "the copy drafter never matched a repeat"
    # the loop again on the same state object gives the same tokens (state reset)
    toks2, acc2, _, _ = st.generate_speculative(prompt, n)
    np.testing.assert_array_equal(toks2, ref)
    assert acc2 == acc
    st.close()
    m.close()


def test_speculative_errors(model):
    from peregrine_amd._lib import PrgError
    from peregrine_amd.model import DeviceModel, ModelConfig, ModelState

    st = ModelState(model, max_seq=32)
    with pytest.raises(PrgError) as e:
        st.generate_speculative(np.zeros(20, np.uint32), 11)  # 20 + 11 + 2 > 32
    assert e.value.code == 5
    st.close()
    plain = DeviceModel(ModelConfig(num_layers=4, hidden=1024, intermediate=2048, vocab=4096), seed=1)
    ps = ModelState(plain, max_seq=32)
    with pytest.raises(PrgError):
        ps.generate_speculative(np.zeros(4, np.uint32), 4)  # no drafter weights
    ps.close()
    plain.close()
