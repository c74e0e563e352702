"""GPU parity of the norm, embedding, Gated DeltaNet and attention kernels vs
the C oracle (reference shaders/rmsnorm.metal, embedding.metal, conv1d.metal,
gated_delta.metal, gated_norm.metal, attention.metal, attention_decode.metal).

Tolerances: bf16 outputs within rel 1e-2 (helpers.assert_bf16_close); GDN
state within rel 1e-3 (north star); pure data movement (cache append, gate
split, embedding rows) bit-exact.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close
from peregrine_amd.synth import bf16_to_f32, f32_to_bf16, random_bf16, random_q4

pytestmark = pytest.mark.gpu


def _d(a):
    from peregrine_amd.device import DeviceArray

    return DeviceArray.from_numpy(a)


def _e(shape, dtype=np.uint16):
    from peregrine_amd.device import DeviceArray

    return DeviceArray(shape, dtype)


def test_rmsnorm(gpu, orc):
    from peregrine_amd import ops

    rng = np.random.default_rng(0)
    x = random_bf16(rng, (3, 4096), std=2.0)
    w = random_bf16(rng, (4096,), std=0.1, mean=1.0)
    out = _e((3, 4096))
    ops.rmsnorm(_d(x), _d(w), out, 4096, 3)
    assert_bf16_close(out.numpy(), orc.rmsnorm(x, w), min_exact=0.98, what="rmsnorm")


@pytest.mark.parametrize("hidden", [4096, 4104, 8192, 12288])
def test_add_rmsnorm(gpu, orc, hidden):
    """Rows up to 8192 wide normalise the rounded sum from registers, wider
    ones read it back (4104: one thread holds a third unit). Either way the
    normalised row equals the standalone RMSNorm of the stored sum bit for
    bit, and the sum equals the oracle's."""
    from peregrine_amd import ops

    rng = np.random.default_rng(1 + hidden)
    a, b = random_bf16(rng, (2, hidden), std=3.0), random_bf16(rng, (2, hidden), std=3.0)
    w = random_bf16(rng, (hidden,), std=0.1, mean=1.0)
    r, n, n2 = _e((2, hidden)), _e((2, hidden)), _e((2, hidden))
    wd = _d(w)
    ops.add_rmsnorm(_d(a), _d(b), wd, r, n, hidden, 2)
    ops.rmsnorm(r, wd, n2, hidden, 2)
    rr, rn = orc.add_rmsnorm(a, b, w)
    np.testing.assert_array_equal(r.numpy(), rr)
    np.testing.assert_array_equal(n.numpy(), n2.numpy())
    assert_bf16_close(n.numpy(), rn, min_exact=0.98, what="add_rmsnorm")


def test_embedding_exact(gpu, orc):
    from peregrine_amd import ops
    from peregrine_amd.ops import Q4Linear

    rng = np.random.default_rng(2)
    wt = random_q4(rng, 1000, 4096)
    table = Q4Linear.upload(wt)
    out = _e((4096,))
    for tok in [0, 1, 499, 999]:
        ops.embedding_gather(table, tok, out)
        np.testing.assert_array_equal(out.numpy(), orc.embedding(wt, tok))
    from peregrine_amd._lib import PrgError

    with pytest.raises(PrgError):
        ops.embedding_gather(table, 1000, out)  # InvalidTokenId (model.zig:806)


def test_conv1d_decode(gpu, orc):
    from peregrine_amd import ops

    rng = np.random.default_rng(3)
    state = rng.normal(size=(3, 8192)).astype(np.float32)
    w = random_bf16(rng, (8192, 4), std=0.5)
    ds, dw = _d(state), _d(w)
    for step in range(4):
        x = random_bf16(rng, (8192,))
        out = _e((8192,))
        ops.conv1d_silu_decode(ds, _d(x), dw, out)
        ref, state = orc.conv1d_decode(state, x, w)
        assert_bf16_close(out.numpy(), ref, min_exact=0.99, what=f"conv step {step}")
        np.testing.assert_array_equal(ds.numpy(), state)


def _gdn(rng):
    conv = random_bf16(rng, (8192,))
    a, b = random_bf16(rng, (32,)), random_bf16(rng, (32,))
    A_log = rng.normal(0, 0.5, 32).astype(np.float32)
    dt = random_bf16(rng, (32,), std=0.5)
    S = rng.normal(0, 0.1, size=(32, 128, 128)).astype(np.float32)
    return conv, a, b, A_log, dt, S


@pytest.mark.parametrize("has_prev", [True, False])
def test_gated_delta_decode(gpu, orc, has_prev):
    from peregrine_amd import ops

    rng = np.random.default_rng(4 + has_prev)
    conv, a, b, A_log, dt, S = _gdn(rng)
    dS = _d(S)
    y = _e((4096,))
    ops.gated_delta_decode(dS, _d(conv), _d(a), _d(b), _d(A_log), _d(dt), y, has_prev)
    ry, rS = orc.gated_delta_decode(S, conv, a, b, A_log, dt, has_prev)
    assert_bf16_close(y.numpy(), ry, min_exact=0.95, what="gdn y")
    gS = dS.numpy()
    np.testing.assert_allclose(gS, rS, rtol=1e-3, atol=1e-3 * float(np.sqrt(np.mean(rS * rS))))


def test_gated_delta_multistep_state(gpu, orc):
    """24 steps of one layer: state stays within rel 1e-3 of the oracle's."""
    from peregrine_amd import ops

    rng = np.random.default_rng(6)
    _, _, _, A_log, dt, S = _gdn(rng)
    dS = _d(S)
    dA, ddt = _d(A_log), _d(dt)
    y = _e((4096,))
    for step in range(24):
        conv = random_bf16(rng, (8192,))
        a, b = random_bf16(rng, (32,)), random_bf16(rng, (32,))
        ops.gated_delta_decode(dS, _d(conv), _d(a), _d(b), dA, ddt, y, True)
        ry, S = orc.gated_delta_decode(S, conv, a, b, A_log, dt, True)
        assert_bf16_close(y.numpy(), ry, what=f"gdn step {step}")
    gS = dS.numpy()
    np.testing.assert_allclose(gS, S, rtol=1e-3, atol=1e-3 * float(np.sqrt(np.mean(S * S))))


def test_gated_delta_fused_norm(gpu, orc):
    from peregrine_amd import ops

    rng = np.random.default_rng(7)
    conv, a, b, A_log, dt, S = _gdn(rng)
    nw = random_bf16(rng, (128,), std=0.1, mean=1.0)
    z = random_bf16(rng, (4096,))
    out = _e((4096,))
    ops.gated_delta_decode_norm(_d(S), _d(conv), _d(a), _d(b), _d(A_log), _d(dt), _d(nw), _d(z), out)
    ry, _ = orc.gated_delta_decode(S, conv, a, b, A_log, dt, True)
    ref = orc.rmsnorm_gated(ry, nw, z, 128)
    assert_bf16_close(out.numpy(), ref, min_exact=0.9, what="gdn+norm")


@pytest.mark.parametrize("shift", [0, 1])
def test_rmsnorm_gated(gpu, orc, shift):
    """shift 0: 16-byte aligned rows (16 lanes per row); shift 1: x, gate and
    out one bf16 element past alignment, which takes the one-block-per-row
    kernel. Both against the oracle (gated_norm.metal:163-189)."""
    from peregrine_amd._lib import call
    from peregrine_amd.device import ptr

    rng = np.random.default_rng(8)
    x, z = random_bf16(rng, (4096,)), random_bf16(rng, (4096,))
    w = random_bf16(rng, (128,), std=0.1, mean=1.0)
    pad = np.zeros(shift, np.uint16)
    dx, dz, dw = _d(np.concatenate([pad, x])), _d(np.concatenate([pad, z])), _d(w)
    out = _e((4096 + shift,))

    def at(a):
        return ptr(a).value + 2 * shift

    call("prg_rmsnorm_gated_bf16", None, at(dx), ptr(dw), at(dz), at(out), 128, 1e-6, 32)
    got = out.numpy()[shift:]
    assert_bf16_close(got, orc.rmsnorm_gated(x, w, z, 128), min_exact=0.97, what=f"gated norm shift {shift}")


@pytest.mark.parametrize("pos", [0, 7, 4096, 65535])
def test_attn_prepare(gpu, orc, pos):
    from peregrine_amd import ops

    rng = np.random.default_rng(9 + pos)
    stride = 512
    dst = pos % stride
    pq = random_bf16(rng, (16 * 512,))
    qw, kw = random_bf16(rng, (256,), std=0.1, mean=1.0), random_bf16(rng, (256,), std=0.1, mean=1.0)
    kin, vin = random_bf16(rng, (4 * 256,)), random_bf16(rng, (4 * 256,))
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    dkc, dvc = _d(kc), _d(vc)
    q, g = _e((16 * 256,)), _e((16 * 256,))
    ops.attn_decode_prepare(_d(pq), _d(qw), q, g, _d(kin), _d(vin), _d(kw), dkc, dvc, stride, dst, pos)
    rq, rg, rkc, rvc = orc.attn_prepare(pq, qw, kin, vin, kw, kc, vc, stride, dst, pos)
    np.testing.assert_array_equal(g.numpy(), rg)
    np.testing.assert_array_equal(dvc.numpy(), rvc)
    assert_bf16_close(q.numpy(), rq, min_exact=0.97, what="q")
    gk = dkc.numpy()
    mask = np.ones(stride, bool)
    mask[dst] = False
    np.testing.assert_array_equal(gk[:, mask], rkc[:, mask])  # untouched slots
    assert_bf16_close(gk[:, dst], rkc[:, dst], min_exact=0.97, what="k")


@pytest.mark.parametrize("L,stride", [(1, 64), (100, 128), (1025, 2048), (4096, 4096), (24576, 24576),
                                      (65536, 65536), (2000, 65536)])
def test_attn_decode(gpu, orc, L, stride):
    from peregrine_amd import ops

    rng = np.random.default_rng(L)
    q = random_bf16(rng, (16 * 256,))
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    if L < stride:  # slots past seq_len must not leak in, even as NaN
        kc[:, L:] = 0x7FC0
        vc[:, :, L:] = 0x7FC0
    gate = random_bf16(rng, (16 * 256,))
    out = _e((16 * 256,))
    part = _e((ops.attn_partials_bytes(stride) // 4,), np.float32)
    ops.attn_decode(_d(q), _d(kc), _d(vc), _d(gate), out, part, stride, L)
    ref = orc.attn_decode(q, kc, vc, gate, stride, L)
    assert_bf16_close(out.numpy(), ref, min_exact=0.8, what=f"attn L={L}")


def test_attn_decode_bad_len_is_error(gpu):
    from peregrine_amd import ops
    from peregrine_amd._lib import PrgError

    z = _e((16 * 256,))
    with pytest.raises(PrgError):
        ops.attn_decode(z, z, z, z, z, z, 64, 65)


@pytest.mark.parametrize("L,stride", [(0, 64), (1, 64), (100, 128), (1023, 2048), (4095, 4096), (30000, 65536),
                                      (24575, 24576), (65535, 65536)])
def test_attn_decode_step(gpu, orc, L, stride):
    """prg_attn_decode_step_bf16 (q/k norm + RoPE, attention over the L cached
    slots plus the new token, K/V append at slot L) against the oracle's
    prepare (attention.metal:327-421) then flash decode over L + 1 tokens.
    The last two cases are BASELINE config 4's contexts (24576 and 65536
    tokens attended) on the path the model runs, with the new token in the
    cache's last slot."""
    from peregrine_amd import ops

    rng = np.random.default_rng(100 + L)
    pq = random_bf16(rng, (16 * 512,))
    qw, kw = random_bf16(rng, (256,), std=0.1, mean=1.0), random_bf16(rng, (256,), std=0.1, mean=1.0)
    kin, vin = random_bf16(rng, (4 * 256,)), random_bf16(rng, (4 * 256,))
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    kc[:, L:] = 0x7FC0  # slots from L on are not attended before the append, even as NaN
    vc[:, :, L:] = 0x7FC0
    dkc, dvc = _d(kc), _d(vc)
    out = _e((16 * 256,))
    ws = _e((ops.attn_step_workspace_bytes(stride),), np.uint8)
    ops.attn_decode_step(_d(pq), _d(qw), _d(kin), _d(vin), _d(kw), dkc, dvc, out, ws, stride, L, L)
    rq, rg, rkc, rvc = orc.attn_prepare(pq, qw, kin, vin, kw, kc, vc, stride, L, L)
    ref = orc.attn_decode(rq, rkc, rvc, rg, stride, L + 1)
    assert_bf16_close(out.numpy(), ref, min_exact=0.8, what=f"attn step L={L}")
    gk, gv = dkc.numpy(), dvc.numpy()
    np.testing.assert_array_equal(gv[:, :, L], rvc[:, :, L])  # V column copied
    assert_bf16_close(gk[:, L], rkc[:, L], min_exact=0.97, what="appended k")
    np.testing.assert_array_equal(gk[:, :L], kc[:, :L])  # cached slots untouched
    np.testing.assert_array_equal(gv[:, :, :L], vc[:, :, :L])
