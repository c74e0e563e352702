"""GPU parity of the Q4 GEMV family vs the C oracle (reference
shaders/linear.metal, shaders/linear_decode.metal, shaders/argmax.metal).

bf16 outputs: within rel 1e-2 of the fp32-accumulated oracle (one bf16 ulp
from a different summation order) — tests/helpers.assert_bf16_close.
Argmax: exact, on identical inputs to the reduction and on one-hot inputs
whose logits are exact on both sides.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close
from peregrine_amd.synth import Q4Weight, bf16_to_f32, f32_to_bf16, pack_q4, random_bf16, random_q4

pytestmark = pytest.mark.gpu

SHAPES = [(12288, 4096), (4096, 12288), (4096, 4096), (32, 4096), (8, 512), (64, 1536), (1024, 8192),
          (256, 6144)]


def _dev(a):
    from peregrine_amd.device import DeviceArray

    return DeviceArray.from_numpy(a)


def _lin(wt):
    from peregrine_amd.ops import Q4Linear

    return Q4Linear.upload(wt)


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 2])
def test_gemv_parity(gpu, orc, N, K, M):
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(N + K + M)
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (M, K))
    lin = _lin(wt)
    dx = _dev(x)
    dy = DeviceArray((M, N), np.uint16)
    lin.encode_bf16_fast(dx, dy, token_count=M)
    got = dy.numpy()
    ref = orc.q4_gemv(x, wt)
    assert_bf16_close(got, ref, min_exact=0.9, what=f"gemv {N}x{K} M={M}")


def test_gemv_config1_seed0(gpu, orc):
    """x ~ N(0,1) [1,4096], W [12288,4096], s ~ U(.001,.02),
    b ~ N(0,.05), seed 0."""
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(0)
    wt = random_q4(rng, 12288, 4096)
    x = random_bf16(rng, (1, 4096))
    lin = _lin(wt)
    dy = DeviceArray((1, 12288), np.uint16)
    lin.encode_bf16_fast(_dev(x), dy)
    stats = assert_bf16_close(dy.numpy(), orc.q4_gemv(x, wt), min_exact=0.95, what="config1")
    print("config1", stats)


def test_gemv_many_tokens(gpu, orc):
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(11)
    wt = random_q4(rng, 256, 2048)
    x = random_bf16(rng, (5, 2048))
    dy = DeviceArray((5, 256), np.uint16)
    _lin(wt).encode_bf16_fast(_dev(x), dy, token_count=5)
    assert_bf16_close(dy.numpy(), orc.q4_gemv(x, wt), what="5 tokens")


def test_gemv_one_hot_exact(gpu, orc):
    """x = e_k gives exactly representable logits on both sides: bit-exact."""
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(12)
    N, K = 64, 4096
    wt = random_q4(rng, N, K)
    lin = _lin(wt)
    dy = DeviceArray((1, N), np.uint16)
    for k in [0, 1, 7, 63, 64, 2047, 2048, 4095]:
        x = np.zeros((1, K), np.uint16)
        x[0, k] = f32_to_bf16(np.float32(1.0))[()]
        lin.encode_bf16_fast(_dev(x), dy)
        np.testing.assert_array_equal(dy.numpy(), orc.q4_gemv(x, wt), err_msg=f"k={k}")


@pytest.mark.parametrize("N,K", [(4096, 12288), (4096, 4096), (64, 1024)])
@pytest.mark.parametrize("M", [1, 2])
def test_residual_add_parity(gpu, orc, N, K, M):
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(N * 3 + K + M)
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (M, K))
    res = random_bf16(rng, (M, N), std=3.0)
    lin = _lin(wt)
    out = DeviceArray((M, N), np.uint16)
    if M == 1:
        lin.encode_bf16_fast_residual_add(_dev(x), _dev(res), out)
        got = out.numpy()
    else:
        o1 = DeviceArray((1, N), np.uint16)
        lin.encode_bf16_fast_residual_add2(_dev(x[:1]), _dev(x[1:]), _dev(res[:1]), _dev(res[1:]), out, o1)
        got = np.concatenate([out.numpy()[:1], o1.numpy()])
    assert_bf16_close(got, orc.q4_gemv_residual_add(x, wt, res), min_exact=0.9, what=f"resid {N}x{K}")


@pytest.mark.parametrize("N,K", [(12288, 4096), (512, 2048)])
@pytest.mark.parametrize("M", [1, 2])
def test_silu_gate_parity(gpu, orc, N, K, M):
    from peregrine_amd.device import DeviceArray
    from peregrine_amd.ops import gate_up_silu, gate_up_silu2

    rng = np.random.default_rng(N + 7 * K + M)
    g, u = random_q4(rng, N, K), random_q4(rng, N, K)
    x = random_bf16(rng, (M, K))
    lg, lu = _lin(g), _lin(u)
    if M == 1:
        out = DeviceArray((1, N), np.uint16)
        gate_up_silu(lg, lu, _dev(x), out)
        got = out.numpy()
    else:
        o0, o1 = DeviceArray((1, N), np.uint16), DeviceArray((1, N), np.uint16)
        gate_up_silu2(lg, lu, _dev(x[:1]), _dev(x[1:]), o0, o1)
        got = np.concatenate([o0.numpy(), o1.numpy()])
    assert_bf16_close(got, orc.q4_gemv_silu_gate(x, g, u), min_exact=0.9, what=f"silu {N}x{K}")


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288), (256, 6144)])
def test_fused_norm_equals_standalone_norm(gpu, N, K):
    """The GEMV's fused RMSNorm prologue and the standalone RMSNorm reduce in
    the same order, so rmsnorm-then-GEMV equals the fused launch bit for bit
    (plain and SiLU-pair epilogues). The model relies on it: decode fuses the
    final norm into the lm_head, the two-token verify normalises first."""
    from peregrine_amd._lib import call
    from peregrine_amd.device import DeviceArray, ptr
    from peregrine_amd.ops import gate_up_silu, rmsnorm

    rng = np.random.default_rng(N + K)
    wt, up = random_q4(rng, N, K), random_q4(rng, N, K)
    x = random_bf16(rng, (1, K), std=3.0)
    nw = random_bf16(rng, (K,), std=0.3, mean=1.0)
    lin, lup = _lin(wt), _lin(up)
    xd, nwd = _dev(x), _dev(nw)
    normed = DeviceArray((1, K), np.uint16)
    rmsnorm(xd, nwd, normed, K, 1, 1e-6)
    ref = DeviceArray((1, N), np.uint16)
    lin.encode_bf16_fast(normed, ref)
    fused = DeviceArray((1, N), np.uint16)
    call("prg_q4_gemv_norm_bf16", None, ptr(xd), ptr(nwd), 1e-6, *lin._wsb(), ptr(fused), N, K)
    np.testing.assert_array_equal(fused.numpy(), ref.numpy())

    ref2 = DeviceArray((1, N), np.uint16)
    gate_up_silu(lin, lup, normed, ref2)
    fused2 = DeviceArray((1, N), np.uint16)
    call("prg_q4_gemv_silu_gate_norm_bf16", None, ptr(xd), ptr(nwd), 1e-6, *lin._wsb(), *lup._wsb(), ptr(fused2),
         N, K)
    np.testing.assert_array_equal(fused2.numpy(), ref2.numpy())


def test_argmax_pairs_exact(gpu, orc):
    """Same partials in, same index out — ties, NaN, -inf, lengths."""
    from peregrine_amd.device import DeviceArray
    from peregrine_amd.ops import argmax_pairs

    rng = np.random.default_rng(13)
    out = DeviceArray((1,), np.uint32)
    for trial in range(40):
        n = int(rng.integers(1, 40000))
        vals = rng.integers(-4, 5, size=n).astype(np.float32)
        if trial % 5 == 1:
            vals[rng.integers(0, n, size=7)] = np.nan
        if trial % 5 == 2:
            vals[:] = -np.inf
        if trial % 5 == 3:
            vals = rng.normal(size=n).astype(np.float32)
        idx = rng.permutation(8 * n)[:n].astype(np.uint32)
        argmax_pairs(_dev(vals), _dev(idx), out, n)
        assert int(out.numpy()[0]) == orc.argmax_pairs(vals, idx), f"trial {trial} n={n}"


def test_argmax_partial_planted_ties(gpu, orc):
    """One-hot x makes every logit exact; planted equal logits exercise the
    first-strict-max rule inside a partial and the tie order across them."""
    from peregrine_amd.device import DeviceArray
    from peregrine_amd.ops import argmax_pairs

    N, K = 248320 // 40, 4096
    rng = np.random.default_rng(14)
    q = rng.integers(0, 12, size=(N, K), dtype=np.uint8)
    for r in [5, 6, 2051, 4099, 1030]:
        q[r, 100] = 15  # 5 tied maxima
    wt = Q4Weight(pack_q4(q), f32_to_bf16(np.full((N, K // 64), 0.5, np.float32)),
                  np.zeros((N, K // 64), np.uint16))
    x = np.zeros((1, K), np.uint16)
    x[0, 100] = f32_to_bf16(np.float32(1.0))[()]
    lin = _lin(wt)
    pv = DeviceArray((N // 8,), np.float32)
    pi = DeviceArray((N // 8,), np.uint32)
    lin.encode_bf16_argmax_partial(_dev(x), pv, pi)
    rpv, rpi = orc.q4_argmax_partial(x, wt)
    np.testing.assert_array_equal(pv.numpy(), rpv[0])
    np.testing.assert_array_equal(pi.numpy(), rpi[0])
    out = DeviceArray((1,), np.uint32)
    argmax_pairs(pv, pi, out, N // 8)
    assert int(out.numpy()[0]) == orc.argmax_pairs(rpv[0], rpi[0])


@pytest.mark.parametrize("M", [1, 2])
def test_lm_head_argmax_full_vocab(gpu, orc, M):
    """Full lm_head shape 248320x4096: partial values within bf16 tolerance,
    and the final token equal to the oracle's whenever the oracle's top-2
    logit margin exceeds two bf16 ulps (otherwise a summation-order flip is
    legitimate)."""
    from peregrine_amd.device import DeviceArray
    from peregrine_amd.ops import argmax_pairs

    N, K = 248320, 4096
    rng = np.random.default_rng(15 + M)
    wt = random_q4(rng, N, K, zero_mean=True)
    x = random_bf16(rng, (M, K))
    lin = _lin(wt)
    pv = [DeviceArray((N // 8,), np.float32) for _ in range(M)]
    pi = [DeviceArray((N // 8,), np.uint32) for _ in range(M)]
    dx = [_dev(x[m:m + 1]) for m in range(M)]
    if M == 1:
        lin.encode_bf16_argmax_partial(dx[0], pv[0], pi[0])
    else:
        lin.encode_bf16_argmax_partial2(dx[0], dx[1], pv[0], pi[0], pv[1], pi[1])
    rpv, rpi = orc.q4_argmax_partial(x, wt)
    out = DeviceArray((1,), np.uint32)
    for m in range(M):
        gv = pv[m].numpy()
        assert_bf16_close(f32_to_bf16(gv), f32_to_bf16(rpv[m]), min_exact=0.95, what="partials")
        argmax_pairs(pv[m], pi[m], out, N // 8)
        tok = int(out.numpy()[0])
        ref_tok = orc.argmax_pairs(rpv[m], rpi[m])
        srt = np.sort(rpv[m])
        margin = float(srt[-1] - srt[-2])
        ulp = float(np.abs(srt[-1])) * 2.0**-7
        if margin > 2 * ulp:
            assert tok == ref_tok
        # The GPU reduction is exact on the GPU's own partials:
        assert tok == orc.argmax_pairs(gv, pi[m].numpy())


def test_dequantize_exact(gpu, orc):
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(16)
    wt = random_q4(rng, 96, 1024)
    out = DeviceArray((96, 1024), np.uint16)
    _lin(wt).dequantize(out)
    np.testing.assert_array_equal(out.numpy(), orc.q4_dequantize(wt))


def test_bad_shape_is_an_error(gpu):
    from peregrine_amd._lib import PrgError
    from peregrine_amd.device import DeviceArray

    rng = np.random.default_rng(17)
    wt = random_q4(rng, 12, 512)  # out_dim not a multiple of 8
    lin = _lin(wt)
    with pytest.raises(PrgError):
        lin.encode_bf16_fast(_dev(random_bf16(rng, (1, 512))), DeviceArray((12,), np.uint16))
