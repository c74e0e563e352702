"""GPU parity of the matrix-core Q4 GEMV over the decode layout
(peregrine_amd/csrc/q4_gemv_t16.hip) vs the C oracle (reference
shaders/linear.metal:158-255, shaders/argmax.metal:6-43).

The decode layout is a permutation of the MLX bytes: checked bit for bit
against a numpy restatement of its index map. GEMV outputs: within the bf16
tolerance of the fp32-accumulated oracle (a different summation order,
tests/helpers.assert_bf16_close); an M = 2 launch's rows equal M = 1 launches
bit for bit (the two-token verify relies on it). Argmax: exact on one-hot
inputs with planted ties; on random inputs the token equals the oracle's
whenever the oracle's top-2 margin is decisive.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close
from peregrine_amd.synth import Q4Weight, f32_to_bf16, pack_q4, random_bf16, random_q4

pytestmark = pytest.mark.gpu


def repack_ref(wt):
    """The decode layout's index map restated in numpy: unit (tile, window,
    step, lane = j + 16 c) holds words 32 window + 16 step + 4 c .. +3 of row
    16 tile + j; meta entry (tile, window, lane) is group 4 window + c."""
    N, K = wt.shape
    W = K // 256
    w6 = wt.w.reshape(N // 16, 16, W, 2, 4, 4)  # tile, j, window, step, c, word
    tw = np.ascontiguousarray(w6.transpose(0, 2, 3, 4, 1, 5)).reshape(-1)

    def meta(a):
        m4 = a.reshape(N // 16, 16, W, 4)  # tile, j, window, c
        return np.ascontiguousarray(m4.transpose(0, 2, 3, 1)).reshape(-1)

    return tw, meta(wt.s), meta(wt.b)


class T16Weight:
    """A device copy of wt in the decode layout, through the op layer's
    DecodeLayoutQ4 (prg_q4_repack_t16 and the decode-layout entry points)."""

    def __init__(self, wt):
        from peregrine_amd.ops import DecodeLayoutQ4, Q4Linear

        self.N, self.K = wt.shape
        self._src = Q4Linear.upload(wt)
        self.lin = DecodeLayoutQ4(self._src)
        self.dst = [self.lin.weight, self.lin.scales, self.lin.biases]

    def ptrs(self):
        return list(self.lin._wsb())

    def gemv(self, x):
        from peregrine_amd.device import DeviceArray

        M = x.shape[0]
        dx = DeviceArray.from_numpy(np.ascontiguousarray(x))
        dy = DeviceArray((M, self.N), np.uint16)
        self.lin.encode_bf16_fast(dx, dy, token_count=M)
        return dy.numpy()

    def argmax(self, x):
        from peregrine_amd.device import DeviceArray
        from peregrine_amd.ops import t16_argmax_workspace_bytes

        M = x.shape[0]
        dx = DeviceArray.from_numpy(np.ascontiguousarray(x))
        out = DeviceArray((2,), np.uint32)
        ws = DeviceArray((t16_argmax_workspace_bytes(),), np.uint8)
        self.lin.encode_argmax(dx, out, ws, token_count=M)
        return [int(v) for v in out.numpy()[:M]]


@pytest.mark.parametrize("N,K", [(64, 4096), (32, 12288), (48, 8192)])
def test_repack_layout_exact(gpu, N, K):
    rng = np.random.default_rng(N + K)
    wt = random_q4(rng, N, K)
    t = T16Weight(wt)
    tw, ts, tb = repack_ref(wt)
    np.testing.assert_array_equal(t.dst[0].numpy().reshape(-1), tw)
    np.testing.assert_array_equal(t.dst[1].numpy().reshape(-1), ts)
    np.testing.assert_array_equal(t.dst[2].numpy().reshape(-1), tb)


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288), (4096, 8192), (9216, 4096), (1024, 4096)])
@pytest.mark.parametrize("M", [1, 2])
def test_t16_gemv_parity(gpu, orc, N, K, M):
    rng = np.random.default_rng(3 * N + K + M)
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (M, K))
    got = T16Weight(wt).gemv(x)
    assert_bf16_close(got, orc.q4_gemv(x, wt), min_exact=0.9, what=f"t16 gemv {N}x{K} M={M}")


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288)])
def test_t16_two_rows_equal_single_rows(gpu, N, K):
    """Each row of an M = 2 launch has the bits of the M = 1 launch on that row."""
    rng = np.random.default_rng(N + 2 * K)
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (2, K))
    t = T16Weight(wt)
    both = t.gemv(x)
    np.testing.assert_array_equal(both[0], t.gemv(x[:1])[0])
    np.testing.assert_array_equal(both[1], t.gemv(x[1:])[0])


def test_t16_gemv_bad_shapes_are_errors(gpu):
    from peregrine_amd._lib import PrgError, call

    with pytest.raises(PrgError):
        call("prg_q4_gemv_t16_bf16", None, 1, 1, 1, 1, 1, 1, 40, 4096)  # out_dim % 16
    with pytest.raises(PrgError):
        call("prg_q4_gemv_t16_bf16", None, 1, 1, 1, 1, 1, 1, 64, 2048)  # no kernel for in_dim 2048


@pytest.mark.parametrize("M", [1, 2])
def test_t16_argmax_planted_ties(gpu, orc, M):
    """One-hot x with s = 0.5, b = 0 makes every logit exact (0.5 q); planted
    equal maxima exercise the first-strict-max rule inside an 8-row partial
    and the tie order across partials and blocks."""
    N, K = 248320 // 40, 4096
    rng = np.random.default_rng(14 + M)
    q = rng.integers(0, 12, size=(N, K), dtype=np.uint8)
    for r in [5, 6, 2051, 4099, 1030, 6207]:
        q[r, 100] = 15
    for r in [17, 3000]:
        q[r, 200] = 15
    wt = Q4Weight(pack_q4(q), f32_to_bf16(np.full((N, K // 64), 0.5, np.float32)), np.zeros((N, K // 64), np.uint16))
    x = np.zeros((M, K), np.uint16)
    x[0, 100] = f32_to_bf16(np.float32(1.0))[()]
    if M == 2:
        x[1, 200] = f32_to_bf16(np.float32(1.0))[()]
    got = T16Weight(wt).argmax(x)
    rpv, rpi = orc.q4_argmax_partial(x, wt)
    for m in range(M):
        assert got[m] == orc.argmax_pairs(rpv[m], rpi[m]), f"row {m}"


@pytest.mark.parametrize("M", [1, 2])
def test_t16_argmax_full_vocab(gpu, orc, M):
    """lm_head shape 248320 x 4096: the token equals the oracle's whenever the
    oracle's top-2 logit margin exceeds two bf16 ulps of the top logit."""
    N, K = 248320, 4096
    rng = np.random.default_rng(25 + M)
    wt = random_q4(rng, N, K, zero_mean=True)
    x = random_bf16(rng, (M, K))
    got = T16Weight(wt).argmax(x)
    rpv, rpi = orc.q4_argmax_partial(x, wt)
    for m in range(M):
        srt = np.sort(rpv[m])
        margin = float(srt[-1] - srt[-2])
        ulp = float(np.abs(srt[-1])) * 2.0**-7
        if margin > 2 * ulp:
            assert got[m] == orc.argmax_pairs(rpv[m], rpi[m]), f"row {m}"


@pytest.mark.parametrize("N", [12288, 10240, 1024])
def test_t16_silu_gate_norm_parity(gpu, orc, N):
    """The model's post-attention RMSNorm + gate/up SiLU launch on the decode
    layout vs the oracle's rmsnorm then SiLU pair (block_mlp.zig:313-345).
    12288 rows is the 9B MLP, 10240 the attention q/k/v row count, 1024 a
    launch of few tiles."""
    from peregrine_amd._lib import call
    from peregrine_amd.device import DeviceArray, ptr

    K = 4096
    rng = np.random.default_rng(N + 11)
    g, u = random_q4(rng, N, K), random_q4(rng, N, K)
    x = random_bf16(rng, (1, K), std=3.0)
    nw = random_bf16(rng, (K,), std=0.3, mean=1.0)
    tg, tu = T16Weight(g), T16Weight(u)
    dx, dnw = DeviceArray.from_numpy(x), DeviceArray.from_numpy(nw)
    out = DeviceArray((1, N), np.uint16)
    call("prg_q4_gemv_t16_silu_gate_norm_bf16", None, ptr(dx), ptr(dnw), 1e-6, *tg.ptrs(), *tu.ptrs(), ptr(out), N, K)
    want = orc.q4_gemv_silu_gate(orc.rmsnorm(x, nw, 1e-6), g, u)
    assert_bf16_close(out.numpy(), want, min_exact=0.9, what=f"t16 silu norm {N}x{K}")
