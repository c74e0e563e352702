"""GPU parity of the prompt-path (prefill) kernels vs the C oracle: the MFMA
Q4 QMM family (shaders/linear.metal:780-988), attention prepare + causal
prefill attention (shaders/attention.metal:146-220, 1463-1523;
src/model/block_attn.zig:500-631), conv1d prefill (shaders/conv1d.metal:136-198)
and the Gated DeltaNet prefill (shaders/gated_norm.metal:191-268,
gated_delta.metal:35-138).

Tolerances: bf16 outputs within rel 1e-2 (helpers.assert_bf16_close) with a
stated bit-exact fraction; f32 q/k/gates rel 1e-5; GDN state rel 1e-3; data
movement (cache append, gate split) bit-exact. At the full 9B shapes, where the
oracle is too slow for whole outputs, sampled rows are checked against it and
the rest through row independence.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close
from peregrine_amd.synth import bf16_to_f32, random_bf16, random_q4

pytestmark = pytest.mark.gpu


def _d(a):
    from peregrine_amd.device import DeviceArray

    return DeviceArray.from_numpy(np.ascontiguousarray(a))


def _e(shape, dtype=np.uint16):
    from peregrine_amd.device import DeviceArray

    return DeviceArray(shape, dtype)


# ------------------------------------------------------------------ QMM ----
@pytest.mark.parametrize("M,N,K", [(1, 256, 512), (37, 96, 1024), (130, 1024, 512), (300, 8192, 1024),
                                   (64, 32, 4096), (200, 4096, 12288 // 4)])
def test_qmm_vs_oracle(gpu, orc, M, N, K):
    from peregrine_amd.ops import Q4Linear

    print(f"[qmm] M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N)
    wt = random_q4(rng, N, K, zero_mean=True)
    x = random_bf16(rng, (M, K), std=2.0)
    lin = Q4Linear.upload(wt)
    out = _e((M, N))
    lin.encode_prefill_qmm(_d(x), out, M)
    gpu.synchronize()
    assert_bf16_close(out.numpy(), orc.q4_qmm(x, wt), min_exact=0.97, what=f"qmm {M}x{N}x{K}")


def test_qmm_residual_and_silu_pair(gpu, orc):
    from peregrine_amd import ops
    from peregrine_amd.ops import Q4Linear

    rng = np.random.default_rng(3)
    M, N, K = 77, 320, 1024
    g, u = random_q4(rng, N, K, zero_mean=True), random_q4(rng, N, K, zero_mean=True)
    x = random_bf16(rng, (M, K), std=2.0)
    res = random_bf16(rng, (M, N), std=3.0)
    G, U = Q4Linear.upload(g), Q4Linear.upload(u)
    out = _e((M, N))
    G.encode_prefill_qmm_residual_add(_d(x), _d(res), out, M)
    gpu.synchronize()
    assert_bf16_close(out.numpy(), orc.q4_qmm(x, g, residual=res), min_exact=0.97, what="qmm residual")
    ops.prefill_gate_up_silu(G, U, _d(x), out, M)
    gpu.synchronize()
    ref = orc.silu_mul_pair(orc.q4_qmm(x, g), orc.q4_qmm(x, u))
    assert_bf16_close(out.numpy(), ref, min_exact=0.95, what="qmm silu pair")


def test_qmm_full_shape_rows(gpu, orc):
    """The MLP gate projection at the config-5 prompt shape (1600 x 12288 x
    4096): 6 sampled rows against the oracle; every row equals the same
    row computed alone (row independence, bit-exact)."""
    from peregrine_amd.ops import Q4Linear

    rng = np.random.default_rng(4)
    M, N, K = 1600, 12288, 4096
    wt = random_q4(rng, N, K, zero_mean=True)
    x = random_bf16(rng, (M, K), std=2.0)
    lin = Q4Linear.upload(wt)
    xd = _d(x)
    out = _e((M, N))
    lin.encode_prefill_qmm(xd, out, M)
    gpu.synchronize()
    full = out.numpy()
    rows = np.array([0, 1, 127, 128, 1000, 1599])
    assert_bf16_close(full[rows], orc.q4_qmm(x[rows], wt), min_exact=0.97, what="qmm full-shape sampled rows")
    for r0 in (0, 1536):
        part = _e((64, N))
        lin.encode_prefill_qmm(_d(x[r0:r0 + 64]), part, 64)
        gpu.synchronize()
        np.testing.assert_array_equal(part.numpy(), full[r0:r0 + 64])


def test_qmm_rejects_bad_shapes(gpu):
    from peregrine_amd._lib import PrgError
    from peregrine_amd.ops import Q4Linear

    rng = np.random.default_rng(5)
    lin = Q4Linear.upload(random_q4(rng, 64, 512))
    x, out = _e((4, 512)), _e((4, 64))
    with pytest.raises(PrgError):
        lin.encode_prefill_qmm(x, out, 0)


# ------------------------------------------------------------ attention ----
def _prepare_inputs(rng, T, stride):
    qp = random_bf16(rng, (T, 16 * 512), std=2.0)
    k = random_bf16(rng, (T, 4 * 256), std=2.0)
    v = random_bf16(rng, (T, 4 * 256))
    qw = random_bf16(rng, (256,), std=0.1, mean=1.0)
    kw = random_bf16(rng, (256,), std=0.1, mean=1.0)
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    return qp, k, v, qw, kw, kc, vc


@pytest.mark.parametrize("T,start", [(1, 0), (9, 0), (20, 300)])
def test_attn_prefill_prepare_vs_oracle(gpu, orc, T, start):
    from peregrine_amd import ops

    rng = np.random.default_rng(T + start)
    stride = 512
    qp, k, v, qw, kw, kc, vc = _prepare_inputs(rng, T, stride)
    q_out, gate = _e((T, 4096)), _e((T, 4096))
    kcd, vcd = _d(kc), _d(vc)
    ops.attn_prefill_prepare(_d(qp), _d(qw), _d(k), _d(kw), _d(v), q_out, gate, kcd, vcd, T, start, start, stride)
    gpu.synchronize()
    rq, rg = orc.split_qg_many(qp)
    np.testing.assert_array_equal(gate.numpy(), rg)
    rq2, rkc, rvc = orc.qk_norm_rope_append_many(rq, qw, k, kw, v, kc, vc, start, start, stride)
    assert_bf16_close(q_out.numpy(), rq2, min_exact=0.98, what="prefill q")
    gk = kcd.numpy().reshape(4, stride, 256)
    assert_bf16_close(gk, rkc.reshape(4, stride, 256), min_exact=0.98, what="prefill K cache")
    np.testing.assert_array_equal(vcd.numpy(), rvc)


def _check_attn(got, ref, vc, what):
    """Probabilities are rounded to bf16 on both sides; the GPU's exp2 and the
    oracle's differ in the last f32 bit, which now and then flips one
    probability by an ulp and moves the outputs of that (row, head) by up to
    2^-8 * p * |v|. Bound: one output ulp plus one such flip at p <= 1, with
    99% of outputs bit-exact (the same bound pins the oracle against float64)."""
    g, r = bf16_to_f32(got).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    assert np.isfinite(g).all(), what
    bound = 2.0 ** -7 * np.abs(r) + 2.0 ** -8 * np.abs(bf16_to_f32(vc)).max()
    bad = np.abs(g - r) > bound
    exact = float(np.mean(got == ref))
    print(f"{what}: exact {exact:.5f}, max err {np.abs(g - r).max():.3e}")
    assert not bad.any(), f"{what}: {int(bad.sum())} outside the bound"
    assert exact >= 0.99, f"{what}: bit-exact fraction {exact}"


@pytest.mark.parametrize("T,prefix", [(1, 0), (5, 0), (67, 0), (130, 0), (9, 100), (70, 200)])
def test_attn_prefill_vs_oracle(gpu, orc, T, prefix):
    from peregrine_amd import ops

    print(f"[attn_prefill] T={T} prefix={prefix}", flush=True)
    rng = np.random.default_rng(T * 31 + prefix)
    stride = 512
    q = random_bf16(rng, (T, 4096))
    gate = random_bf16(rng, (T, 4096), std=2.0)
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    out = _e((T, 4096))
    scores = _e((ops.attn_prefill_scores_bytes(T, prefix) // 2,))
    ops.attn_prefill(_d(q), _d(kc), _d(vc), _d(gate), out, scores, T, prefix, stride)
    gpu.synchronize()
    ref = orc.sigmoid_mul_pair(orc.attn_prefill(q, kc, vc, T, prefix, stride), gate)
    _check_attn(out.numpy(), ref, vc, f"attn prefill T={T} prefix={prefix}")


def test_attn_prefill_chunks_match_whole(gpu):
    """A prompt attended in one call equals the same prompt split in two calls
    (second with prefix = first), bit for bit: rows never read past their own
    position and the GEMMs' per-element sums do not depend on the row tiling."""
    from peregrine_amd import ops

    rng = np.random.default_rng(9)
    T, stride, T1 = 150, 256, 61
    q = random_bf16(rng, (T, 4096))
    gate = random_bf16(rng, (T, 4096))
    kc, vc = _d(random_bf16(rng, (4, stride, 256))), _d(random_bf16(rng, (4, 256, stride)))
    whole = _e((T, 4096))
    scores = _e((ops.attn_prefill_scores_bytes(T, 0) // 2,))
    ops.attn_prefill(_d(q), kc, vc, _d(gate), whole, scores, T, 0, stride)
    a, b = _e((T1, 4096)), _e((T - T1, 4096))
    ops.attn_prefill(_d(q[:T1]), kc, vc, _d(gate[:T1]), a, scores, T1, 0, stride)
    ops.attn_prefill(_d(q[T1:]), kc, vc, _d(gate[T1:]), b, scores, T - T1, T1, stride)
    gpu.synchronize()
    w = whole.numpy()
    np.testing.assert_array_equal(a.numpy(), w[:T1])
    np.testing.assert_array_equal(b.numpy(), w[T1:])


# ------------------------------------------------------------------ GDN ----
@pytest.mark.parametrize("T,has_prev", [(1, True), (2, False), (17, True), (100, False)])
def test_conv1d_prefill_vs_oracle(gpu, orc, T, has_prev):
    from peregrine_amd import ops

    rng = np.random.default_rng(T + 7 * has_prev)
    state = bf16_to_f32(random_bf16(rng, (3, 8192), std=2.0))
    w = random_bf16(rng, (8192, 4), std=0.5)
    x = random_bf16(rng, (T, 8192), std=2.0)
    sd, out = _d(state), _e((T, 8192))
    ops.conv1d_silu_prefill(sd, _d(x), _d(w), out, T, has_prev)
    gpu.synchronize()
    ro, rs = orc.conv1d_prefill(state, x, w, has_prev)
    assert_bf16_close(out.numpy(), ro, min_exact=0.999, what="conv prefill")
    np.testing.assert_array_equal(sd.numpy(), rs)


def _gdn_inputs(rng, T):
    co = random_bf16(rng, (T, 8192), std=1.5)
    a = random_bf16(rng, (T, 32), std=1.0)
    b = random_bf16(rng, (T, 32), std=1.0)
    A_log = rng.uniform(-4, -1, 32).astype(np.float32)
    dtb = random_bf16(rng, (32,), std=0.5)
    state = (rng.normal(size=(32, 128, 128)) * 0.1).astype(np.float32)
    return co, a, b, A_log, dtb, state


def test_gdn_prefill_prepare_vs_oracle(gpu, orc):
    from peregrine_amd import ops

    rng = np.random.default_rng(11)
    T = 33
    co, a, b, A_log, dtb, _ = _gdn_inputs(rng, T)
    qn, kn = _e((T, 2048), np.float32), _e((T, 2048), np.float32)
    g, beta = _e((T, 32), np.float32), _e((T, 32), np.float32)
    kq = _e((T, 16), np.float32)
    ops.gated_delta_prefill_prepare(_d(co), _d(a), _d(b), _d(A_log), _d(dtb), qn, kn, g, beta, T, kq_out=kq)
    gpu.synchronize()
    rq, rk = orc.qk_l2norm_prefill(co)
    # k.q of the normalised pair, per (token, k-head): the float64 dot of the
    # oracle's vectors (|kq| <= 1/sqrt(128) since both are unit-norm up to it).
    ref_kq = np.einsum("thd,thd->th", rq.reshape(T, 16, 128).astype(np.float64), rk.reshape(T, 16, 128))
    np.testing.assert_allclose(kq.numpy(), ref_kq, rtol=1e-4, atol=1e-6)
    rg, rb = orc.gating_many(A_log, a, dtb, b)
    np.testing.assert_allclose(qn.numpy(), rq, rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(kn.numpy(), rk, rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(g.numpy(), rg, rtol=1e-5)
    np.testing.assert_allclose(beta.numpy(), rb, rtol=1e-5)


@pytest.mark.parametrize("T,has_prev", [(1, True), (7, False), (64, True)])
def test_gdn_prefill_vs_oracle(gpu, orc, T, has_prev):
    from peregrine_amd import ops

    rng = np.random.default_rng(T * 3 + has_prev)
    co, a, b, A_log, dtb, state = _gdn_inputs(rng, T)
    qn, kn = orc.qk_l2norm_prefill(co)
    g, beta = orc.gating_many(A_log, a, dtb, b)
    sd, y = _d(state), _e((T, 4096))
    ops.gated_delta_prefill(sd, _d(qn), _d(kn), _d(co), _d(g), _d(beta), y, T, has_prev)
    gpu.synchronize()
    ry, rs = orc.gated_delta_prefill(state, qn, kn, co, g, beta, has_prev)
    assert_bf16_close(y.numpy(), ry, min_exact=0.95, what=f"gdn prefill y T={T}")
    gs = sd.numpy().astype(np.float64)
    rel = np.linalg.norm(gs - rs) / np.linalg.norm(rs)
    print(f"gdn prefill state rel {rel:.2e}")
    assert rel <= 1e-3
