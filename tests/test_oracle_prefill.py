"""Pin the oracle's prompt-path (prefill) restatements: the Q4 QMM
(shaders/linear.metal:780-941), the materialised causal attention
(src/model/block_attn.zig:500-631, shaders/attention.metal:146-220,1463-1523),
and the Gated DeltaNet prefill kernels (shaders/conv1d.metal:136-198,
gated_norm.metal:191-268, gated_delta.metal:35-138). Pins are float64
references, exact identities with the (separately pinned) decode restatements,
limiting cases and invariants. CPU only.
"""
import numpy as np
import pytest

from peregrine_amd.synth import bf16_to_f32, f32_to_bf16, random_bf16, random_q4

F = lambda b: bf16_to_f32(b).astype(np.float64)  # noqa: E731


def ulps(a_bits, b_bits):
    return np.abs(a_bits.astype(np.int64) - b_bits.astype(np.int64))


def bf(x):
    return f32_to_bf16(np.asarray(x, np.float64).astype(np.float32))


# -------------------------------------------------------------- A22 QMM ---
@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (37, 96, 512), (130, 40, 1024)])
def test_qmm_is_gemm_over_bf16_rounded_weights(orc, M, N, K):
    rng = np.random.default_rng(M + N)
    wt = random_q4(rng, N, K, zero_mean=True)
    x = random_bf16(rng, (M, K), std=2.0)
    got = orc.q4_qmm(x, wt)
    w_rounded = F(orc.q4_dequantize(wt))           # bf16(s*q + b), pinned elsewhere
    ref = bf(F(x) @ w_rounded.T)
    d = ulps(got, ref)
    assert d.max() <= 1
    assert np.mean(d == 0) >= 0.99
    # The rounding of the weights is visible: the unrounded product disagrees
    # on a clearly larger share of outputs.
    unrounded = bf(F(x) @ wt.dequant_f64().T)
    assert np.mean(ulps(unrounded, ref) != 0) > 4 * np.mean(d != 0) + 0.005


def test_qmm_residual_rounds_twice(orc):
    rng = np.random.default_rng(5)
    wt = random_q4(rng, 64, 256, zero_mean=True)
    x = random_bf16(rng, (9, 256), std=2.0)
    plain = orc.q4_qmm(x, wt)
    np.testing.assert_array_equal(orc.q4_qmm(x, wt, residual=np.zeros_like(plain)), plain)
    neg = plain ^ np.uint16(0x8000)
    assert np.all(F(orc.q4_qmm(x, wt, residual=neg)) == 0.0)
    res = random_bf16(rng, plain.shape, std=4.0)
    got = orc.q4_qmm(x, wt, residual=res)
    assert ulps(got, bf(F(plain) + F(res))).max() == 0


def test_qmm_row_independent(orc):
    rng = np.random.default_rng(6)
    wt = random_q4(rng, 48, 512, zero_mean=True)
    x = random_bf16(rng, (11, 512))
    full = orc.q4_qmm(x, wt)
    for m in [0, 5, 10]:
        np.testing.assert_array_equal(orc.q4_qmm(x[m:m + 1], wt)[0], full[m])


def test_silu_and_sigmoid_pairs_vs_float64(orc):
    rng = np.random.default_rng(7)
    g = random_bf16(rng, (4096,), std=3.0)
    u = random_bf16(rng, (4096,), std=3.0)
    gf, uf = F(g), F(u)
    assert ulps(orc.silu_mul_pair(g, u), bf(gf / (1 + np.exp(-gf)) * uf)).max() <= 1
    assert ulps(orc.sigmoid_mul_pair(u, g), bf(uf / (1 + np.exp(-gf)))).max() <= 1


def test_embedding_many_matches_single_rows(orc):
    rng = np.random.default_rng(8)
    wt = random_q4(rng, 200, 512)
    toks = np.array([3, 0, 199, 3, 77], np.uint32)
    out = orc.embedding_many(wt, toks)
    for i, t in enumerate(toks):
        np.testing.assert_array_equal(out[i], orc.embedding(wt, int(t)))


# ----------------------------------------------- A23 attention prefill ---
def test_split_qg_many_layout(orc):
    rng = np.random.default_rng(9)
    qp = random_bf16(rng, (3, 16 * 512))
    q, g = orc.split_qg_many(qp)
    r = qp.reshape(3, 16, 2, 256)
    np.testing.assert_array_equal(q, r[:, :, 0, :].reshape(3, -1))
    np.testing.assert_array_equal(g, r[:, :, 1, :].reshape(3, -1))


def _rope_ref(x, w, pos, theta=1.0e7, rot=64):
    xf = F(x)
    n = xf / np.sqrt(np.mean(xf * xf) + 1e-6) * F(w)
    out = n.copy()
    half = rot // 2
    i = np.arange(half)
    # The reference forms the angle in f32 (float(pos) * inv_freq); at large
    # positions that rounding dominates, so the float64 reference takes the
    # same f32 angle and is exact from there on.
    inv = np.float32(theta) ** (-(np.float32(2.0) * i.astype(np.float32)) / np.float32(rot))
    ang = (np.float32(pos) * inv.astype(np.float32)).astype(np.float64)
    a, b = n[:half], n[half:rot]
    out[:half] = a * np.cos(ang) - b * np.sin(ang)
    out[half:rot] = b * np.cos(ang) + a * np.sin(ang)
    return out


def _rope_err(got, ref):
    """Error in units of one bf16 ulp of the reference value, except that a
    rotated pair cancelling to near zero is held to 1e-5 of the row RMS."""
    g = F(got)
    ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -8
    floor = 1e-5 * np.sqrt(np.mean(ref * ref))
    return float(np.max(np.abs(g - ref) / np.maximum(ulp, floor)))


def test_qk_norm_rope_append_many_vs_float64(orc):
    rng = np.random.default_rng(10)
    T, stride, start_cache, start_rope = 5, 64, 7, 1000
    q = random_bf16(rng, (T, 16 * 256), std=2.0)
    k = random_bf16(rng, (T, 4 * 256), std=2.0)
    v = random_bf16(rng, (T, 4 * 256))
    qw = random_bf16(rng, (256,), std=0.1, mean=1.0)
    kw = random_bf16(rng, (256,), std=0.1, mean=1.0)
    kc0 = random_bf16(rng, (4 * stride * 256,))
    vc0 = random_bf16(rng, (4 * 256 * stride,))
    q2, kc, vc = orc.qk_norm_rope_append_many(q, qw, k, kw, v, kc0, vc0, start_rope, start_cache, stride)
    kc = kc.reshape(4, stride, 256)
    vc = vc.reshape(4, 256, stride)
    worst = 0
    for t in range(T):
        for h in range(16):
            ref = _rope_ref(q[t, h * 256:(h + 1) * 256], qw, start_rope + t)
            worst = max(worst, _rope_err(q2.reshape(T, 16, 256)[t, h], ref))
        for h in range(4):
            ref = _rope_ref(k[t, h * 256:(h + 1) * 256], kw, start_rope + t)
            worst = max(worst, _rope_err(kc[h, start_cache + t], ref))
            np.testing.assert_array_equal(vc[h, :, start_cache + t], v[t, h * 256:(h + 1) * 256])
    assert worst <= 2  # one bf16 ulp is 2^-8..2^-7 of the value
    # Untouched cache slots keep their contents.
    mask = np.ones(stride, bool)
    mask[start_cache:start_cache + T] = False
    np.testing.assert_array_equal(kc[:, mask], kc0.reshape(4, stride, 256)[:, mask])
    np.testing.assert_array_equal(vc[:, :, mask], vc0.reshape(4, 256, stride)[:, :, mask])


def _attn_inputs(rng, T, prefix, stride):
    q = random_bf16(rng, (T, 16 * 256))
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    return q, kc, vc


def _attn_prefill_f64(q, kc, vc, T, prefix, scale=1.0 / 16):
    """float64 restatement with the reference's three bf16 rounding points."""
    out = np.zeros((T, 16, 256))
    L = prefix + T
    qf = F(q).reshape(T, 16, 256)
    for h in range(16):
        g = h // 4
        s = F(bf(qf[:, h, :] @ F(kc[g, :L]).T)) * scale    # bf16 scores, scale after
        mask = np.arange(L)[None, :] > (prefix + np.arange(T))[:, None]
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p = F(bf(p / p.sum(axis=1, keepdims=True)))
        out[:, h, :] = p @ F(vc[g, :, :L]).T
    return bf(out.reshape(T, -1))


@pytest.mark.parametrize("T,prefix", [(1, 0), (7, 0), (33, 0), (5, 40), (300, 20)])
def test_attn_prefill_vs_float64(orc, T, prefix):
    rng = np.random.default_rng(T * 100 + prefix)
    stride = 512
    q, kc, vc = _attn_inputs(rng, T, prefix, stride)
    got = orc.attn_prefill(q, kc, vc, T, prefix, stride)
    ref = _attn_prefill_f64(q, kc, vc, T, prefix)
    # Probabilities are rounded to bf16 on both sides, so an f32-vs-f64
    # difference in exp() occasionally flips one of them by an ulp; such a
    # flip moves every output of that (row, head) by <= 2^-8 * p * |v|.
    # Bound: one output ulp plus one probability-ulp flip at p <= 1; and
    # 99% of outputs must agree bit for bit (a wrong scale, mask or rounding
    # point breaks most of them).
    e = np.abs(F(got) - F(ref))
    r = F(ref)
    assert np.all(e <= 2.0 ** -7 * np.abs(r) + 2.0 ** -8 * np.abs(F(vc)).max())
    assert np.mean(ulps(got, ref) == 0) >= 0.99


def test_attn_prefill_first_row_sees_only_itself(orc):
    rng = np.random.default_rng(11)
    T, stride = 4, 64
    q, kc, vc = _attn_inputs(rng, T, 0, stride)
    got = orc.attn_prefill(q, kc, vc, T, 0, stride).reshape(T, 16, 256)
    for h in range(16):
        np.testing.assert_array_equal(got[0, h], vc[h // 4, :, 0])


def test_attn_prefill_is_causal_and_chunkable(orc):
    """Rows never read later columns, and a prompt split into two chunks (the
    second with prefix = first chunk) gives the same rows bit for bit."""
    rng = np.random.default_rng(12)
    T, stride = 40, 128
    q, kc, vc = _attn_inputs(rng, T, 0, stride)
    full = orc.attn_prefill(q, kc, vc, T, 0, stride)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, 25:] = random_bf16(rng, kc2[:, 25:].shape, std=5.0)
    vc2[:, :, 25:] = random_bf16(rng, vc2[:, :, 25:].shape, std=5.0)
    np.testing.assert_array_equal(orc.attn_prefill(q[:25], kc2, vc2, 25, 0, stride), full[:25])
    tail = orc.attn_prefill(q[25:], kc, vc, T - 25, 25, stride)
    np.testing.assert_array_equal(tail, full[25:])


def test_attn_prefill_single_token_matches_decode(orc):
    """T = 1 with a prefix is one decode step. The decode restatement keeps
    scores and probabilities in f32 and applies the gate before rounding; the
    prefill rounds scores (|s| ~ 16-50, so up to 2^-9*|s|/16 of a logit) and
    probabilities to bf16. They agree to ~1% (gate +88 gives sigmoid = 1.0f)."""
    rng = np.random.default_rng(13)
    stride, L = 256, 200
    q, kc, vc = _attn_inputs(rng, 1, L - 1, stride)
    pre = orc.attn_prefill(q, kc, vc, 1, L - 1, stride)[0]
    gate = np.full(16 * 256, f32_to_bf16(np.float32(88.0)), np.uint16)
    dec = orc.attn_decode(q[0], kc, vc, gate, stride, L)
    err = F(pre) - F(dec)
    assert np.linalg.norm(err) <= 2e-2 * np.linalg.norm(F(dec))


# --------------------------------------------------- A24 GDN prefill -----
@pytest.mark.parametrize("T,has_prev", [(1, True), (2, True), (3, False), (9, True), (9, False)])
def test_conv1d_prefill_equals_decode_steps(orc, T, has_prev):
    rng = np.random.default_rng(T + 10 * has_prev)
    C = 256
    state = f32_to_bf16(rng.normal(size=(3, C)).astype(np.float32))
    state = bf16_to_f32(state).astype(np.float32)
    w = random_bf16(rng, (C, 4), std=0.5)
    x = random_bf16(rng, (T, C), std=2.0)
    out, st = orc.conv1d_prefill(state, x, w, has_prev)
    s = state.copy() if has_prev else np.zeros_like(state)
    for t in range(T):
        o, s = orc.conv1d_decode(s, x[t], w)
        np.testing.assert_array_equal(out[t], o)
    np.testing.assert_array_equal(st, s)


def test_qk_l2norm_prefill_vs_float64(orc):
    rng = np.random.default_rng(14)
    T = 3
    co = random_bf16(rng, (T, 8192), std=2.0)
    qn, kn = orc.qk_l2norm_prefill(co)
    c = F(co)
    for t in range(T):
        for h in range(16):
            qv = c[t, h * 128:(h + 1) * 128]
            kv = c[t, 2048 + h * 128:2048 + (h + 1) * 128]
            np.testing.assert_allclose(qn[t, h * 128:(h + 1) * 128], qv / np.sqrt(qv @ qv + 1e-6) / np.sqrt(128), rtol=2e-6)
            np.testing.assert_allclose(kn[t, h * 128:(h + 1) * 128], kv / np.sqrt(kv @ kv + 1e-6), rtol=2e-6)


def test_gating_many_vs_float64(orc):
    rng = np.random.default_rng(15)
    T = 4
    A_log = rng.uniform(-5, -2, 32).astype(np.float32)
    a = random_bf16(rng, (T, 32), std=3.0)
    b = random_bf16(rng, (T, 32), std=3.0)
    dtb = random_bf16(rng, (32,), std=1.0)
    g, beta = orc.gating_many(A_log, a, dtb, b)
    x = F(a) + F(dtb)[None, :]
    sp = np.log1p(np.exp(x))
    np.testing.assert_allclose(g, np.exp(-np.exp(A_log.astype(np.float64))[None, :] * sp), rtol=1e-5)
    np.testing.assert_allclose(beta, 1 / (1 + np.exp(-F(b))), rtol=1e-6)


def _gdn_inputs(rng, T):
    co = random_bf16(rng, (T, 8192), std=1.5)
    a = random_bf16(rng, (T, 32), std=1.0)
    b = random_bf16(rng, (T, 32), std=1.0)
    A_log = rng.uniform(-4, -1, 32).astype(np.float32)
    dtb = random_bf16(rng, (32,), std=0.5)
    state = (rng.normal(size=(32, 128, 128)) * 0.1).astype(np.float32)
    return co, a, b, A_log, dtb, state


@pytest.mark.parametrize("has_prev", [True, False])
def test_gdn_prefill_tracks_decode_steps(orc, has_prev):
    """T prefill steps vs T decode steps of the (separately pinned) decode
    restatement. They differ only in how the q/k norms are summed (128-thread
    tree vs 32 lanes x 4 chunks), i.e. in the last f32 bits."""
    rng = np.random.default_rng(16 + has_prev)
    T = 6
    co, a, b, A_log, dtb, state = _gdn_inputs(rng, T)
    qn, kn = orc.qk_l2norm_prefill(co)
    g, beta = orc.gating_many(A_log, a, dtb, b)
    y, st = orc.gated_delta_prefill(state, qn, kn, co, g, beta, has_prev)
    s = state.copy()
    for t in range(T):
        yd, s = orc.gated_delta_decode(s, co[t], a[t], b[t], A_log, dtb, has_prev=(has_prev or t > 0))
        r = F(yd)
        assert np.all(np.abs(F(y[t]) - r) <= 2.0 ** -7 * np.abs(r) + 1e-3 * np.sqrt(np.mean(r * r)))
        assert np.mean(y[t] == yd) >= 0.99
    np.testing.assert_allclose(st, s, rtol=1e-4, atol=1e-6)


def test_gdn_prefill_vs_float64_delta_rule(orc):
    rng = np.random.default_rng(18)
    T = 4
    co, a, b, A_log, dtb, state = _gdn_inputs(rng, T)
    qn, kn = orc.qk_l2norm_prefill(co)
    g, beta = orc.gating_many(A_log, a, dtb, b)
    y, st = orc.gated_delta_prefill(state, qn, kn, co, g, beta, True)
    S = state.astype(np.float64)
    v = F(co)[:, 4096:].reshape(T, 32, 128)
    for t in range(T):
        for hv in range(32):
            hk = hv // 2
            q = qn[t, hk * 128:(hk + 1) * 128].astype(np.float64)
            k = kn[t, hk * 128:(hk + 1) * 128].astype(np.float64)
            d = S[hv] * g[t, hv]
            delta = (v[t, hv] - d @ k) * beta[t, hv]
            S[hv] = d + np.outer(delta, k)
            ref = S[hv] @ q
            got = F(y[t, hv * 128:(hv + 1) * 128])
            assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-3 * np.sqrt(np.mean(ref * ref)))
    np.testing.assert_allclose(st, S, rtol=1e-4, atol=1e-6)
