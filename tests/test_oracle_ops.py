"""Pin the oracle's norm / embedding / conv1d / Gated DeltaNet / attention
restatements (reference shaders/rmsnorm.metal, embedding.metal, conv1d.metal,
gated_delta.metal, gated_norm.metal, attention.metal, attention_decode.metal)
with float64 references, closed forms, limiting cases and identities. CPU only.
"""
import numpy as np
import pytest

from peregrine_amd.synth import bf16_to_f32, f32_to_bf16, random_bf16, random_q4

F = lambda b: bf16_to_f32(b).astype(np.float64)  # noqa: E731


def ulps(a_bits, b_bits):
    return np.abs(a_bits.astype(np.int64) - b_bits.astype(np.int64))


# ----------------------------------------------------------------- norms ---
def test_rmsnorm_vs_float64(orc):
    rng = np.random.default_rng(0)
    x = random_bf16(rng, (3, 4096), std=2.0)
    w = random_bf16(rng, (4096,), std=0.1, mean=1.0)
    got = orc.rmsnorm(x, w)
    xf = F(x)
    ref = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-6) * F(w)
    assert ulps(got, f32_to_bf16(ref.astype(np.float32))).max() <= 1


def test_add_rmsnorm_rounds_residual_first(orc):
    rng = np.random.default_rng(1)
    a = random_bf16(rng, (2, 1024), std=3.0)
    b = random_bf16(rng, (2, 1024), std=3.0)
    w = random_bf16(rng, (1024,), std=0.1, mean=1.0)
    r, n = orc.add_rmsnorm(a, b, w)
    np.testing.assert_array_equal(r, f32_to_bf16(bf16_to_f32(a) + bf16_to_f32(b)))
    np.testing.assert_array_equal(n, orc.rmsnorm(r, w))


def test_embedding_is_dequantised_row(orc):
    rng = np.random.default_rng(2)
    wt = random_q4(rng, 300, 1024)
    deq = orc.q4_dequantize(wt)
    for tok in [0, 1, 157, 299]:
        np.testing.assert_array_equal(orc.embedding(wt, tok), deq[tok])


# ---------------------------------------------------------------- conv1d ---
def test_conv1d_one_hot_taps_and_roll(orc):
    rng = np.random.default_rng(3)
    C = 64
    state = rng.normal(size=(3, C)).astype(np.float32)
    x = random_bf16(rng, (C,))
    for j in range(4):  # weight = e_j: output = silu(tap j)
        w = np.zeros((C, 4), np.float32)
        w[:, j] = 1.0
        out, st = orc.conv1d_decode(state, x, f32_to_bf16(w))
        tap = state[j] if j < 3 else bf16_to_f32(x)
        silu = tap / (1.0 + np.exp(-tap.astype(np.float64)))
        assert ulps(out, f32_to_bf16(silu.astype(np.float32))).max() <= 1
        np.testing.assert_array_equal(st[0], state[1])
        np.testing.assert_array_equal(st[1], state[2])
        np.testing.assert_array_equal(st[2], bf16_to_f32(x))
    # three steps from zero state: state == the three inputs, oldest first
    st = np.zeros((3, C), np.float32)
    xs = [random_bf16(rng, (C,)) for _ in range(3)]
    w = random_bf16(rng, (C, 4), std=0.5)
    for xi in xs:
        _, st = orc.conv1d_decode(st, xi, w)
    for i in range(3):
        np.testing.assert_array_equal(st[i], bf16_to_f32(xs[i]))


# ------------------------------------------------------------------- GDN ---
def _gdn_inputs(rng, has_state=True):
    conv = random_bf16(rng, (8192,))
    a = random_bf16(rng, (32,))
    b = random_bf16(rng, (32,))
    A_log = np.zeros(32, np.float32)
    dt = np.zeros(32, np.uint16)
    S = rng.normal(0, 0.1, size=(32, 128, 128)).astype(np.float32)
    return conv, a, b, A_log, dt, S


def _qk(conv, hv):
    hk = hv // 2
    q = F(conv[hk * 128:(hk + 1) * 128])
    k = F(conv[2048 + hk * 128:2048 + (hk + 1) * 128])
    qn = q / np.sqrt(np.sum(q * q) + 1e-6) / np.sqrt(128.0)
    kn = k / np.sqrt(np.sum(k * k) + 1e-6)
    return qn, kn


def test_gdn_vs_float64_delta_rule(orc):
    rng = np.random.default_rng(4)
    conv, a, b, A_log, dt, S = _gdn_inputs(rng)
    y, S1 = orc.gated_delta_decode(S, conv, a, b, A_log, dt)
    for hv in [0, 1, 17, 31]:
        qn, kn = _qk(conv, hv)
        x = F(a[hv])
        decay = np.exp(-np.exp(0.0) * np.log1p(np.exp(x)))
        beta = 1.0 / (1.0 + np.exp(-F(b[hv])))
        d = S[hv].astype(np.float64) * decay
        v = F(conv[4096 + hv * 128:4096 + (hv + 1) * 128])
        delta = (v - d @ kn) * beta
        Snew = d + np.outer(delta, kn)
        yref = Snew @ qn
        np.testing.assert_allclose(S1[hv], Snew, rtol=1e-4, atol=1e-6)
        assert ulps(y[hv * 128:(hv + 1) * 128], f32_to_bf16(yref.astype(np.float32))).max() <= 1


def test_gdn_beta_zero_is_pure_decay(orc):
    rng = np.random.default_rng(5)
    conv, a, b, A_log, dt, S = _gdn_inputs(rng)
    b = f32_to_bf16(np.full(32, -200.0, np.float32))  # sigmoid -> exactly 0
    _, S1 = orc.gated_delta_decode(S, conv, a, b, A_log, dt)
    x = bf16_to_f32(a)
    sp = np.maximum(x, 0) + np.log1p(np.exp(-np.abs(x)))
    decay = np.exp(-sp.astype(np.float32)).astype(np.float32)
    np.testing.assert_allclose(S1, S * decay[:, None, None], rtol=2e-6)


def test_gdn_exact_recall_and_identity(orc):
    """decay = 1 (A_log = -inf), beta = 1, zero state, q = k: the step writes
    v along k, and y = ob + delta*(k.q) equals S_new.q."""
    rng = np.random.default_rng(6)
    conv, a, b, _, dt, S = _gdn_inputs(rng)
    conv[:2048] = conv[2048:4096]  # q_raw == k_raw
    A_log = np.full(32, -np.inf, np.float32)
    b = f32_to_bf16(np.full(32, 200.0, np.float32))
    y, S1 = orc.gated_delta_decode(S, conv, a, b, A_log, dt, has_prev=False)
    for hv in [0, 9, 30]:
        qn, kn = _qk(conv, hv)
        v = F(conv[4096 + hv * 128:4096 + (hv + 1) * 128])
        np.testing.assert_allclose(S1[hv] @ kn, v * (kn @ kn), rtol=1e-4, atol=1e-5)  # recall
        np.testing.assert_allclose(F(y[hv * 128:(hv + 1) * 128]), S1[hv].astype(np.float64) @ qn,
                                   rtol=1e-2, atol=1e-3)
    # has_previous_state = 0 ignores the incoming state entirely
    y2, S2 = orc.gated_delta_decode(S * 7 + 1, conv, a, b, A_log, dt, has_prev=False)
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(S1, S2)


def test_gated_rmsnorm_vs_float64(orc):
    rng = np.random.default_rng(7)
    x = random_bf16(rng, (32 * 128,))
    w = random_bf16(rng, (128,), std=0.1, mean=1.0)
    z = random_bf16(rng, (32 * 128,))
    got = orc.rmsnorm_gated(x, w, z, 128)
    xf, zf = F(x).reshape(32, 128), F(z).reshape(32, 128)
    ref = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-6) * F(w) * (zf / (1 + np.exp(-zf)))
    assert ulps(got, f32_to_bf16(ref.ravel().astype(np.float32))).max() <= 1


# ------------------------------------------------------------- attention ---
def _prep_inputs(rng, stride=256):
    pq = random_bf16(rng, (16 * 512,))
    qw = random_bf16(rng, (256,), std=0.1, mean=1.0)
    kin = random_bf16(rng, (4 * 256,))
    vin = random_bf16(rng, (4 * 256,))
    kw = random_bf16(rng, (256,), std=0.1, mean=1.0)
    kc = np.zeros((4, stride, 256), np.uint16)
    vc = np.zeros((4, 256, stride), np.uint16)
    return pq, qw, kin, vin, kw, kc, vc


def test_attn_prepare_pos0_identity_and_layout(orc):
    rng = np.random.default_rng(8)
    pq, qw, kin, vin, kw, kc, vc = _prep_inputs(rng)
    q, gate, kc1, vc1 = orc.attn_prepare(pq, qw, kin, vin, kw, kc, vc, 256, dst=37, pos=0)
    pq2 = pq.reshape(16, 2, 256)
    np.testing.assert_array_equal(gate.reshape(16, 256), pq2[:, 1])
    np.testing.assert_array_equal(vc1[:, :, 37], vin.reshape(4, 256))  # V value-dim-major
    assert not vc1[:, :, 36].any() and not kc1[:, 36].any()
    # position 0: RoPE is the identity -> plain RMSNorm of q and k
    np.testing.assert_array_equal(q.reshape(16, 256), orc.rmsnorm(pq2[:, 0], qw))
    np.testing.assert_array_equal(kc1[:, 37], orc.rmsnorm(kin.reshape(4, 256), kw))


def test_attn_prepare_rope_rotation(orc):
    rng = np.random.default_rng(9)
    pq, qw, kin, vin, kw, kc, vc = _prep_inputs(rng)
    pos = 1234
    q, _, kc1, _ = orc.attn_prepare(pq, qw, kin, vin, kw, kc, vc, 256, dst=0, pos=pos)
    normed = F(orc.rmsnorm(pq.reshape(16, 2, 256)[:, 0], qw))
    i = np.arange(32)
    inv_freq = (1.0e7 ** (-(2.0 * i) / 64.0)).astype(np.float32)
    ang = (np.float32(pos) * inv_freq).astype(np.float64)
    x1, x2 = normed[:, :32], normed[:, 32:64]
    r1 = x1 * np.cos(ang) - x2 * np.sin(ang)
    r2 = x2 * np.cos(ang) + x1 * np.sin(ang)
    qq = F(q).reshape(16, 256)
    np.testing.assert_allclose(qq[:, :32], r1, rtol=1e-2, atol=2e-2)
    np.testing.assert_allclose(qq[:, 32:64], r2, rtol=1e-2, atol=2e-2)
    np.testing.assert_array_equal(q.reshape(16, 256)[:, 64:], f32_to_bf16(normed[:, 64:].astype(np.float32)))
    # rotation preserves the pair norms
    np.testing.assert_allclose(np.hypot(qq[:, :32], qq[:, 32:64]), np.hypot(x1, x2), rtol=2e-2, atol=2e-2)


def _attn_f64(q, kc, vc, gate, L):
    qf = F(q).reshape(16, 256)
    out = np.empty((16, 256))
    for h in range(16):
        kvh = h // 4
        K = F(kc[kvh, :L])
        V = F(vc[kvh, :, :L]).T
        s = K @ qf[h] / 16.0
        p = np.exp(s - s.max())
        out[h] = (p @ V) / p.sum()
    g = F(gate).reshape(16, 256)
    return out * (1 / (1 + np.exp(-g)))


@pytest.mark.parametrize("L", [1, 63, 1024, 1025, 3000])
def test_attn_decode_vs_float64(orc, L):
    rng = np.random.default_rng(10 + L)
    stride = ((L + 255) // 256) * 256
    q = random_bf16(rng, (16 * 256,))
    kc = random_bf16(rng, (4, stride, 256))
    vc = random_bf16(rng, (4, 256, stride))
    gate = random_bf16(rng, (16 * 256,))
    got = F(orc.attn_decode(q, kc, vc, gate, stride, L)).reshape(16, 256)
    ref = _attn_f64(q, kc, vc, gate, L)
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2 * np.sqrt(np.mean(ref * ref)) + 1e-6)
    if L == 1:  # one token: softmax weight 1 -> v * sigmoid(gate)
        v0 = F(vc[:, :, 0])
        np.testing.assert_allclose(got, np.repeat(v0, 4, axis=0) / (1 + np.exp(-F(gate).reshape(16, 256))),
                                   rtol=1e-2, atol=1e-3)


def test_decisive_margin_rule():
    """The greedy-parity guard: four bf16 ulps of the top logit (ulp of a
    value in [2^e, 2^(e+1)) is 2^(e-7)). Top 8.0 (ulp 1/16, guard 0.25) beside
    7.875 is a near-tie, beside 7.5 decisive; the runner-up is the second
    largest even when it precedes the winner; negative tops use |top|."""
    from oracle.model import decisive_margin

    lg = np.zeros(10)
    lg[3], lg[7] = 8.0, 7.875
    assert decisive_margin(lg) == (3, 7, 0.125, 0.25)
    lg[7] = 7.5
    i1, i2, m, g = decisive_margin(lg)
    assert (i1, i2, m, g) == (3, 7, 0.5, 0.25) and m > g
    lg = np.full(6, -20.0)
    lg[4], lg[1] = -3.0, -3.25  # |top| in [2, 4): ulp 1/64, guard 1/16
    assert decisive_margin(lg) == (4, 1, 0.25, 0.0625)
