"""Pin the C oracle's Q4 GEMV family (reference shaders/linear*.metal,
shaders/argmax.metal) against independent checks: brute-force unpacking,
float64 dense GEMV, closed forms and algebraic invariants. CPU only.

The reference holds no numeric golden vectors for this path (its tests pin
dispatch geometry only, src/model/linear_q4.zig:304-316); these checks are
chosen so that a dropped term, a wrong nibble/group index or a transposed
operand fails at least one of them.
"""
import numpy as np
import pytest

from peregrine_amd.synth import (Q4Weight, bf16_to_f32, f32_to_bf16, pack_q4, random_bf16,
                                 random_q4, unpack_q4)


def test_bf16_rounding_matches_numpy(orc):
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.normal(0, 1, 5000), rng.normal(0, 1e-30, 100), [0.0, -0.0, 1.0, np.inf, -np.inf],
                        # exact ties: 1 + 2^-8 (tie to even -> 1), 1 + 3*2^-8 (tie -> up)
                        [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, -(1.0 + 2.0**-8)]]).astype(np.float32)
    ref = f32_to_bf16(v)
    assert bf16_to_f32(ref[-3]) == 1.0 and bf16_to_f32(ref[-2]) == 1.0 + 2.0**-6
    np.testing.assert_array_equal(orc.f2bf(v), ref)


def test_pack_unpack_bruteforce():
    rng = np.random.default_rng(2)
    q = rng.integers(0, 16, size=(5, 128), dtype=np.uint8)
    w = pack_q4(q)
    # brute force: nibble j of word c is column 8c + j
    for n in range(5):
        for k in range(128):
            assert (int(w[n, k // 8]) >> (4 * (k % 8))) & 0xF == q[n, k]
    np.testing.assert_array_equal(unpack_q4(w), q)


def test_dequantize_exact(orc):
    rng = np.random.default_rng(3)
    wt = random_q4(rng, 16, 256)
    got = orc.q4_dequantize(wt)
    q = unpack_q4(wt.w).astype(np.float32)
    s = np.repeat(bf16_to_f32(wt.s), 64, axis=1)
    b = np.repeat(bf16_to_f32(wt.b), 64, axis=1)
    # s*q is exact in f32 (8-bit x 4-bit mantissas), so one rounding total.
    np.testing.assert_array_equal(got, f32_to_bf16((s * q).astype(np.float32) + b))


@pytest.mark.parametrize("N,K", [(64, 512), (48, 2048), (16, 4096)])
def test_gemv_vs_float64(orc, N, K):
    rng = np.random.default_rng(N * K)
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (1, K))
    dots = orc.q4_dots(x, wt)[0].astype(np.float64)
    exact = bf16_to_f32(x[0]).astype(np.float64) @ wt.dequant_f64().T
    mag = np.abs(bf16_to_f32(x[0]).astype(np.float64)) @ np.abs(wt.dequant_f64()).T
    # fp32 accumulation error bound: a few ulps of the magnitude sum
    assert np.all(np.abs(dots - exact) <= 1e-5 * mag + 1e-30)
    y = bf16_to_f32(orc.q4_gemv(x, wt)[0]).astype(np.float64)
    assert np.all(np.abs(y - exact) <= 1e-2 * np.abs(exact) + 1e-5 * mag)


def test_gemv_one_hot_indexing(orc):
    """x = e_k picks column k: y[n] = bf16(s[n,k/64]*q[n,k] + b[n,k/64]) exactly.
    A wrong nibble order or group index changes the answer."""
    rng = np.random.default_rng(4)
    N, K = 24, 1024
    wt = random_q4(rng, N, K)
    deq = orc.q4_dequantize(wt)
    for k in [0, 1, 7, 8, 63, 64, 65, 511, 512, 1000, 1023]:
        x = np.zeros((1, K), np.uint16)
        x[0, k] = f32_to_bf16(np.float32(1.0))
        np.testing.assert_array_equal(orc.q4_gemv(x, wt)[0], deq[:, k], err_msg=f"k={k}")


def test_gemv_zero_q_and_zero_scale(orc):
    rng = np.random.default_rng(5)
    N, K = 16, 1024
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (1, K))
    xf = bf16_to_f32(x[0]).astype(np.float64)
    gsum = xf.reshape(K // 64, 64).sum(axis=1)
    # q == 0 -> y = sum_g b_g * sum(x_g)
    zq = Q4Weight(np.zeros_like(wt.w), wt.s, wt.b)
    ref = bf16_to_f32(wt.b).astype(np.float64) @ gsum
    got = orc.q4_dots(x, zq)[0]
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # s == 0 -> bias only, independent of q
    zs = Q4Weight(wt.w, np.zeros_like(wt.s), wt.b)
    np.testing.assert_allclose(orc.q4_dots(x, zs)[0], ref, rtol=1e-5, atol=1e-5)


def test_m2_equals_two_m1(orc):
    rng = np.random.default_rng(6)
    wt = random_q4(rng, 32, 2048)
    x = random_bf16(rng, (2, 2048))
    both = orc.q4_gemv(x, wt)
    np.testing.assert_array_equal(both[0], orc.q4_gemv(x[:1], wt)[0])
    np.testing.assert_array_equal(both[1], orc.q4_gemv(x[1:], wt)[0])


def test_residual_add_is_gemv_then_add(orc):
    rng = np.random.default_rng(7)
    wt = random_q4(rng, 40, 1536)
    x = random_bf16(rng, (2, 1536))
    res = random_bf16(rng, (2, 40), std=4.0)
    got = orc.q4_gemv_residual_add(x, wt, res)
    y = bf16_to_f32(orc.q4_gemv(x, wt))
    np.testing.assert_array_equal(got, f32_to_bf16(y + bf16_to_f32(res)))


def test_silu_gate_is_two_gemvs(orc):
    rng = np.random.default_rng(8)
    g = random_q4(rng, 48, 1024)
    u = random_q4(rng, 48, 1024)
    x = random_bf16(rng, (2, 1024))
    got = orc.q4_gemv_silu_gate(x, g, u)
    gv = bf16_to_f32(orc.q4_gemv(x, g)).astype(np.float32)
    uv = bf16_to_f32(orc.q4_gemv(x, u)).astype(np.float32)
    silu = gv / (np.float32(1.0) + np.exp(-gv))
    ref = f32_to_bf16((silu * uv).astype(np.float32))
    # exp may differ by an ulp between libm and numpy: allow 1 bf16 ulp
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99


def test_argmax_partial_first_strict_max(orc):
    """Rows with equal bf16 logits: the partial keeps the lowest row."""
    N, K = 64, 512
    q = np.zeros((N, K), np.uint8)
    q[:, 0] = 5
    q[10, 0] = 9
    q[13, 0] = 9   # tie with row 10 inside partial 1 -> row 10
    q[40, 0] = 9   # tie in partial 5 -> row 40
    wt = Q4Weight(pack_q4(q), f32_to_bf16(np.full((N, K // 64), 0.25, np.float32)),
                  np.zeros((N, K // 64), np.uint16))
    x = np.zeros((1, K), np.uint16)
    x[0, 0] = f32_to_bf16(np.float32(1.0))
    pv, pi = orc.q4_argmax_partial(x, wt)
    assert pi[0, 1] == 10 and pv[0, 1] == 2.25
    assert pi[0, 5] == 40
    assert pi[0, 0] == 0 and pv[0, 0] == 1.25
    assert orc.argmax_pairs(pv[0], pi[0]) == 10


def _bitrev8(t: int) -> int:
    return int(f"{t:08b}"[::-1], 2)


def _closed_form_pairs(values, indices):
    """Reference tie order for argmax_pairs (shaders/argmax.metal:6-43).

    Thread t scans p = t, t+256, ... keeping the first strict max, so within a
    thread the smallest p div 256 wins. The tree then compares (tid, tid+stride)
    for stride 128..1 and keeps the lower position on ties: the last level
    prefers even threads over odd, the one before prefers t = 0 mod 4 over
    2 mod 4, and so on. Among equal maxima the winner minimises
    (bitreverse8(p mod 256), p div 256). NaN and -inf never win; if nothing
    beats -inf the result is 0."""
    v = np.asarray(values, np.float64)
    ok = np.isfinite(v) | (v == np.inf)
    ok &= v > -np.inf
    if not ok.any():
        return 0
    m = v[ok].max()
    cand = [p for p in range(len(v)) if ok[p] and v[p] == m]
    best = min(cand, key=lambda p: (_bitrev8(p % 256), p // 256))
    return int(indices[best])


@pytest.mark.parametrize("seed", range(6))
def test_argmax_pairs_tie_order(orc, seed):
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(1, 2000))
    vals = rng.integers(-3, 4, size=n).astype(np.float32)  # many ties
    if seed == 3:
        vals[rng.integers(0, n, size=5)] = np.nan
    if seed == 4:
        vals[:] = -np.inf
    idx = rng.permutation(10 * n)[:n].astype(np.uint32)
    assert orc.argmax_pairs(vals, idx) == _closed_form_pairs(vals, idx)


def test_argmax_tie_order_is_not_lowest_index(orc):
    """Ties between partials 1 and 2: bitrev8(1) = 128 > bitrev8(2) = 64, so
    partial 2 wins although partial 1 comes first."""
    vals = np.zeros(600, np.float32)
    vals[1] = 5.0
    vals[2] = 5.0
    idx = np.arange(600, dtype=np.uint32)
    assert orc.argmax_pairs(vals, idx) == 2
    vals[258] = 5.0  # same thread as 2 (258 mod 256), later in its scan -> 2 still wins
    assert orc.argmax_pairs(vals, idx) == 2
    vals[0] = 5.0    # thread 0 has the smallest bit-reversed id
    assert orc.argmax_pairs(vals, idx) == 0


def test_partial_count_matches_reference():
    # argmax.zig:9-12: vocab / 8 partials
    assert 248320 // 8 == 31040
