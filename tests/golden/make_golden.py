#!/usr/bin/env python3
"""Writes tests/golden/golden_v1.npz: small known-answer vectors for the
decode path, each computed here by a method independent of the C oracle.

    python tests/golden/make_golden.py

The reference repository holds no numeric fixtures for this path (its tests
pin dispatch geometry only), so these vectors come from the mathematics:

* gemv_*   BASELINE config 1's generator (seed 0, x ~ N(0,1), q ~ U{0..15},
           s ~ U(0.001, 0.02), b ~ N(0, 0.05) per 64-group) at 64 x 1024:
           the dense product in float64 over w = s*q + b
           (shaders/linear.metal:12-19), and its round-to-nearest-even bf16.
* argmax_* 31040 lm_head partials (248320 rows / 8) drawn from five values
           plus NaN and -inf, so most of the maximum is tied; the winner comes
           from a step-by-step simulation of argmax_pairs_f32_u32's 256 threads
           and halving tree (shaders/argmax.metal:6-43) in plain Python.
* gdn_*    one Gated DeltaNet decode step (shaders/gated_delta.metal:147-261)
           in float64 as the textbook delta rule S' = decay*S + beta*(v -
           decay*S k) k^T, y = S' q, with the gates of the same kernel.
* attn_*   GQA decode attention (shaders/attention_decode.metal:24-243) at
           L = 64 in float64: softmax(q K^T / 16) V, times sigmoid(gate).

Nothing here imports or runs reference code. Inputs are stored with the
expected outputs, so the tests do not depend on numpy's random streams.
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from peregrine_amd.synth import bf16_to_f32, f32_to_bf16, random_bf16, random_q4  # noqa: E402

OUT = HERE / "golden_v1.npz"


def bf16_rne_from_f64(v: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits with one rounding (RNE on the exact value)."""
    v = np.asarray(v, np.float64)
    out = np.empty(v.shape, np.uint16)
    flat, res = v.ravel(), out.ravel()
    for i, x in enumerate(flat):
        lo = f32_to_bf16(np.float32(x))  # candidate near x
        cands = [int(lo), (int(lo) + 1) & 0xFFFF, (int(lo) - 1) & 0xFFFF]
        vals = [float(bf16_to_f32(np.uint16(c))) for c in cands]
        best = min(range(3), key=lambda j: (abs(vals[j] - x), cands[j] & 1))
        res[i] = cands[best]
    return out


def gemv_case(rng):
    N, K = 64, 1024
    wt = random_q4(rng, N, K)
    x = random_bf16(rng, (K,))
    y64 = wt.dequant_f64() @ bf16_to_f32(x).astype(np.float64)
    return {"gemv_x": x, "gemv_w": wt.w, "gemv_s": wt.s, "gemv_b": wt.b, "gemv_y_f64": y64,
            "gemv_y_bf16": bf16_rne_from_f64(y64)}


def argmax_sim(values: np.ndarray, indices: np.ndarray) -> int:
    """Thread t of 256 keeps the first strict maximum of p = t, t+256, ...;
    then for stride 128, 64, ..., 1 thread t < stride takes t+stride's pair
    when its value is strictly greater. NaN never compares greater."""
    T = 256
    bv = [-math.inf] * T
    bi = [0] * T
    for t in range(T):
        for p in range(t, len(values), T):
            v = float(values[p])
            if v > bv[t]:
                bv[t], bi[t] = v, int(indices[p])
    stride = T // 2
    while stride > 0:
        for t in range(stride):
            if bv[t + stride] > bv[t]:
                bv[t], bi[t] = bv[t + stride], bi[t + stride]
        stride //= 2
    return bi[0]


def argmax_case(rng):
    P = 248320 // 8
    pool = np.array([0.5, 1.25, 2.0, 3.0, 3.0], np.float32)  # 3.0 is the max, drawn most often
    vals = pool[rng.integers(0, len(pool), P)]
    vals[rng.integers(0, P, 50)] = np.nan
    vals[rng.integers(0, P, 50)] = -np.inf
    idx = (np.arange(P, dtype=np.uint32) * 8 + rng.integers(0, 8, P).astype(np.uint32)).astype(np.uint32)
    return {"argmax_values": vals, "argmax_indices": idx,
            "argmax_winner": np.array([argmax_sim(vals, idx)], np.uint32)}


GDN_SAMPLE = 61  # every 61st element of the new state is stored


def gdn_state() -> np.ndarray:
    """The 2 MiB f32 recurrent state is not stored: it is this closed form
    (|S| <= 0.1, no two heads or rows alike), rebuilt by the tests."""
    h, i, j = np.meshgrid(np.arange(32.0), np.arange(128.0), np.arange(128.0), indexing="ij")
    return (0.1 * np.sin(1.3 * h + 0.37 * i + 0.011 * j * (1.0 + 0.05 * h))).astype(np.float32)


def gdn_case(rng):
    Hk, Hv, D = 16, 32, 128
    conv = random_bf16(rng, (2 * Hk * D + Hv * D,))
    a = random_bf16(rng, (Hv,))
    b = random_bf16(rng, (Hv,))
    A_log = rng.normal(0, 0.5, Hv).astype(np.float32)
    dt = random_bf16(rng, (Hv,), std=0.5)
    S = gdn_state()  # [hv, dv, dk]
    c = bf16_to_f32(conv).astype(np.float64)
    q = c[:Hk * D].reshape(Hk, D)
    k = c[Hk * D:2 * Hk * D].reshape(Hk, D)
    v = c[2 * Hk * D:].reshape(Hv, D)
    q = q / np.sqrt((q * q).sum(1, keepdims=True) + 1e-6) / math.sqrt(D)
    k = k / np.sqrt((k * k).sum(1, keepdims=True) + 1e-6)
    x = bf16_to_f32(a).astype(np.float64) + bf16_to_f32(dt).astype(np.float64)
    softplus = np.maximum(x, 0) + np.log1p(np.exp(-np.abs(x)))
    decay = np.exp(-np.exp(A_log.astype(np.float64)) * softplus)
    beta = 1.0 / (1.0 + np.exp(-bf16_to_f32(b).astype(np.float64)))
    S64 = S.astype(np.float64)
    Snew = np.empty_like(S64)
    y = np.empty((Hv, D))
    for h in range(Hv):
        kk, qq = k[h // 2], q[h // 2]
        Sd = decay[h] * S64[h]
        delta = beta[h] * (v[h] - Sd @ kk)
        Snew[h] = Sd + np.outer(delta, kk)
        y[h] = Snew[h] @ qq
    return {"gdn_conv": conv, "gdn_a": a, "gdn_b": b, "gdn_A_log": A_log, "gdn_dt_bias": dt,
            "gdn_y_f64": y.reshape(-1), "gdn_S_new_sample_f64": Snew.reshape(-1)[::GDN_SAMPLE]}


def attn_case(rng):
    L, Hq, Hkv, D = 64, 16, 4, 256
    q = random_bf16(rng, (Hq * D,))
    kc = random_bf16(rng, (Hkv, L, D))
    vc = random_bf16(rng, (Hkv, D, L))
    gate = random_bf16(rng, (Hq * D,))
    qf = bf16_to_f32(q).astype(np.float64).reshape(Hq, D)
    kf = bf16_to_f32(kc).astype(np.float64)
    vf = bf16_to_f32(vc).astype(np.float64)
    gf = bf16_to_f32(gate).astype(np.float64).reshape(Hq, D)
    out = np.empty((Hq, D))
    for h in range(Hq):
        s = kf[h // 4] @ qf[h] / 16.0
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = (vf[h // 4] @ p) / (1.0 + np.exp(-gf[h]))
    return {"attn_q": q, "attn_k": kc, "attn_v": vc, "attn_gate": gate, "attn_out_f64": out.reshape(-1)}


def main() -> None:
    rng = np.random.default_rng(0)
    data = {}
    data.update(gemv_case(rng))
    data.update(argmax_case(np.random.default_rng(1)))
    data.update(gdn_case(np.random.default_rng(2)))
    data.update(attn_case(np.random.default_rng(3)))
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
