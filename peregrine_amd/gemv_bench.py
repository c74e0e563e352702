"""Q4 GEMV sweep on one GPU with MALL-defeating rotation,
on the decode layout the model runs and on the MLX layout beside it.

Each shape is timed over a ring of distinct weight copies totalling >= 512 MiB
(MI355X's Infinity Cache is 256 MiB), so every launch streams its weights from
HBM. One launch per ring copy is captured into a HIP graph and the graph is
replayed; the per-launch time is the median over replays (each bracketed by
HIP events on the graph's stream) divided by the ring length, so no host
launch overhead enters, as in the decode loop. Reported with the algorithmic
bytes (weights + scales + biases + x + outputs) and GB/s.
"""
from __future__ import annotations

import numpy as np

from .device import DeviceArray, Stream, synchronize
from .op_bench import time_graph
from .ops import DecodeLayoutQ4, Q4Linear, argmax_pairs, gate_up_silu, t16_argmax_workspace_bytes
from .synth import random_bf16, random_q4

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 512 * 1024 * 1024


def q4_bytes(N: int, K: int) -> int:
    return N * K // 2 + N * K // 16  # nibbles + bf16 scale + bf16 bias


def _ring(rng, N: int, K: int, **kw) -> list[Q4Linear]:
    one = random_q4(rng, N, K, **kw)
    copies = max(2, -(-ROTATE_BYTES // one.nbytes))
    ring = [Q4Linear.upload(one)]
    for _ in range(copies - 1):
        # distinct allocations holding the same bits: the cache cannot tell
        ring.append(Q4Linear.upload(one))
    return ring


def time_launches(fn, ring, reps: int = 10) -> float:
    """Milliseconds per launch of fn(item, stream) over the rotated ring, from
    graph replays (at least 50 launches in total)."""
    st = Stream()
    reps = max(reps, -(-50 // len(ring)))
    ms = time_graph(st, lambda: [fn(item, st.handle) for item in ring], reps) / len(ring)
    st.close()
    return ms


def sweep(shapes=None, Ms=(1, 2), seed: int = 0, reps: int = 10) -> list[dict]:
    """Each shape and M on the decode layout (DecodeLayoutQ4, the matrix-core
    kernel the model runs) and, beside it, on the MLX layout (Q4Linear). The
    lm_head rows time the decode-layout GEMV + final argmax to the token (two
    launches) and the MLX-layout argmax partials alone."""
    rng = np.random.default_rng(seed)
    shapes = shapes or [(12288, 4096), (4096, 12288), (4096, 4096), (248320, 4096)]
    rows = []
    for N, K in shapes:
        lm_head = N == 248320
        ring = _ring(rng, N, K, zero_mean=lm_head)
        tring = [DecodeLayoutQ4(lin) for lin in ring]
        synchronize()
        for M in Ms:
            x = [DeviceArray.from_numpy(random_bf16(rng, (1, K))) for _ in range(M)]
            xx = DeviceArray.from_numpy(random_bf16(rng, (M, K)))
            if lm_head:
                P = N // 8
                pv = [DeviceArray((P,), np.float32) for _ in range(M)]
                pi = [DeviceArray((P,), np.uint32) for _ in range(M)]
                if M == 1:
                    fn = lambda lin, s: lin.encode_bf16_argmax_partial(x[0], pv[0], pi[0], stream=s)
                else:
                    fn = lambda lin, s: lin.encode_bf16_argmax_partial2(x[0], x[1], pv[0], pi[0], pv[1], pi[1],
                                                                        stream=s)
                tok = DeviceArray((2,), np.uint32)
                ws = DeviceArray((t16_argmax_workspace_bytes(),), np.uint8)
                tfn = lambda lin, s: lin.encode_argmax(xx, tok, ws, token_count=M, stream=s)
                out_bytes, t_out_bytes = M * P * 8, M * 4
                names = ("lm_head_argmax_t16", "lm_head_argmax_partials")
            else:
                y = DeviceArray((M, N), np.uint16)
                fn = lambda lin, s: lin.encode_bf16_fast(xx, y, token_count=M, stream=s)
                tfn = fn
                out_bytes = t_out_bytes = M * N * 2
                names = ("q4_gemv_t16", "q4_gemv")
            for name, f, items, ob in ((names[0], tfn, tring, t_out_bytes), (names[1], fn, ring, out_bytes)):
                ms = time_launches(f, items, reps=reps)
                algo = q4_bytes(N, K) + M * K * 2 + ob
                gbs = algo / (ms * 1e-3) / 1e9
                rows.append({"kernel": name, "layout": "decode" if items is tring else "mlx", "N": N, "K": K,
                             "M": M, "us": ms * 1e3, "algo_bytes": algo, "GBps": gbs,
                             "frac_peak": gbs / HBM_PEAK_GBS, "ring": len(ring)})
            if lm_head:
                o = DeviceArray((1,), np.uint32)
                argmax_pairs(pv[0], pi[0], o, N // 8)
                synchronize()
        for t in tring:
            t.close()
        for lin in ring:
            for a in (lin.weight, lin.scales, lin.biases):
                a.close()
    return rows


def silu_sweep(seed: int = 1, reps: int = 10) -> dict:
    rng = np.random.default_rng(seed)
    N, K = 12288, 4096
    one_g, one_u = random_q4(rng, N, K), random_q4(rng, N, K)
    copies = max(2, -(-ROTATE_BYTES // (2 * one_g.nbytes)))
    ring = [(Q4Linear.upload(one_g), Q4Linear.upload(one_u)) for _ in range(copies)]
    x = DeviceArray.from_numpy(random_bf16(rng, (1, K)))
    out = DeviceArray((1, N), np.uint16)
    ms = time_launches(lambda gu, s: gate_up_silu(gu[0], gu[1], x, out, stream=s), ring, reps=reps)
    algo = 2 * q4_bytes(N, K) + K * 2 + N * 2
    gbs = algo / (ms * 1e-3) / 1e9
    return {"kernel": "q4_gemv_silu_gate", "N": N, "K": K, "M": 1, "us": ms * 1e3, "algo_bytes": algo,
            "GBps": gbs, "frac_peak": gbs / HBM_PEAK_GBS}
