#!/usr/bin/env python3
"""Headline benchmark: single-stream greedy decode of the Qwen3.5-9B-shaped
4-bit model on one MI355X, plus the HBM roofline of
the dominant Q4 GEMV and the CPU oracle baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one greedy decode token of the whole 32-layer stack (embedding,
24 Gated DeltaNet + 8 GQA layers, final norm, lm_head argmax). Synthetic data:
random-initialised weights in the MLX affine Q4 format, a 1600-token random
prompt ingested first (untimed), then W untimed and K timed decode steps.
Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s @batch1 (9B-shaped Q4) + Q4 GEMV achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
PROMPT_TOKENS = 1600
# HBM bytes per launch of the dominant kernel (the decode-layout gate/up GEMV),
# from two rocprofv3 --pmc passes (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000, the
# factors a plain 256 MiB copy kernel reads on the same counters);
# profiles/gemv_silu_gate_hbm_traffic.md.
DOMINANT_TRAFFIC_BYTES = 56_957_952


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def token_gemv_bytes(cfg) -> int:
    """Algorithmic bytes of one decode token's GEMV launches (Q4 weights +
    scales + biases): per GDN layer in_proj (qkv 8192 | z 4096 rows; the a / b
    gate rows, 32 each, are read by the recurrence kernel when hidden <= 4096)
    and out_proj 4096 x 4096, per attention layer q|gate 8192 + k 1024 + v 1024
    rows and o_proj 4096 x 4096, per layer gate/up 2 x 12288 and down
    4096 x 12288, and the lm_head."""
    from peregrine_amd.gemv_bench import q4_bytes

    H, F = cfg.hidden, cfg.intermediate
    n_attn = cfg.num_layers // cfg.full_attention_interval
    n_gdn = cfg.num_layers - n_attn
    gate_rows = 0 if H <= 4096 else 64
    gdn = q4_bytes(8192 + 4096 + gate_rows, H) + q4_bytes(4096, 4096)
    attn = q4_bytes(8192 + 1024 + 1024, H) + q4_bytes(H, 4096)
    mlp = 2 * q4_bytes(F, H) + q4_bytes(H, F)
    return n_gdn * gdn + n_attn * attn + cfg.num_layers * mlp + q4_bytes(cfg.vocab, H)


def dominant_kernel_roofline(iters: int = 100) -> dict:
    """Fused post_attention_layernorm + gate/up SiLU GEMV at the MLP shape
    (2 x 12288x4096 Q4): ~40% of the bytes a decode step streams. The kernel
    timed is the one the model runs: the matrix-core GEMV over the decode
    layout (prg_q4_gemv_t16_silu_gate_norm_bf16); the MLX-layout kernel
    (prg_q4_gemv_silu_gate_norm_bf16) is timed beside it. One launch per ring
    copy (>= 512 MiB of distinct weights, so every launch reads HBM, not the
    256 MiB Infinity Cache) is captured into a HIP graph on its own stream; the
    graph is replayed `iters / copies` times between two HIP events on that
    stream, as the decode loop replays its graph, so the average launch
    duration carries no host launch overhead."""
    import ctypes as C

    from peregrine_amd._lib import call
    from peregrine_amd.device import DeviceArray, Event, Graph, Stream, synchronize
    from peregrine_amd.gemv_bench import ROTATE_BYTES, q4_bytes
    from peregrine_amd.ops import Q4Linear
    from peregrine_amd.synth import random_bf16, random_q4

    N, K = 12288, 4096
    rng = np.random.default_rng(42)
    g, u = random_q4(rng, N, K, zero_mean=True), random_q4(rng, N, K, zero_mean=True)
    copies = max(2, -(-ROTATE_BYTES // (2 * g.nbytes)))
    ring = [(Q4Linear.upload(g), Q4Linear.upload(u)) for _ in range(copies)]

    def t16_copy(lin):
        dst = [DeviceArray(a.shape, a.dtype) for a in (lin.weight, lin.scales, lin.biases)]
        call("prg_q4_repack_t16", None, *lin._wsb(), *[C.c_void_p(d.ptr) for d in dst], N, K)
        return dst

    tring = [(t16_copy(gl), t16_copy(ul)) for gl, ul in ring]
    x = DeviceArray.from_numpy(random_bf16(rng, (K,), std=3.0))
    nw = DeviceArray.from_numpy(random_bf16(rng, (K,), std=0.1, mean=1.0))
    out = DeviceArray((N,), np.uint16)
    stream = Stream()
    sp = C.c_void_p(stream.handle)
    reps = max(1, iters // copies)
    launches = reps * copies
    a, b = Event(), Event()

    def time_ring(launch) -> float:
        """Average launch duration (us) of launch(i) over the ring, graph-replayed."""
        launch(0)  # eager first launch: kernel selection and occupancy queries happen outside the capture
        stream.synchronize()
        with Graph.capture(stream) as graph:
            for i in range(copies):
                launch(i)
        for _ in range(2):
            graph.launch()
        stream.synchronize()
        a.record(sp)
        for _ in range(reps):
            graph.launch()
        b.record(sp)
        stream.synchronize()
        graph.close()
        return a.elapsed_ms(b) * 1e3 / launches

    def launch_t16(i: int) -> None:
        gt, ut = tring[i % copies]
        call("prg_q4_gemv_t16_silu_gate_norm_bf16", sp, C.c_void_p(x.ptr), C.c_void_p(nw.ptr), C.c_float(1e-6),
             *[C.c_void_p(d.ptr) for d in gt], *[C.c_void_p(d.ptr) for d in ut], C.c_void_p(out.ptr), N, K)

    def launch_mlx(i: int) -> None:
        gl, ul = ring[i % copies]
        call("prg_q4_gemv_silu_gate_norm_bf16", sp, C.c_void_p(x.ptr), C.c_void_p(nw.ptr), C.c_float(1e-6),
             *gl._wsb(), *ul._wsb(), C.c_void_p(out.ptr), N, K)

    avg_us = time_ring(launch_t16)
    mlx_us = time_ring(launch_mlx)
    del ring, tring
    algo = 2 * q4_bytes(N, K) + 2 * K * 2 + N * 2  # gate+up weights, x + norm weight, out
    gbs = algo / (avg_us * 1e-6) / 1e9

    # The single-launch read floor: a streaming read of the same number of
    # bytes (prg_hip_read_kernel), over a ring of the same size, timed the same way.
    nbytes = (algo + 15) // 16 * 16
    bufs = [DeviceArray((nbytes,), np.uint8) for _ in range(copies)]
    sink = DeviceArray((1,), np.uint32)
    read_us = time_ring(lambda i: call("prg_hip_read_kernel", C.c_void_p(bufs[i % copies].ptr), C.c_size_t(nbytes),
                                       C.c_void_p(sink.ptr), sp))
    # Cross-check: a device-to-device hipMemcpyAsync of the same bytes from the
    # same ring (reads them once and writes them once), timed the same way.
    dst = DeviceArray((nbytes,), np.uint8)
    copy_us = time_ring(lambda i: call("prg_hip_memcpy", C.c_void_p(dst.ptr), C.c_void_p(bufs[i % copies].ptr),
                                       C.c_size_t(nbytes), 2, sp, 0))
    dst.close()
    for buf in bufs:
        buf.close()
    stream.close()
    synchronize()
    return {"kernel": "q4_gemv_t16_kernel<M=1,NMAT=2,S=4,EPI=silu_gate,NORM=rms> (mlp.gate_up, 2x12288x4096 Q4, "
                      "decode layout, matrix cores)",
            "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": DOMINANT_TRAFFIC_BYTES,
            "traffic_unit": "bytes/launch (PMC, calibrated)",
            "avg_us": round(avg_us, 3), "timing": "HIP events around graph replays (no host launch overhead)",
            "read_floor_us": round(read_us, 3), "read_floor_GBps": round(nbytes / (read_us * 1e-6) / 1e9, 1),
            "frac_of_read_floor": round(read_us / avg_us, 4),
            "memcpy_d2d_us": round(copy_us, 3), "memcpy_d2d_GBps_rw": round(2 * nbytes / (copy_us * 1e-6) / 1e9, 1),
            "mlx_layout_kernel": {"kernel": "q4_gemv_kernel<M=1,ROWS=1,ITERS=2,EPI=silu_gate,NORM=rms>",
                                  "avg_us": round(mlx_us, 3), "GBps": round(algo / (mlx_us * 1e-6) / 1e9, 1)},
            "algo_bytes_per_launch": int(algo), "launches": launches, "ring_copies": copies}


def prefill_flops(cfg, T: int) -> float:
    """Matmul FLOPs of one T-token prompt from an empty cache: 2 per weight per
    token over every Q4 projection (embedding gather and lm_head excluded; the
    lm_head runs on the last token only), plus causal attention (QK^T and PV,
    2 * 2 * T*(T+1)/2 * 256 per q head)."""
    h, f = cfg.hidden, cfg.intermediate
    gdn = (8192 + 4096 + 32 + 32) * h + h * 4096
    att = (8192 + 1024 + 1024) * h + h * 4096
    mlp = 3 * f * h
    n_att = sum(1 for i in range(cfg.num_layers) if not cfg.is_linear(i))
    n_gdn = cfg.num_layers - n_att
    weights = n_gdn * gdn + n_att * att + cfg.num_layers * mlp
    attn = n_att * 16 * 2 * 2 * (T * (T + 1) / 2) * 256
    return 2.0 * weights * T + attn + 2.0 * cfg.vocab * h


def gemv_sweep() -> list[dict]:
    from peregrine_amd.gemv_bench import sweep

    return [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()} for r in sweep()]


def host_info() -> dict:
    """Host CPUs of this box: nproc, the CPU model name, and the threads the
    CPU baselines use (the box's CPU share is 16 threads for one GPU)."""
    name = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    return {"nproc": nproc, "cpu_model": name, "threads": max(1, min(16, nproc))}


def _timed(fn, min_s: float = 0.3, max_reps: int = 20) -> float:
    """Seconds per call of fn(): at least one call, repeated until min_s."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or n >= max_reps:
            return dt / n


def cpu_configs(threads: int) -> list[dict]:
    """The C oracle (scalar restatement of the reference shaders) on BASELINE
    configs 1-4, on this box's host cores: single-threaded and row-parallel
    on `threads` threads (the row split keeps every output's arithmetic, so
    results do not depend on the thread count). Same seeded distributions as
    the GPU runs; per call, with the algorithmic bytes of the call."""
    from oracle import oracle
    from peregrine_amd.gemv_bench import q4_bytes
    from peregrine_amd.synth import random_bf16, random_q4

    o = oracle()
    rows = []

    def both(case, config, algo, fn, parallel=True):
        r = {"config": config, "case": case, "algo_bytes": int(algo)}
        for t in ((1, threads) if parallel else (1,)):
            o.set_threads(t)
            sec = _timed(fn)
            r[f"ms_{t}t"] = round(sec * 1e3, 3)
            r[f"GBps_{t}t"] = round(algo / sec / 1e9, 3)
        if not parallel:
            r["note"] = "the oracle's decode recurrence runs on one thread"
        rows.append(r)

    rng = np.random.default_rng(0)  # config 1: seed 0, the BASELINE distributions
    wt = random_q4(rng, 12288, 4096)
    x = random_bf16(rng, (1, 4096))
    both("q4 gemv 12288x4096 (seed 0)", 1, q4_bytes(12288, 4096) + 4096 * 2 + 12288 * 2, lambda: o.q4_gemv(x, wt))
    rng = np.random.default_rng(1)
    for N, K in ((4096, 12288), (4096, 4096)):
        w2, x2 = random_q4(rng, N, K), random_bf16(rng, (1, K))
        both(f"q4 gemv {N}x{K}", 2, q4_bytes(N, K) + K * 2 + N * 2, lambda: o.q4_gemv(x2, w2))
    wl, xl = random_q4(rng, 248320, 4096, zero_mean=True), random_bf16(rng, (4096,))

    def lm_head():
        pv, pi = o.q4_argmax_partial(xl, wl)
        o.argmax_pairs(pv[0], pi[0])

    both("lm_head 248320x4096 + argmax", 2, q4_bytes(248320, 4096) + 4096 * 2 + 31040 * 8, lm_head)
    del wl

    # config 3: one Gated DeltaNet decode layer (conv, recurrence, gated norm)
    rng = np.random.default_rng(3)
    cs = rng.normal(0, 1.0, size=(3, 8192)).astype(np.float32)
    cw = random_bf16(rng, (8192, 4), std=0.5)
    qkv = random_bf16(rng, (8192,))
    S = rng.normal(0, 0.1, size=(32, 128, 128)).astype(np.float32)
    a, b = random_bf16(rng, (32,)), random_bf16(rng, (32,))
    A_log = np.zeros(32, np.float32)
    dt = np.zeros(32, np.uint16)
    nw, z = random_bf16(rng, (128,), std=0.1, mean=1.0), random_bf16(rng, (4096,))

    def gdn_layer():
        c, _ = o.conv1d_decode(cs, qkv, cw)
        y, _ = o.gated_delta_decode(S, c, a, b, A_log, dt)
        o.rmsnorm_gated(y, nw, z, 128)

    both("gdn decode layer (conv + recurrence + gated norm)", 3,
         2 * S.nbytes + 2 * cs.nbytes + cw.nbytes + qkv.nbytes + z.nbytes + 4096 * 2, gdn_layer, parallel=False)

    # config 4: one GQA decode attention layer (prepare + attention) at L
    for L in (4096, 24576, 65536):
        rng = np.random.default_rng(4 + L)
        kc, vc = random_bf16(rng, (4, L, 256)), random_bf16(rng, (4, 256, L))
        pq, kin, vin = random_bf16(rng, (16 * 512,)), random_bf16(rng, (1024,)), random_bf16(rng, (1024,))
        qw, kw = random_bf16(rng, (256,), std=0.1, mean=1.0), random_bf16(rng, (256,), std=0.1, mean=1.0)

        # the q/k norm + RoPE + append (~40 KB of work) runs once, untimed: the
        # numpy binding copies both caches around it
        q, g, kc, vc = o.attn_prepare(pq, qw, kin, vin, kw, kc, vc, L, L - 1, L - 1)
        both(f"gqa decode attention L={L} (split-context attention + gated merge)", 4,
             4096 * L + 16 * 256 * 2 * 3, lambda: o.attn_decode(q, kc, vc, g, L, L))
    o.set_threads(threads)
    return rows


def cpu_baseline(model, snapshot: dict, tokens, start: int, info: dict, budget_s: float = 20.0) -> dict:
    """The C oracle running the same 9B-shaped decode step on the host cores,
    row-parallel, at the GPU's context: its state is the GPU's state after
    the prompt (KV caches and GDN states copied from the device), and it is
    teacher-forced on the GPU's greedy tokens from position `start`, until
    ~budget_s. Each step also computes the oracle's full bf16 logits, so the
    agreement with the GPU's next token is classified by the oracle's top-2
    margin: on a decisive step (margin above four bf16 ulps of the top logit)
    the tokens must agree; below it a different winner is a tie-break by a
    different fp32 summation order. Every disagreement is listed with both
    tokens, the margin and the oracle's logit of the GPU's token."""
    from oracle import oracle
    from oracle.model import OracleModel, decisive_margin

    threads = info["threads"]
    o = oracle()
    o.set_threads(threads)
    t0 = time.time()
    om = OracleModel(model, snapshot["max_seq"])
    load_s = time.time() - t0
    om.load_state(snapshot)
    n = same = decisive = decisive_same = 0
    mismatches = []
    t0 = time.time()
    while n + 1 < len(tokens):
        pred, logits = om.step(int(tokens[n]), start + n, want_logits=True)
        gpu = int(tokens[n + 1])
        i1, i2, margin, guard = decisive_margin(logits)
        dec = margin > guard
        same += int(pred == gpu)
        decisive += int(dec)
        decisive_same += int(dec and pred == gpu)
        if pred != gpu:
            mismatches.append({"pos": start + n, "gpu": gpu, "oracle": int(pred), "runner_up": i2,
                               "margin": float(margin), "guard": float(guard), "decisive": bool(dec),
                               "oracle_logit_of_gpu_token": float(logits[gpu]), "oracle_top": float(logits[i1])})
        n += 1
        if time.time() - t0 > budget_s:
            break
    dt = time.time() - t0
    return {"value": round(n / dt, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "nproc": info["nproc"], "cpu_model": info["cpu_model"],
            "sample": f"{n} decode steps of the same 9B-shaped model at positions {start}..{start + n - 1}, "
                      f"on the GPU's state after the {start}-token prompt, teacher-forced on the GPU's tokens "
                      f"(C oracle, {threads} threads, each step with its full lm_head logits; weight readback "
                      f"{load_s:.1f}s excluded)",
            "predicts_gpu_token": f"{same}/{n}",
            "decisive_agree": f"{decisive_same}/{decisive}",
            "decisive_rule": "oracle top-1 minus top-2 logit > 4 bf16 ulps of the top logit",
            "mismatches": mismatches}


def snapshot_state(st) -> dict:
    """Host copy of a ModelState's GDN states and KV caches."""
    snap = {"max_seq": st.max_seq, "stride": st.stride}
    cfg = st.model.cfg
    for i in range(cfg.num_layers):
        names = ("conv", "recur") if cfg.is_linear(i) else ("cache_k", "cache_v")
        for nm in names:
            snap[f"layers.{i}.{nm}"] = st.read(f"layers.{i}.{nm}", np.float32 if cfg.is_linear(i) else np.uint16)
    return snap


def long_prefill(model, tokens: int = 16384) -> dict:
    """Cold prefill of a `tokens`-token random prompt (no cached prefix) on a
    fresh state: the reference's reason for chunked prefill is 16k-token agent
    prefixes. The prompt workspace is allocated by a 1-token prefill first;
    the timed call is the whole multi-chunk ingestion to the first token."""
    from peregrine_amd.model import ModelState

    st = ModelState(model, tokens + 64)
    prompt = np.random.default_rng(5).integers(0, model.cfg.vocab, size=tokens).astype(np.uint32)
    st.prefill(prompt[:1])
    t0 = time.time()
    st.prefill(prompt)
    sec = time.time() - t0
    st.close()
    return {"tokens": tokens, "ms": round(sec * 1e3, 1), "tok_s": round(tokens / sec, 1),
            "tflops": round(prefill_flops(model.cfg, tokens) / sec / 1e12, 2), "max_seq": tokens + 64}


def mtp_run(steps: int) -> dict:
    """BASELINE configs[4]'s repeat with a 1-layer MTP draft head: the same
    9B-shaped model plus a random-init drafter (fc 4096x8192 Q4, one attention
    layer, shared lm_head). The device-resident speculative loop drafts one
    token, verifies two rows through all 32 layers (M = 2 GEMVs), advances the
    drafter and accepts or rejects, one captured graph per step. A random
    drafter is almost never accepted, so this measures the cost of a
    speculative step; emitted tokens equal plain greedy decoding (tested)."""
    from dataclasses import replace

    from peregrine_amd.model import QWEN35_9B, DeviceModel, ModelState

    cfg = replace(QWEN35_9B, mtp_layers=1)
    model = DeviceModel(cfg, seed=0)
    st = ModelState(model, PROMPT_TOKENS + steps + 8)
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, cfg.vocab, size=PROMPT_TOKENS).astype(np.uint32)
    st.generate_speculative(prompt, 8)  # first call: prompt workspace and graph capture
    toks, acc, att, ms = st.generate_speculative(prompt, steps)
    out = {"emitted_tokens": steps, "loop_ms": round(ms, 2), "tok_s": round(steps / (ms * 1e-3), 2),
           "verify_steps": att, "accepted_drafts": acc, "ms_per_verify_step": round(ms / max(att, 1), 4),
           "drafter": "random-init 1-layer MTP head (fc + attention layer + shared lm_head)"}
    # The accept path: the same model with the drafter rewritten into a copy
    # drafter (draft = the token it is given) and the target's final norm
    # e_0 (greedy then picks one of two tokens and repeats often), so most
    # drafts are accepted; same kernels and bytes per step as above.
    from peregrine_amd.synth import copy_drafter_tensors, unit_norm_e0

    o_meta = model.tensor_ptr("mtp.layers.0.self_attn.o_proj.scales")[1] // 2
    d_meta = model.tensor_ptr("mtp.layers.0.mlp.down_proj.scales")[1] // 2
    for name, arr in copy_drafter_tensors(cfg.hidden, o_meta, d_meta).items():
        model.write(name, arr)
    model.write("language_model.model.norm.weight", unit_norm_e0(cfg.hidden))
    st.generate_speculative(prompt, 8)
    toks, acc, att, ms = st.generate_speculative(prompt, steps)
    st.close()
    model.close()
    out["accept_path"] = {"emitted_tokens": steps, "loop_ms": round(ms, 2), "tok_s": round(steps / (ms * 1e-3), 2),
                          "verify_steps": att, "accepted_drafts": acc,
                          "acceptance": round(acc / max(att, 1), 4),
                          "tokens_per_verify_step": round(steps / max(att, 1), 4),
                          "ms_per_verify_step": round(ms / max(att, 1), 4),
                          "drafter": "copy drafter (fc = [0 | I], zero o_proj / down_proj) with the target's final "
                                     "norm e_0: synthetic weights that make drafts agree, to time accepted steps"}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-mtp", action="store_true", help="skip the MTP speculative run (BASELINE configs[4], repeat)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the operator benchmarks of BASELINE configs 2-4 (graph-replayed)")
    ap.add_argument("--no-long-prefill", action="store_true", help="skip the 16k-token cold prefill")
    ap.add_argument("--eager", action="store_true",
                    help="launch each token's kernels directly instead of replaying the HIP graph "
                         "(for kernel tracers; slower)")
    ap.add_argument("--configs", action="store_true",
                    help="only the operator benchmarks of BASELINE configs 2-4 (Q4 GEMV sweep, 24 GDN layers, "
                         "GQA decode attention at L = 4096 / 24576 / 65536), one JSON line")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant-kernel loop and a 256 MiB copy-kernel reference (for PMC runs)")
    ap.add_argument("--prefill-only", type=int, default=0, metavar="N",
                    help="only N ingests of the 1600-token prompt into the 9B-shaped model with the prepared dense "
                         "prompt weights (the first allocates the prompt workspace), one JSON line (for PMC runs "
                         "on the prompt GEMMs)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU (no multi-GPU path); use --gpus 1"}))
        return 2

    if a.eager:
        os.environ["PEREGRINE_EAGER"] = "1"
    from peregrine_amd import device
    from peregrine_amd.model import QWEN35_9B, DeviceModel, ModelState

    device.init(0)
    log("[bench]", device.device_name())
    if a.configs:
        from peregrine_amd.op_bench import configs_3_4

        rows = gemv_sweep()
        for r in rows:
            r["config"] = 2
        rows += configs_3_4()
        for r in rows:
            log(f"[bench] {r}")
        print(json.dumps({"configs": rows, "device": device.device_name()}), flush=True)
        return 0
    if a.roofline_only:
        import ctypes as C

        from peregrine_amd._lib import call
        from peregrine_amd.device import DeviceArray

        nbytes = 256 * 1024 * 1024
        src, dst = DeviceArray((nbytes,), np.uint8), DeviceArray((nbytes,), np.uint8)
        for _ in range(4):
            call("prg_hip_copy_kernel", C.c_void_p(dst.ptr), C.c_void_p(src.ptr), C.c_size_t(nbytes), None)
        device.synchronize()
        roof = dominant_kernel_roofline(iters=20)
        print(json.dumps({"copy_bytes": nbytes, "roofline": roof}), flush=True)
        return 0
    if a.prefill_only:
        model = DeviceModel(QWEN35_9B, seed=0)
        model.prepare_dense()
        st = ModelState(model, PROMPT_TOKENS + 64)
        prompt = np.random.default_rng(0).integers(0, QWEN35_9B.vocab, size=PROMPT_TOKENS).astype(np.uint32)
        runs = []
        for i in range(a.prefill_only):
            t0 = time.time()
            first = st.prefill(prompt)
            runs.append(round((time.time() - t0) * 1e3, 2))
            log(f"[bench] ingest {i}: {runs[-1]} ms, first token {first}")
        best = min(runs[1:] or runs)
        print(json.dumps({"prefill_ms": runs, "tokens": PROMPT_TOKENS, "first_token": int(first),
                          "tflops_best": round(prefill_flops(QWEN35_9B, PROMPT_TOKENS) / (best * 1e-3) / 1e12, 2)}),
              flush=True)
        st.close()
        model.close()
        return 0
    t0 = time.time()
    model = DeviceModel(QWEN35_9B, seed=0)
    log(f"[bench] model init {time.time() - t0:.1f}s, {model.weight_bytes / 1e9:.2f} GB weights")
    # prepared dense weights for the prompt GEMMs (decode reads the Q4 weights)
    t0 = time.time()
    dense_bytes = model.prepare_dense()
    dense_ms = (time.time() - t0) * 1e3
    log(f"[bench] prepared dense prompt weights: {dense_bytes / 1e9:.2f} GB in {dense_ms:.1f} ms")
    max_seq = PROMPT_TOKENS + a.warmup + a.steps
    st = ModelState(model, max_seq)
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, QWEN35_9B.vocab, size=PROMPT_TOKENS).astype(np.uint32)
    t0 = time.time()
    st.prefill(prompt)  # first call also allocates the prompt-path workspace
    cold_s = time.time() - t0
    runs = []
    for _ in range(3):  # warm ingests of the same prompt; the median is reported
        t0 = time.time()
        first = st.prefill(prompt)
        runs.append(time.time() - t0)
    prefill_s = sorted(runs)[1]
    prefill = {"tokens": PROMPT_TOKENS, "ms": round(prefill_s * 1e3, 2), "runs_ms": [round(r * 1e3, 2) for r in runs],
               "tok_s": round(PROMPT_TOKENS / prefill_s, 1),
               "tflops": round(prefill_flops(QWEN35_9B, PROMPT_TOKENS) / prefill_s / 1e12, 2),
               "first_call_ms": round(cold_s * 1e3, 2),
               "dense_weights": {"bytes": dense_bytes, "prepare_ms": round(dense_ms, 2)}}
    log(f"[bench] prompt ingest {PROMPT_TOKENS} tokens {prefill_s * 1e3:.1f} ms "
        f"({prefill['tok_s']} tok/s, {prefill['tflops']} TFLOP/s), first token {first}")
    snap = None if a.no_cpu else snapshot_state(st)
    wtoks = st.decode(a.warmup)[0] if a.warmup else np.zeros(0, np.uint32)
    device.synchronize()
    toks, ms = st.decode(a.steps)
    device.synchronize()
    tok_s = a.steps / (ms * 1e-3)
    log(f"[bench] decode {a.steps} steps {ms:.1f} ms -> {tok_s:.1f} tok/s; last tokens {toks[-4:].tolist()}")

    # The token loop's GEMVs alone, graph-replayed with the model's weights
    # (the decode state is not used again: the CPU baseline starts from `snap`).
    # Not under --eager: that mode is for kernel tracers, and rocprofv3's
    # kernel trace has crashed in this capture (host SIGSEGV inside the tool).
    token_loop = None
    if not a.eager:
        gemv_us = st.time_token_gemvs(32)
        gemv_bytes = token_gemv_bytes(QWEN35_9B)
        token_loop = {"gemv_us_per_token": round(gemv_us, 2), "gemv_bytes_per_token": gemv_bytes,
                      "gemv_launches_per_token": 4 * QWEN35_9B.num_layers + 1,
                      "GBps": round(gemv_bytes / (gemv_us * 1e-6) / 1e9, 1),
                      "frac_peak": round(gemv_bytes / (gemv_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                      "share_of_step": round(gemv_us / (ms / a.steps * 1e3), 4)}
        log(f"[bench] token-loop GEMVs {token_loop}")

    roof = dominant_kernel_roofline()
    log(f"[bench] dominant kernel {roof['avg_us']} us, {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}% of peak); "
        f"a streaming read of the same bytes takes {roof['read_floor_us']} us ({roof['read_floor_GBps']} GB/s)")
    extra = {}
    if not a.no_long_prefill:
        extra["prefill_16k"] = long_prefill(model)
        log(f"[bench] 16k cold prefill {extra['prefill_16k']}")
    cpu = None
    info = host_info()
    if not a.no_cpu:
        # the GPU's tokens from position PROMPT_TOKENS: the prompt's next token, then every decode step's
        gpu_toks = np.concatenate([[first], wtoks, toks]).astype(np.uint32)
        cpu = cpu_baseline(model, snap, gpu_toks, PROMPT_TOKENS, info)
        log(f"[bench] cpu baseline {cpu}")
    st.close()
    weight_bytes = int(model.weight_bytes)
    model.close()
    mtp = None
    if not a.no_mtp:
        mtp = mtp_run(a.steps)
        log(f"[bench] mtp speculative loop {mtp}")
    if not a.no_configs:
        from peregrine_amd.op_bench import configs_3_4

        rows = gemv_sweep()
        for r in rows:
            r["config"] = 2
        extra["configs_2_4"] = rows + configs_3_4()
        for r in extra["configs_2_4"]:
            log(f"[bench] {r}")
    if not a.no_cpu:
        extra["cpu_configs_1_4"] = {"host": info, "rows": cpu_configs(info["threads"])}
        for r in extra["cpu_configs_1_4"]["rows"]:
            log(f"[bench] cpu {r}")

    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms / a.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init Q4 weights (MLX affine g64), random prompt ids, greedy decode",
        "config": {"workload": "qwen3.5-9b-shaped q4 decode, batch 1 (BASELINE configs[4])",
                   "layers": QWEN35_9B.num_layers, "gdn_layers": 24, "attention_layers": 8,
                   "hidden": QWEN35_9B.hidden, "ffn": QWEN35_9B.intermediate, "vocab": QWEN35_9B.vocab,
                   "prompt_tokens": PROMPT_TOKENS, "context_at_end": int(max_seq), "batch": 1,
                   "weight_bytes": weight_bytes, "parallelism": "single GPU",
                   "execution": "eager launches" if a.eager else "one HIP graph replay per token"},
        "roofline": roof,
        "token_loop": token_loop,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "mtp": mtp,
        **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
