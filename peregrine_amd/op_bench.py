"""Timing of the decode-path operators at BASELINE configs 3 and 4 on one GPU.

* Config 3: 24 Gated DeltaNet decode layers back to back. A layer is the
  depthwise causal conv1d over the 8192-channel rolling state
  (prg_conv1d_silu_decode_bf16) followed by the recurrent state update with
  the gated RMSNorm of its output (prg_gated_delta_decode_norm_bf16). Every
  layer owns its states; sets of 24 layers are rotated so that >= 512 MiB of
  distinct state is touched between two uses (MI355X's Infinity Cache is
  256 MiB).
* Config 4: one full-attention GQA decode layer at context L (16 q heads,
  4 KV heads, head_dim 256, RoPE theta 1e7 at position L - 1) as the model
  runs it (prg_attn_decode_step_bf16: split partials over the cached tokens
  with q normalised and rotated in the kernel, then the gated merge that adds
  the new token and appends its K/V), alone and as 8 stacked layers with
  distinct caches, rotated the same way.

Each case is captured once into a HIP graph on its own stream and replayed;
times are the median over replays bracketed by HIP events, per layer (or per
stack), with no host launch overhead. Inputs are synthetic and seeded.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import ops
from .device import DeviceArray, Event, Graph, Stream, synchronize
from .synth import random_bf16

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 512 * 1024 * 1024


def time_graph(stream: Stream, issue, reps: int) -> float:
    """Milliseconds per replay of the graph of issue(): the median over
    `reps` replays, each bracketed by its own pair of HIP events on `stream`."""
    issue()  # eager first pass: kernel selection outside the capture
    stream.synchronize()
    with Graph.capture(stream) as g:
        issue()
    for _ in range(2):
        g.launch()
    stream.synchronize()
    evs = [(Event(), Event()) for _ in range(reps)]
    for a, b in evs:
        a.record(C.c_void_p(stream.handle))
        g.launch()
        b.record(C.c_void_p(stream.handle))
    stream.synchronize()
    ms = float(np.median([a.elapsed_ms(b) for a, b in evs]))
    for a, b in evs:
        a.close()
        b.close()
    g.close()
    return ms


def gdn_layers(layers: int = 24, seed: int = 3, reps: int = 20, fused_norm: bool = True) -> dict:
    rng = np.random.default_rng(seed)
    conv_dim, hv, d = 8192, 32, 128
    state_bytes = hv * d * d * 4
    conv_state_bytes = 3 * conv_dim * 4
    per_layer = 2 * state_bytes + 2 * conv_state_bytes + conv_dim * 4 * 2 + conv_dim * 2 + 2 * conv_dim * 2 \
        + 3 * 4096 * 2 + 32 * (2 + 2 + 4 + 2) + 128 * 2
    sets = max(1, -(-ROTATE_BYTES // (layers * per_layer)))
    # shared small inputs (read-only), per-layer states and weights
    a, b = DeviceArray.from_numpy(random_bf16(rng, (hv,))), DeviceArray.from_numpy(random_bf16(rng, (hv,)))
    # A_log = 0 and dt_bias = 0, so decay = exp(-softplus(a))
    A_log = DeviceArray.from_numpy(np.zeros(hv, np.float32))
    dt = DeviceArray.from_numpy(np.zeros(hv, np.uint16))
    nw = DeviceArray.from_numpy(random_bf16(rng, (d,), std=0.1, mean=1.0))
    S0 = rng.normal(0, 0.1, size=(hv, d, d)).astype(np.float32)
    cs0 = rng.normal(0, 1.0, size=(3, conv_dim)).astype(np.float32)
    L = []
    for _ in range(sets * layers):
        L.append({
            "S": DeviceArray.from_numpy(S0), "cs": DeviceArray.from_numpy(cs0),
            "w": DeviceArray.from_numpy(random_bf16(rng, (conv_dim, 4), std=0.5)),
            "x": DeviceArray.from_numpy(random_bf16(rng, (conv_dim,))),
            "z": DeviceArray.from_numpy(random_bf16(rng, (hv * d,))),
            "c": DeviceArray((conv_dim,), np.uint16), "o": DeviceArray((hv * d,), np.uint16),
            "y": DeviceArray((hv * d,), np.uint16),
        })
    st = Stream()

    def issue():
        for ly in L:
            ops.conv1d_silu_decode(ly["cs"], ly["x"], ly["w"], ly["c"], stream=st.handle)
            if fused_norm:
                ops.gated_delta_decode_norm(ly["S"], ly["c"], a, b, A_log, dt, nw, ly["z"], ly["o"], stream=st.handle)
            else:
                ops.gated_delta_decode(ly["S"], ly["c"], a, b, A_log, dt, ly["y"], stream=st.handle)
                ops.rmsnorm_gated(ly["y"], nw, ly["z"], ly["o"], stream=st.handle)

    ms = time_graph(st, issue, reps) / sets
    st.close()
    for ly in L:
        for v in ly.values():
            v.close()
    synchronize()
    total = layers * per_layer
    gbs = total / (ms * 1e-3) / 1e9
    how = "conv1d, state update with the gated norm fused" if fused_norm else "conv1d, state update, gated norm"
    return {"config": 3, "case": f"gdn decode x{layers} layers ({how})",
            "us": round(ms * 1e3, 2), "us_per_layer": round(ms * 1e3 / layers, 3),
            "algo_bytes": int(total), "GBps": round(gbs, 1), "frac_peak": round(gbs / HBM_PEAK_GBS, 4),
            "launches_per_layer": 2 if fused_norm else 3, "rotated_sets": sets}


def attention(L: int, layers: int = 1, seed: int = 4, reps: int = 20) -> dict:
    """One decode step of a full-attention layer as the model runs it
    (prg_attn_decode_step_bf16: q/k norm + RoPE, split partials over the L - 1
    cached tokens, merge with the new token and its K/V append) at context L."""
    rng = np.random.default_rng(seed + L + layers)
    stride = L
    kv_bytes = 4 * stride * 256 * 2
    per_layer_algo = 2 * 4 * L * 256 * 2 + 16 * 512 * 2 + 2 * 1024 * 2 + 2 * 4096 * 2
    sets = max(1, -(-ROTATE_BYTES // (layers * 2 * kv_bytes)))
    pq = DeviceArray.from_numpy(random_bf16(rng, (16 * 512,)))
    qw = DeviceArray.from_numpy(random_bf16(rng, (256,), std=0.1, mean=1.0))
    kw = DeviceArray.from_numpy(random_bf16(rng, (256,), std=0.1, mean=1.0))
    kin = DeviceArray.from_numpy(random_bf16(rng, (1024,)))
    vin = DeviceArray.from_numpy(random_bf16(rng, (1024,)))
    kc0 = random_bf16(rng, (4, stride, 256))
    vc0 = random_bf16(rng, (4, 256, stride))
    caches = [(DeviceArray.from_numpy(kc0), DeviceArray.from_numpy(vc0)) for _ in range(sets * layers)]
    out = DeviceArray((16 * 256,), np.uint16)
    ws = DeviceArray((ops.attn_step_workspace_bytes(stride),), np.uint8)
    st = Stream()
    pos = L - 1

    def issue():
        for kc, vc in caches:
            ops.attn_decode_step(pq, qw, kin, vin, kw, kc, vc, out, ws, stride, pos, pos, stream=st.handle)

    ms = time_graph(st, issue, reps) / sets
    st.close()
    for kc, vc in caches:
        kc.close()
        vc.close()
    for x in (pq, qw, kw, kin, vin, out, ws):
        x.close()
    synchronize()
    total = layers * per_layer_algo
    gbs = total / (ms * 1e-3) / 1e9
    return {"config": 4, "case": f"gqa decode attention L={L} x{layers} layer(s) (decode step: partials + merge)",
            "L": L, "layers": layers, "us": round(ms * 1e3, 2), "us_per_layer": round(ms * 1e3 / layers, 3),
            "algo_bytes": int(total), "GBps": round(gbs, 1), "frac_peak": round(gbs / HBM_PEAK_GBS, 4),
            "launches_per_layer": 2, "rotated_sets": sets}


def configs_3_4() -> list[dict]:
    rows = [gdn_layers(fused_norm=True), gdn_layers(fused_norm=False)]
    for L in (4096, 24576, 65536):
        for layers in (1, 8):
            rows.append(attention(L, layers))
    return rows
