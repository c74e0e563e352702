"""Seeded synthetic inputs in the reference's data formats (numpy, host side).

MLX affine Q4, group 64: weight u32 [N, K/8] with nibble j of word c holding
column 8c+j; scales/biases bf16 [N, K/64]; dequantised w = s*q + b.
bf16 values are carried as uint16 bit patterns everywhere.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def f32_to_bf16(a) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (NaN stays NaN)."""
    shape = np.shape(a)
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r.reshape(shape)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_q4(q: np.ndarray) -> np.ndarray:
    """q uint8 [N, K] with values 0..15 -> u32 [N, K/8] (lowest nibble first)."""
    q = np.asarray(q, dtype=np.uint32)
    N, K = q.shape
    assert K % 8 == 0
    q = q.reshape(N, K // 8, 8)
    w = np.zeros((N, K // 8), dtype=np.uint32)
    for j in range(8):
        w |= q[:, :, j] << np.uint32(4 * j)
    return w


def unpack_q4(w: np.ndarray) -> np.ndarray:
    """u32 [N, K/8] -> uint8 [N, K]."""
    w = np.asarray(w, dtype=np.uint32)
    N, W = w.shape
    out = np.empty((N, W, 8), dtype=np.uint8)
    for j in range(8):
        out[:, :, j] = (w >> np.uint32(4 * j)) & 0xF
    return out.reshape(N, W * 8)


@dataclass
class Q4Weight:
    w: np.ndarray  # u32 [N, K/8]
    s: np.ndarray  # bf16 bits [N, K/64]
    b: np.ndarray  # bf16 bits [N, K/64]

    @property
    def shape(self) -> tuple[int, int]:
        return self.w.shape[0], self.w.shape[1] * 8

    @property
    def nbytes(self) -> int:
        return self.w.nbytes + self.s.nbytes + self.b.nbytes

    def dequant_f64(self) -> np.ndarray:
        """Exact dense weights (float64) — s*q + b without rounding."""
        q = unpack_q4(self.w).astype(np.float64)
        N, K = q.shape
        s = np.repeat(bf16_to_f32(self.s).astype(np.float64), 64, axis=1)
        b = np.repeat(bf16_to_f32(self.b).astype(np.float64), 64, axis=1)
        return s * q + b


def random_q4(rng: np.random.Generator, N: int, K: int, scale_lo: float = 0.001,
              scale_hi: float = 0.02, bias_std: float = 0.05, zero_mean: bool = False) -> Q4Weight:
    """BASELINE config-1 distribution: q ~ U{0..15}, s ~ U(lo, hi), b ~ N(0, std)
    per (row, 64-group). zero_mean shifts b by -7.5*s so dequantised weights are
    centred (healthier logits for multi-layer runs)."""
    assert K % 64 == 0
    w = np.frombuffer(rng.bytes(N * K // 2), dtype=np.uint32).reshape(N, K // 8).copy()
    s = rng.uniform(scale_lo, scale_hi, size=(N, K // 64)).astype(np.float32)
    b = rng.normal(0.0, bias_std, size=(N, K // 64)).astype(np.float32)
    s16 = f32_to_bf16(s)
    if zero_mean:
        b = b - 7.5 * bf16_to_f32(s16)
    return Q4Weight(w=w, s=s16, b=f32_to_bf16(b))


def random_bf16(rng: np.random.Generator, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    return f32_to_bf16(rng.normal(mean, std, size=shape).astype(np.float32))


def copy_drafter_tensors(hidden: int, o_proj_meta: int, down_meta: int) -> dict:
    """Tensors that turn a random 1-layer MTP drafter into a "copy" drafter
    whose draft is the token it is given: fc = [0 | I] passes the target's
    normalised hidden through (unit scales, zero biases), the drafter layer's
    o_proj and down_proj have zero scales and biases (so its attention and
    MLP add nothing), and the pre-fc hidden norm and final norm are ones, so
    the shared lm_head sees the target's own hidden. o_proj_meta / down_meta:
    element counts of those projections' scale (and bias) tensors.
    Used to time and test the speculative loop's accept path."""
    H = hidden
    q = np.zeros((H, 2 * H), np.uint32)
    q[np.arange(H), H + np.arange(H)] = 1
    one = f32_to_bf16(np.float32(1.0))
    return {
        "mtp.fc.weight": pack_q4(q),
        "mtp.fc.scales": np.full((H, 2 * H // 64), one, np.uint16),
        "mtp.fc.biases": np.zeros((H, 2 * H // 64), np.uint16),
        "mtp.layers.0.self_attn.o_proj.scales": np.zeros(o_proj_meta, np.uint16),
        "mtp.layers.0.self_attn.o_proj.biases": np.zeros(o_proj_meta, np.uint16),
        "mtp.layers.0.mlp.down_proj.scales": np.zeros(down_meta, np.uint16),
        "mtp.layers.0.mlp.down_proj.biases": np.zeros(down_meta, np.uint16),
        "mtp.pre_fc_norm_hidden.weight": np.full(H, one, np.uint16),
        "mtp.norm.weight": np.full(H, one, np.uint16),
    }


def unit_norm_e0(hidden: int) -> np.ndarray:
    """Final-norm weight e_0: the logits become lm_head[:, 0] * h_0 / rms(h),
    so greedy decoding picks one of two tokens (by the sign of h_0) and
    repeats often, which a copy drafter then predicts."""
    w = np.zeros(hidden, np.uint16)
    w[0] = f32_to_bf16(np.float32(1.0))
    return w
