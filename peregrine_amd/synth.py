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
