"""TEST INFRASTRUCTURE: numpy wrappers over the C oracle (liboracle.so)."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "liboracle.so"

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32 = C.c_uint32


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class Oracle:
    def __init__(self, path: Path = ORACLE_LIB) -> None:
        if not path.exists():
            raise RuntimeError(f"{path} not built; run `python -m peregrine_amd.build --oracle`")
        d = C.CDLL(str(path))
        self.d = d
        d.orc_set_threads.argtypes = [C.c_int]
        d.orc_f2bf.argtypes = [C.c_float]
        d.orc_f2bf.restype = C.c_uint16
        d.orc_bf2f.argtypes = [C.c_uint16]
        d.orc_bf2f.restype = C.c_float
        d.orc_get_threads.restype = C.c_int
        d.orc_q4_dequantize_bf16.argtypes = [_u32p, _u16p, _u16p, _u16p, _u32, _u32]
        d.orc_q4_dots.argtypes = [_u16p, _u32, _u32p, _u16p, _u16p, _f32p, _u32, _u32]
        d.orc_q4_gemv_bf16.argtypes = [_u16p, _u32p, _u16p, _u16p, _u16p, _u32, _u32, _u32]
        d.orc_q4_gemv_residual_add_bf16.argtypes = [_u16p, _u32p, _u16p, _u16p, _u16p, _u16p, _u32, _u32, _u32]
        d.orc_q4_gemv_silu_gate_bf16.argtypes = [_u16p, _u32p, _u16p, _u16p, _u32p, _u16p, _u16p, _u16p, _u32, _u32, _u32]
        d.orc_q4_gemv_argmax_partial_bf16.argtypes = [_u16p, _u32p, _u16p, _u16p, _f32p, _u32p, _u32, _u32, _u32]
        d.orc_argmax_pairs_f32_u32.argtypes = [_f32p, _u32p, _u32]
        d.orc_argmax_pairs_f32_u32.restype = C.c_uint32

    # ------------------------------------------------------------------ misc
    def set_threads(self, n: int) -> None:
        self.d.orc_set_threads(int(n))

    @property
    def threads(self) -> int:
        return self.d.orc_get_threads()

    def f2bf(self, v) -> np.ndarray:
        v = np.asarray(v, np.float32).ravel()
        return np.array([self.d.orc_f2bf(float(x)) for x in v], np.uint16)

    # -------------------------------------------------------------- Q4 ops
    def q4_dequantize(self, wt) -> np.ndarray:
        N, K = wt.shape
        out = np.empty((N, K), np.uint16)
        self.d.orc_q4_dequantize_bf16(_c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16), out, N, K)
        return out

    def q4_dots(self, x, wt) -> np.ndarray:
        x = _c(np.atleast_2d(x), np.uint16)
        N, K = wt.shape
        M = x.shape[0]
        out = np.empty((M, N), np.float32)
        self.d.orc_q4_dots(x, M, _c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16), out, N, K)
        return out

    def q4_gemv(self, x, wt) -> np.ndarray:
        x = _c(np.atleast_2d(x), np.uint16)
        N, K = wt.shape
        M = x.shape[0]
        out = np.empty((M, N), np.uint16)
        self.d.orc_q4_gemv_bf16(x, _c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16), out, M, N, K)
        return out

    def q4_gemv_residual_add(self, x, wt, res) -> np.ndarray:
        x = _c(np.atleast_2d(x), np.uint16)
        N, K = wt.shape
        M = x.shape[0]
        res = _c(np.atleast_2d(res), np.uint16)
        out = np.empty((M, N), np.uint16)
        self.d.orc_q4_gemv_residual_add_bf16(x, _c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16), res, out, M, N, K)
        return out

    def q4_gemv_silu_gate(self, x, gate, up) -> np.ndarray:
        x = _c(np.atleast_2d(x), np.uint16)
        N, K = gate.shape
        M = x.shape[0]
        out = np.empty((M, N), np.uint16)
        self.d.orc_q4_gemv_silu_gate_bf16(x, _c(gate.w, np.uint32), _c(gate.s, np.uint16), _c(gate.b, np.uint16),
                                          _c(up.w, np.uint32), _c(up.s, np.uint16), _c(up.b, np.uint16), out, M, N, K)
        return out

    def q4_argmax_partial(self, x, wt):
        x = _c(np.atleast_2d(x), np.uint16)
        N, K = wt.shape
        M = x.shape[0]
        pv = np.empty((M, N // 8), np.float32)
        pi = np.empty((M, N // 8), np.uint32)
        self.d.orc_q4_gemv_argmax_partial_bf16(x, _c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16), pv, pi, M, N, K)
        return pv, pi

    def argmax_pairs(self, values, indices) -> int:
        v = _c(values, np.float32)
        i = _c(indices, np.uint32)
        return int(self.d.orc_argmax_pairs_f32_u32(v, i, v.size))


_singleton: Oracle | None = None


def oracle() -> Oracle:
    global _singleton
    if _singleton is None:
        _singleton = Oracle()
    return _singleton
