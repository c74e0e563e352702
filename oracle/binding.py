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
        _f = C.c_float
        d.orc_rmsnorm_bf16.argtypes = [_u16p, _u16p, _u16p, _u32, _u32, _f]
        d.orc_add_rmsnorm_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _u32, _u32, _f]
        d.orc_q4_embedding_gather_bf16.argtypes = [_u32p, _u16p, _u16p, _u16p, _u32, _u32]
        d.orc_conv1d_silu_decode_bf16.argtypes = [_f32p, _u16p, _u16p, _u16p, _u32, _u32]
        d.orc_gated_delta_decode_bf16.argtypes = [_f32p, _u16p, _u16p, _u16p, _f32p, _u16p, _u16p,
                                                  _u32, _u32, _u32, _u32, _u32]
        d.orc_rmsnorm_gated_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, _u32, _f, _u32]
        d.orc_attn_decode_prepare_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p,
                                                   _u16p, _u32, _u32, _u32, _u32, _u32, _f, _u32, _u32]
        d.orc_attn_decode_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _u32, _u32, _u32, _u32, _f]
        _vp = C.c_void_p
        d.orc_q4_qmm_bf16.argtypes = [_u16p, _u32, _u32p, _u16p, _u16p, _vp, _u16p, _u32, _u32]
        d.orc_silu_mul_pair_bf16.argtypes = [_u16p, _u16p, C.c_size_t]
        d.orc_sigmoid_mul_pair_bf16.argtypes = [_u16p, _u16p, C.c_size_t]
        d.orc_q4_embedding_gather_many_bf16.argtypes = [_u32p, _u16p, _u16p, _u32p, _u32, _u16p, _u32]
        d.orc_split_qg_many_bf16.argtypes = [_u16p, _u16p, _u16p, _u32, _u32, _u32]
        d.orc_qk_norm_rope_append_many_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p,
                                                        _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _f]
        d.orc_attn_prefill_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, _u32, _u32, _u32, _u32, _u32, _u32, _f]
        d.orc_conv1d_silu_prefill_bf16.argtypes = [_f32p, _u16p, _u16p, _u16p, _u32, _u32, _u32, _u32]
        d.orc_qk_l2norm_prefill_bf16.argtypes = [_u16p, _f32p, _f32p, _u32, _u32, _u32, _u32]
        d.orc_gating_many_bf16.argtypes = [_f32p, _u16p, _u16p, _u16p, _f32p, _f32p, _u32, _u32]
        d.orc_gated_delta_prefill_bf16.argtypes = [_f32p, _f32p, _f32p, _u16p, _f32p, _f32p, _u16p,
                                                   _u32, _u32, _u32, _u32, _u32, _u32, _u32]

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

    # ------------------------------------------------------ norms / embed
    def rmsnorm(self, x, w, eps=1e-6) -> np.ndarray:
        x = _c(np.atleast_2d(x), np.uint16)
        out = np.empty_like(x)
        self.d.orc_rmsnorm_bf16(x, _c(w, np.uint16), out, x.shape[1], x.shape[0], eps)
        return out

    def add_rmsnorm(self, a, b, w, eps=1e-6):
        a = _c(np.atleast_2d(a), np.uint16)
        b = _c(np.atleast_2d(b), np.uint16)
        r = np.empty_like(a)
        n = np.empty_like(a)
        self.d.orc_add_rmsnorm_bf16(a, b, _c(w, np.uint16), r, n, a.shape[1], a.shape[0], eps)
        return r, n

    def embedding(self, wt, token: int) -> np.ndarray:
        V, H = wt.shape
        out = np.empty(H, np.uint16)
        self.d.orc_q4_embedding_gather_bf16(_c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16), out,
                                            int(token), H)
        return out

    # ---------------------------------------------------------------- GDN
    def conv1d_decode(self, state, qkv, w):
        """Returns (out, new_state); state is not modified."""
        st = np.array(state, np.float32, copy=True, order="C")
        qkv = _c(qkv, np.uint16)
        out = np.empty_like(qkv)
        self.d.orc_conv1d_silu_decode_bf16(st, qkv, _c(w, np.uint16), out, qkv.size, 4)
        return out, st

    def gated_delta_decode(self, state, conv_out, a, b, A_log, dt_bias, has_prev=True,
                           Hk=16, Hv=32, Dk=128, Dv=128):
        st = np.array(state, np.float32, copy=True, order="C")
        y = np.empty(Hv * Dv, np.uint16)
        self.d.orc_gated_delta_decode_bf16(st, _c(conv_out, np.uint16), _c(a, np.uint16), _c(b, np.uint16),
                                           _c(A_log, np.float32), _c(dt_bias, np.uint16), y, Hk, Hv, Dk, Dv,
                                           int(bool(has_prev)))
        return y, st

    def rmsnorm_gated(self, x, w, gate, dim, eps=1e-6):
        x = _c(x, np.uint16)
        out = np.empty_like(x)
        self.d.orc_rmsnorm_gated_bf16(x, _c(w, np.uint16), _c(gate, np.uint16), out, dim, eps, x.size // dim)
        return out

    # ---------------------------------------------------------- attention
    def attn_prepare(self, packed_q, q_w, k_in, v_in, k_w, key_cache, value_cache, stride, dst, pos,
                     theta=1.0e7):
        """Returns (q_out, gate, key_cache', value_cache') — caches are copied."""
        kc = np.array(key_cache, np.uint16, copy=True, order="C")
        vc = np.array(value_cache, np.uint16, copy=True, order="C")
        q_out = np.empty(16 * 256, np.uint16)
        gate = np.empty(16 * 256, np.uint16)
        self.d.orc_attn_decode_prepare_bf16(_c(packed_q, np.uint16), _c(q_w, np.uint16), q_out, gate,
                                            _c(k_in, np.uint16), _c(v_in, np.uint16), _c(k_w, np.uint16), kc, vc,
                                            16, 4, 256, 64, int(pos), theta, int(stride), int(dst))
        return q_out, gate, kc, vc

    def attn_decode(self, q, key_cache, value_cache, gate, stride, seq_len, scale=1.0 / 16.0):
        out = np.empty(16 * 256, np.uint16)
        self.d.orc_attn_decode_bf16(_c(q, np.uint16), _c(key_cache, np.uint16), _c(value_cache, np.uint16),
                                    _c(gate, np.uint16), out, 16, 4, int(stride), int(seq_len), scale)
        return out


    # ------------------------------------------------------------ prefill
    def q4_qmm(self, x, wt, residual=None) -> np.ndarray:
        """[M, K] x Q4 [N, K]^T -> bf16 [M, N] with bf16-rounded weights."""
        x = _c(np.atleast_2d(x), np.uint16)
        N, K = wt.shape
        M = x.shape[0]
        out = np.empty((M, N), np.uint16)
        res = None
        if residual is not None:
            res = _c(np.reshape(residual, (M, N)), np.uint16)
        self.d.orc_q4_qmm_bf16(x, M, _c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16),
                               None if res is None else res.ctypes.data, out, N, K)
        return out

    def silu_mul_pair(self, gate, up) -> np.ndarray:
        g = np.array(gate, np.uint16, copy=True, order="C")
        self.d.orc_silu_mul_pair_bf16(g, _c(up, np.uint16), g.size)
        return g

    def sigmoid_mul_pair(self, x, gate) -> np.ndarray:
        y = np.array(x, np.uint16, copy=True, order="C")
        self.d.orc_sigmoid_mul_pair_bf16(y, _c(gate, np.uint16), y.size)
        return y

    def embedding_many(self, wt, tokens) -> np.ndarray:
        V, H = wt.shape
        tok = _c(tokens, np.uint32)
        out = np.empty((tok.size, H), np.uint16)
        self.d.orc_q4_embedding_gather_many_bf16(_c(wt.w, np.uint32), _c(wt.s, np.uint16), _c(wt.b, np.uint16),
                                                 tok, tok.size, out, H)
        return out

    def split_qg_many(self, qp, heads=16, head_dim=256):
        qp = _c(qp, np.uint16)
        T = qp.size // (heads * 2 * head_dim)
        q = np.empty((T, heads * head_dim), np.uint16)
        g = np.empty_like(q)
        self.d.orc_split_qg_many_bf16(qp, q, g, head_dim, heads, T)
        return q, g

    def qk_norm_rope_append_many(self, q, q_w, k, k_w, v, key_cache, value_cache, start_rope, start_cache,
                                 stride, theta=1.0e7):
        """Returns (q', key_cache', value_cache'); inputs are not modified."""
        qq = np.array(q, np.uint16, copy=True, order="C")
        kc = np.array(key_cache, np.uint16, copy=True, order="C")
        vc = np.array(value_cache, np.uint16, copy=True, order="C")
        T = qq.size // (16 * 256)
        self.d.orc_qk_norm_rope_append_many_bf16(qq, _c(q_w, np.uint16), _c(k, np.uint16), _c(k_w, np.uint16),
                                                 _c(v, np.uint16), kc, vc, int(start_rope), T, int(start_cache),
                                                 int(stride), 16, 4, 256, 64, theta)
        return qq, kc, vc

    def attn_prefill(self, q, key_cache, value_cache, T, prefix, stride, scale=1.0 / 16.0):
        out = np.empty((T, 16 * 256), np.uint16)
        self.d.orc_attn_prefill_bf16(_c(q, np.uint16), _c(key_cache, np.uint16), _c(value_cache, np.uint16), out,
                                     int(T), int(prefix), int(stride), 16, 4, 256, scale)
        return out

    def conv1d_prefill(self, state, qkv, w, has_prev=True):
        """qkv [T, conv_dim] -> (out [T, conv_dim], new_state)."""
        st = np.array(state, np.float32, copy=True, order="C")
        qkv = _c(np.atleast_2d(qkv), np.uint16)
        T, cd = qkv.shape
        out = np.empty_like(qkv)
        self.d.orc_conv1d_silu_prefill_bf16(st, qkv, _c(w, np.uint16), out, T, cd, 4, int(bool(has_prev)))
        return out, st

    def qk_l2norm_prefill(self, conv_out, Hk=16, Dk=128):
        co = _c(np.atleast_2d(conv_out), np.uint16)
        T, cd = co.shape
        qn = np.empty((T, Hk * Dk), np.float32)
        kn = np.empty_like(qn)
        self.d.orc_qk_l2norm_prefill_bf16(co, qn, kn, T, Hk, Dk, cd)
        return qn, kn

    def gating_many(self, A_log, a, dt_bias, b, Hv=32):
        a = _c(np.atleast_2d(a), np.uint16)
        T = a.shape[0]
        g = np.empty((T, Hv), np.float32)
        beta = np.empty_like(g)
        self.d.orc_gating_many_bf16(_c(A_log, np.float32), a, _c(dt_bias, np.uint16), _c(b, np.uint16), g, beta,
                                    Hv, T)
        return g, beta

    def gated_delta_prefill(self, state, qn, kn, conv_out, g, beta, has_prev=True, Hk=16, Hv=32, Dk=128, Dv=128):
        st = np.array(state, np.float32, copy=True, order="C")
        co = _c(np.atleast_2d(conv_out), np.uint16)
        T, cd = co.shape
        y = np.empty((T, Hv * Dv), np.uint16)
        self.d.orc_gated_delta_prefill_bf16(st, _c(qn, np.float32), _c(kn, np.float32), co, _c(g, np.float32),
                                            _c(beta, np.float32), y, T, Hk, Hv, Dk, Dv, cd, int(bool(has_prev)))
        return y, st


_singleton: Oracle | None = None


def oracle() -> Oracle:
    global _singleton
    if _singleton is None:
        _singleton = Oracle()
    return _singleton
