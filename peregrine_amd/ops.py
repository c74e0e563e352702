"""Python mirror of the reference's op layer over the C ABI.

`Q4Linear` mirrors the reference's Q4Linear (src/model/linear_q4.zig:17-253):
a resident MLX affine Q4 weight whose encode* methods launch the GEMV family.
Every call goes straight to libperegrine_hip.so; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import call
from .device import DeviceArray, ptr
from .synth import Q4Weight

QMV_FAST_RESULTS_PER_THREADGROUP = 8  # linear_q4.zig:11 (partial = 8 rows)


def _s(stream):
    return C.c_void_p(stream) if stream else None


class Q4Linear:
    """Device-resident Q4 weight. Mirrors Q4Linear (linear_q4.zig:17-63)."""

    def __init__(self, w: DeviceArray, s: DeviceArray, b: DeviceArray) -> None:
        self.weight, self.scales, self.biases = w, s, b
        self.out_dim = w.shape[0]
        self.in_dim = w.shape[1] * 8

    @classmethod
    def upload(cls, q: Q4Weight) -> "Q4Linear":
        return cls(DeviceArray.from_numpy(q.w), DeviceArray.from_numpy(q.s), DeviceArray.from_numpy(q.b))

    @property
    def nbytes(self) -> int:
        return self.weight.nbytes + self.scales.nbytes + self.biases.nbytes

    def _wsb(self):
        return ptr(self.weight), ptr(self.scales), ptr(self.biases)

    # linear_q4.zig:77-95
    def encode_bf16_fast(self, x, y, token_count: int = 1, stream=None) -> None:
        call("prg_q4_gemv_bf16", _s(stream), ptr(x), *self._wsb(), ptr(y), token_count,
             self.out_dim, self.in_dim)

    # linear_q4.zig:149-168
    def encode_bf16_fast_residual_add(self, x, residual, out, token_count: int = 1, stream=None) -> None:
        call("prg_q4_gemv_residual_add_bf16", _s(stream), ptr(x), *self._wsb(), ptr(residual), ptr(out),
             token_count, self.out_dim, self.in_dim)

    # linear_q4.zig:170-194
    def encode_bf16_fast_residual_add2(self, x0, x1, r0, r1, o0, o1, stream=None) -> None:
        call("prg_q4_gemv2_residual_add_bf16", _s(stream), ptr(x0), ptr(x1), *self._wsb(), ptr(r0), ptr(r1),
             ptr(o0), ptr(o1), self.out_dim, self.in_dim)

    # linear_q4.zig:97-118
    def encode_bf16_argmax_partial(self, x, pval, pidx, stream=None) -> None:
        call("prg_q4_gemv_argmax_partial_bf16", _s(stream), ptr(x), *self._wsb(), ptr(pval), ptr(pidx),
             self.out_dim, self.in_dim)

    # linear_q4.zig:120-146
    def encode_bf16_argmax_partial2(self, x0, x1, pv0, pi0, pv1, pi1, stream=None) -> None:
        call("prg_q4_gemv_argmax2_partial_bf16", _s(stream), ptr(x0), ptr(x1), *self._wsb(),
             ptr(pv0), ptr(pi0), ptr(pv1), ptr(pi1), self.out_dim, self.in_dim)

    def dequantize(self, out, stream=None) -> None:
        call("prg_q4_dequantize_bf16", _s(stream), *self._wsb(), ptr(out), self.out_dim, self.in_dim)

    # linear_q4.zig:197-214 (prompt path, MFMA QMM)
    def encode_prefill_qmm(self, x, out, token_count: int, stream=None) -> None:
        call("prg_q4_qmm_bf16", _s(stream), ptr(x), *self._wsb(), ptr(out), token_count, self.out_dim,
             self.in_dim)

    # linear_q4.zig:216-233
    def encode_prefill_qmm_residual_add(self, x, residual, out, token_count: int, stream=None) -> None:
        call("prg_q4_qmm_residual_add_bf16", _s(stream), ptr(x), *self._wsb(), ptr(residual), ptr(out),
             token_count, self.out_dim, self.in_dim)


class DecodeLayoutQ4:
    """A Q4Linear's weight permuted into the decode layout (16-row tiles,
    256-wide K windows; prg_q4_repack_t16), read by the matrix-core GEMV the
    model runs for its decode projections. Same results as Q4Linear's
    encode_bf16_fast (linear_q4.zig:77-95) within the bf16 rounding of a
    different summation order; argmax as encode_bf16_argmax_partial +
    argmax_pairs (linear_q4.zig:97-118, argmax.zig:14-35)."""

    def __init__(self, lin: Q4Linear, stream=None) -> None:
        self.out_dim, self.in_dim = lin.out_dim, lin.in_dim
        self.weight = DeviceArray(lin.weight.shape, np.uint32)
        self.scales = DeviceArray(lin.scales.shape, np.uint16)
        self.biases = DeviceArray(lin.biases.shape, np.uint16)
        call("prg_q4_repack_t16", _s(stream), *lin._wsb(), *self._wsb(), self.out_dim, self.in_dim)

    @property
    def nbytes(self) -> int:
        return self.weight.nbytes + self.scales.nbytes + self.biases.nbytes

    def _wsb(self):
        return ptr(self.weight), ptr(self.scales), ptr(self.biases)

    def encode_bf16_fast(self, x, y, token_count: int = 1, stream=None) -> None:
        call("prg_q4_gemv_t16_bf16", _s(stream), ptr(x), *self._wsb(), ptr(y), token_count, self.out_dim,
             self.in_dim)

    def encode_argmax(self, x, out_index, workspace, token_count: int = 1, stream=None) -> None:
        """out_index[t] = greedy token of row t; workspace holds
        prg_q4_gemv_t16_argmax_workspace_bytes() bytes."""
        call("prg_q4_gemv_t16_argmax_bf16", _s(stream), ptr(x), *self._wsb(), ptr(out_index), token_count,
             self.out_dim, self.in_dim, ptr(workspace))

    def close(self) -> None:
        for a in (self.weight, self.scales, self.biases):
            a.close()


def t16_argmax_workspace_bytes() -> int:
    from ._lib import lib

    return int(lib.prg_q4_gemv_t16_argmax_workspace_bytes())


# block_mlp.zig:313-345 / :347-383
def gate_up_silu(gate: Q4Linear, up: Q4Linear, x, out, stream=None) -> None:
    call("prg_q4_gemv_silu_gate_bf16", _s(stream), ptr(x), *gate._wsb(), *up._wsb(), ptr(out),
         gate.out_dim, gate.in_dim)


def gate_up_silu2(gate: Q4Linear, up: Q4Linear, x0, x1, o0, o1, stream=None) -> None:
    call("prg_q4_gemv_silu_gate2_bf16", _s(stream), ptr(x0), ptr(x1), *gate._wsb(), *up._wsb(), ptr(o0),
         ptr(o1), gate.out_dim, gate.in_dim)


# block_mlp.zig:155-214 (prompt path): gate/up QMMs + silu_mul_pair in one pass
def prefill_gate_up_silu(gate: Q4Linear, up: Q4Linear, x, out, token_count: int, stream=None) -> None:
    call("prg_q4_qmm_silu_gate_bf16", _s(stream), ptr(x), *gate._wsb(), *up._wsb(), ptr(out), token_count,
         gate.out_dim, gate.in_dim)


# argmax.zig:14-35
def argmax_pairs(pval, pidx, out_index, pair_count: int, stream=None) -> None:
    call("prg_argmax_pairs_f32_u32", _s(stream), ptr(pval), ptr(pidx), ptr(out_index), pair_count)


# ------------------------------------------------------------ norms / embed
def rmsnorm(x, w, out, hidden: int, rows: int = 1, eps: float = 1e-6, stream=None) -> None:
    call("prg_rmsnorm_bf16", _s(stream), ptr(x), ptr(w), ptr(out), hidden, rows, eps)


def add_rmsnorm(a, b, w, residual_out, norm_out, hidden: int, rows: int = 1, eps: float = 1e-6,
                stream=None) -> None:
    call("prg_add_rmsnorm_bf16", _s(stream), ptr(a), ptr(b), ptr(w), ptr(residual_out), ptr(norm_out), hidden,
         rows, eps)


def embedding_gather(table: Q4Linear, token: int, out, stream=None) -> None:
    call("prg_q4_embedding_gather_bf16", _s(stream), *table._wsb(), ptr(out), int(token), table.in_dim,
         table.out_dim)


# ----------------------------------------------------------------- GDN ops
def conv1d_silu_decode(state, qkv, w, out, conv_dim: int = 8192, stream=None) -> None:
    call("prg_conv1d_silu_decode_bf16", _s(stream), ptr(state), ptr(qkv), ptr(w), ptr(out), conv_dim, 4)


def gated_delta_decode(state, conv_out, a, b, A_log, dt_bias, y, has_previous_state: bool = True,
                       stream=None) -> None:
    call("prg_gated_delta_decode_bf16", _s(stream), ptr(state), ptr(conv_out), ptr(a), ptr(b), ptr(A_log),
         ptr(dt_bias), ptr(y), 16, 32, 128, 128, 8192, int(bool(has_previous_state)))


def gated_delta_decode_norm(state, conv_out, a, b, A_log, dt_bias, norm_w, z, out, eps: float = 1e-6,
                            has_previous_state: bool = True, stream=None) -> None:
    call("prg_gated_delta_decode_norm_bf16", _s(stream), ptr(state), ptr(conv_out), ptr(a), ptr(b), ptr(A_log),
         ptr(dt_bias), ptr(norm_w), ptr(z), ptr(out), eps, int(bool(has_previous_state)))


def rmsnorm_gated(x, w, gate, out, dim: int = 128, rows: int = 32, eps: float = 1e-6, stream=None) -> None:
    call("prg_rmsnorm_gated_bf16", _s(stream), ptr(x), ptr(w), ptr(gate), ptr(out), dim, eps, rows)


# ----------------------------------------------------------- attention ops
def attn_decode_prepare(packed_q, q_w, q_out, gate, k_in, v_in, k_w, key_cache, value_cache, stride: int,
                        dst: int, pos: int, stream=None) -> None:
    call("prg_attn_decode_prepare_bf16", _s(stream), ptr(packed_q), ptr(q_w), ptr(q_out), ptr(gate), ptr(k_in),
         ptr(v_in), ptr(k_w), ptr(key_cache), ptr(value_cache), stride, dst, pos)


def attn_partials_bytes(stride: int) -> int:
    from ._lib import lib

    return int(lib.prg_attn_decode_partials_bytes(stride))


def attn_decode(q, key_cache, value_cache, gate, out, partials, stride: int, seq_len: int,
                scale: float = 1.0 / 16.0, stream=None) -> None:
    call("prg_attn_decode_bf16", _s(stream), ptr(q), ptr(key_cache), ptr(value_cache), ptr(gate), ptr(out),
         ptr(partials), stride, seq_len, scale)


def attn_step_workspace_bytes(stride: int) -> int:
    from ._lib import lib

    return int(lib.prg_attn_decode_step_workspace_bytes(stride))


# block_attn.zig:321-358 (prepare + partials + merge of one decode step)
def attn_decode_step(packed_q, q_w, k_in, v_in, k_w, key_cache, value_cache, out, workspace, stride: int,
                     cache_pos: int, rope_pos: int, scale: float = 1.0 / 16.0, stream=None) -> None:
    call("prg_attn_decode_step_bf16", _s(stream), ptr(packed_q), ptr(q_w), ptr(k_in), ptr(v_in), ptr(k_w),
         ptr(key_cache), ptr(value_cache), ptr(out), ptr(workspace), stride, cache_pos, rope_pos, scale)


def attn_decode_noalloc(q, key_cache, value_cache, gate, out, stride: int, seq_len: int,
                        scale: float = 1.0 / 16.0, stream=None) -> None:
    call("prg_attn_decode_noalloc_bf16", _s(stream), ptr(q), ptr(key_cache), ptr(value_cache), ptr(gate),
         ptr(out), stride, seq_len, scale)


# ------------------------------------------------------------- prefill ops
def attn_prefill_prepare(packed_q, q_w, k_in, k_w, v_in, q_out, gate_out, key_cache, value_cache,
                         token_count: int, start_rope: int, start_cache: int, stride: int, stream=None) -> None:
    call("prg_attn_prefill_prepare_bf16", _s(stream), ptr(packed_q), ptr(q_w), ptr(k_in), ptr(k_w), ptr(v_in),
         ptr(q_out), ptr(gate_out), ptr(key_cache), ptr(value_cache), token_count, start_rope, start_cache, stride)


def attn_prefill_scores_bytes(token_count: int, prefix: int) -> int:
    from ._lib import lib

    return int(lib.prg_attn_prefill_scores_bytes(token_count, prefix))


def attn_prefill(q, key_cache, value_cache, gate, out, scores, token_count: int, prefix: int, stride: int,
                 scale: float = 1.0 / 16.0, stream=None) -> None:
    call("prg_attn_prefill_bf16", _s(stream), ptr(q), ptr(key_cache), ptr(value_cache), ptr(gate), ptr(out),
         ptr(scores), token_count, prefix, stride, scale)


def conv1d_silu_prefill(state, qkv, w, out, token_count: int, has_previous_state: bool = True,
                        stream=None) -> None:
    call("prg_conv1d_silu_prefill_bf16", _s(stream), ptr(state), ptr(qkv), ptr(w), ptr(out), token_count, 8192,
         4, int(bool(has_previous_state)))


def gated_delta_prefill_prepare(conv_out, a, b, A_log, dt_bias, q_out, k_out, g_out, beta_out,
                                token_count: int, kq_out=None, stream=None) -> None:
    call("prg_gated_delta_prefill_prepare_bf16", _s(stream), ptr(conv_out), ptr(a), ptr(b), ptr(A_log),
         ptr(dt_bias), ptr(q_out), ptr(k_out), ptr(g_out), ptr(beta_out),
         None if kq_out is None else ptr(kq_out), token_count)


def gated_delta_prefill(state, q, k, conv_out, g, beta, y, token_count: int, has_previous_state: bool = True,
                        stream=None) -> None:
    call("prg_gated_delta_prefill_bf16", _s(stream), ptr(state), ptr(q), ptr(k), ptr(conv_out), ptr(g),
         ptr(beta), ptr(y), token_count, int(bool(has_previous_state)))
