"""Python handle on the C++ decode model (include/peregrine_model.h).

Mirrors the reference's DeviceModel / ModelState surface
(src/model/model.zig:538-1662, src/model/state.zig:45-180) for tests and the
benchmark. All compute runs in libperegrine_hip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import call, lib
from .device import init


class PrgModelConfig(C.Structure):
    _fields_ = [("num_layers", C.c_uint32), ("hidden", C.c_uint32), ("intermediate", C.c_uint32),
                ("vocab", C.c_uint32), ("full_attention_interval", C.c_uint32), ("rms_eps", C.c_float),
                ("mtp_layers", C.c_uint32)]


@dataclass
class ModelConfig:
    num_layers: int = 32
    hidden: int = 4096
    intermediate: int = 12288
    vocab: int = 248320
    full_attention_interval: int = 4
    rms_eps: float = 1e-6
    mtp_layers: int = 0  # 1: with the MTP drafter (src/model/mtp.zig)

    def c(self) -> PrgModelConfig:
        return PrgModelConfig(self.num_layers, self.hidden, self.intermediate, self.vocab,
                              self.full_attention_interval, self.rms_eps, self.mtp_layers)

    def is_linear(self, i: int) -> bool:  # decoder_layer.zig:29-31
        return (i + 1) % self.full_attention_interval != 0


QWEN35_9B = ModelConfig()


def _tensor(getter, handle, name: str, dtype) -> tuple[int, int]:
    p = C.c_void_p(0)
    n = C.c_size_t(0)
    call(getter, handle, name.encode(), C.byref(p), C.byref(n))
    return p.value, n.value


def _d2h(ptr: int, nbytes: int, dtype) -> np.ndarray:
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    call("prg_hip_memcpy", out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(nbytes), 1, None, 1)
    return out


class DeviceModel:
    """Random-initialised Qwen3.5-shaped Q4 decoder resident on the GPU."""

    def __init__(self, cfg: ModelConfig = QWEN35_9B, seed: int = 0) -> None:
        init()
        self.cfg = cfg
        h = C.c_void_p(0)
        call("prg_model_create_random", C.byref(cfg.c()), C.c_uint64(seed), C.byref(h))
        self.handle = h

    @classmethod
    def load(cls, cfg: ModelConfig, target_dir: str, mtp_dir: str | None = None) -> "DeviceModel":
        """Upload a model of shape cfg from an MLX safetensors checkpoint
        (DeviceModel.upload, model.zig:580-658)."""
        init()
        self = cls.__new__(cls)
        self.cfg = cfg
        h = C.c_void_p(0)
        self.handle = None
        call("prg_model_load", C.byref(cfg.c()), str(target_dir).encode(),
             str(mtp_dir).encode() if mtp_dir is not None else None, C.byref(h))
        self.handle = h
        return self

    def tensor_names(self) -> list[str]:
        buf = C.create_string_buffer(512)
        out = []
        for i in range(int(lib.prg_model_tensor_count(self.handle))):
            call("prg_model_tensor_name", self.handle, i, buf, len(buf))
            out.append(buf.value.decode())
        return out

    def tensor_info(self, name: str) -> tuple[str, tuple[int, ...]]:
        """Checkpoint dtype string and shape of a tensor."""
        dt = C.create_string_buffer(16)
        shape = (C.c_uint64 * 8)()
        nd = C.c_uint32(0)
        call("prg_model_tensor_info", self.handle, name.encode(), dt, len(dt), shape, 8, C.byref(nd))
        return dt.value.decode(), tuple(int(shape[k]) for k in range(nd.value))

    @property
    def weight_bytes(self) -> int:
        return int(lib.prg_model_weight_bytes(self.handle))

    # block_attn.zig:143-215 prepared dense RHS
    def prepare_dense(self) -> int:
        """Dequantise every prompt-GEMM weight once into a bf16 copy (the
        prefill then stages it as is); returns its size in bytes."""
        call("prg_model_prepare_dense", self.handle)
        return int(lib.prg_model_dense_bytes(self.handle))

    def tensor_ptr(self, name: str) -> tuple[int, int]:
        return _tensor("prg_model_tensor", self.handle, name, None)

    def read(self, name: str, dtype) -> np.ndarray:
        p, n = self.tensor_ptr(name)
        return _d2h(p, n, dtype)

    def write(self, name: str, arr: np.ndarray) -> None:
        """Overwrite a weight tensor with host data of exactly its byte size
        (the prepared dense copy, if any, is not refreshed)."""
        p, n = self.tensor_ptr(name)
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != n:
            raise ValueError(f"{name}: {arr.nbytes} bytes given, the tensor holds {n}")
        call("prg_hip_memcpy", C.c_void_p(p), arr.ctypes.data_as(C.c_void_p), C.c_size_t(n), 0, None, 1)

    def close(self) -> None:
        if self.handle:
            lib.prg_model_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class ModelState:
    """KV caches + GDN states + decode workspace for one sequence."""

    def __init__(self, model: DeviceModel, max_seq: int) -> None:
        self.model = model
        h = C.c_void_p(0)
        call("prg_model_state_create", model.handle, max_seq, C.byref(h))
        self.handle = h
        self.max_seq = max_seq
        self.stride = int(lib.prg_model_state_stride(h))

    def reset(self) -> None:  # state.zig:110-118
        call("prg_model_state_reset", self.handle)

    def read(self, name: str, dtype) -> np.ndarray:
        p, n = _tensor("prg_model_state_tensor", self.handle, name, None)
        return _d2h(p, n, dtype)

    # model.zig:1564-1578
    def forward_next_token(self, token: int, cache_pos: int, rope_pos: int | None = None,
                           seq_len: int | None = None) -> int:
        rope_pos = cache_pos if rope_pos is None else rope_pos
        seq_len = cache_pos + 1 if seq_len is None else seq_len
        out = C.c_uint32(0)
        call("prg_model_forward_next_token", self.model.handle, self.handle, token, cache_pos, rope_pos, seq_len,
             C.byref(out))
        return int(out.value)

    # model.zig:1564-1578 with a prefix (decode_loop.zig:96-160 bookkeeping)
    def forward_next_token_prefixed(self, token: int, cache_pos: int, prefix_len: int, rope_pos: int | None = None,
                                    seq_len: int | None = None) -> int:
        """cache_pos is relative to the prefix (logical_pos - prefix_len); the
        state holds the prefix's tokens in its first prefix_len slots."""
        rope_pos = prefix_len + cache_pos if rope_pos is None else rope_pos
        seq_len = prefix_len + cache_pos + 1 if seq_len is None else seq_len
        out = C.c_uint32(0)
        call("prg_model_forward_next_token_prefixed", self.model.handle, self.handle, token, cache_pos, rope_pos,
             seq_len, prefix_len, C.byref(out))
        return int(out.value)

    def prefill(self, prompt) -> int:
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = C.c_uint32(0)
        call("prg_model_prefill", self.model.handle, self.handle, prompt.ctypes.data_as(C.c_void_p), len(prompt),
             C.byref(out))
        return int(out.value)

    def prefill_from(self, prompt, prefix_len: int) -> int:
        """Prefill prompt[prefix_len:] on top of a state holding prompt[:prefix_len]."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = C.c_uint32(0)
        call("prg_model_prefill_from", self.model.handle, self.handle, prompt.ctypes.data_as(C.c_void_p),
             len(prompt), prefix_len, C.byref(out))
        return int(out.value)

    def copy_prefix_from(self, src: "ModelState", token_count: int) -> None:  # state.zig:124-128
        call("prg_model_state_copy_prefix", self.handle, src.handle, token_count)

    def decode(self, n_steps: int) -> tuple[np.ndarray, float]:
        toks = np.empty(n_steps, np.uint32)
        ms = C.c_float(0.0)
        call("prg_model_decode", self.model.handle, self.handle, n_steps, toks.ctypes.data_as(C.c_void_p),
             C.byref(ms))
        return toks, float(ms.value)

    def time_token_gemvs(self, replays: int = 32) -> float:
        """Average GPU us of one decode token's GEMV launches alone (graph
        replay; measurement only: the state needs a new prefill afterwards)."""
        us = C.c_float(0.0)
        call("prg_model_time_token_gemvs", self.model.handle, self.handle, replays, C.byref(us))
        return float(us.value)

    # decode_loop.zig:96-160 (empty prefix)
    def generate(self, prompt, n_new: int, teacher_force: bool = False) -> tuple[np.ndarray, float]:
        prompt = np.ascontiguousarray(prompt, np.uint32)
        steps = len(prompt) if teacher_force else len(prompt) - 1 + n_new
        preds = np.empty(steps, np.uint32)
        ms = C.c_float(0.0)
        call("prg_model_generate", self.model.handle, self.handle, prompt.ctypes.data_as(C.c_void_p), len(prompt),
             0 if teacher_force else n_new, 1 if teacher_force else 0, preds.ctypes.data_as(C.c_void_p),
             C.byref(ms))
        return preds, float(ms.value)

    # decode_loop.zig:163-293 (device-resident; returns tokens, accepted, attempted, ms)
    def generate_speculative(self, prompt, n_new: int) -> tuple[np.ndarray, int, int, float]:
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_new, np.uint32)
        acc, att, ms = C.c_uint32(0), C.c_uint32(0), C.c_float(0.0)
        call("prg_model_generate_speculative", self.model.handle, self.handle, prompt.ctypes.data_as(C.c_void_p),
             len(prompt), n_new, out.ctypes.data_as(C.c_void_p), C.byref(acc), C.byref(att), C.byref(ms))
        return out, int(acc.value), int(att.value), float(ms.value)

    # decode_loop.zig:163-293 with prefix_len > 0, seedMtpDrafter (server.zig:1240-1330)
    def generate_speculative_from(self, prompt, prefix_len: int, prefix_hidden, n_new: int,
                                  hidden_out=None) -> tuple[np.ndarray, int, int, float]:
        """Speculative generation on top of a state holding prompt[:prefix_len]
        (e.g. restored from a prefix cache entry); prefix_hidden: device bf16
        [prefix_len, hidden] rows of that prefix (None when prefix_len == 0);
        hidden_out: optional device bf16 [len(prompt), hidden] for the prompt's
        hidden rows."""
        from .device import ptr

        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_new, np.uint32)
        acc, att, ms = C.c_uint32(0), C.c_uint32(0), C.c_float(0.0)
        call("prg_model_generate_speculative_from", self.model.handle, self.handle,
             prompt.ctypes.data_as(C.c_void_p), len(prompt), prefix_len, ptr(prefix_hidden), ptr(hidden_out), n_new,
             out.ctypes.data_as(C.c_void_p), C.byref(acc), C.byref(att), C.byref(ms))
        return out, int(acc.value), int(att.value), float(ms.value)

    # model.zig:1627-1659
    def forward_two_tokens(self, t0: int, t1: int, cache_pos: int, hidden_out=None) -> tuple[int, int]:
        v, b = C.c_uint32(0), C.c_uint32(0)
        from .device import ptr

        call("prg_model_forward_two_tokens", self.model.handle, self.handle, t0, t1, cache_pos, cache_pos,
             cache_pos + 1, C.byref(v), C.byref(b), ptr(hidden_out))
        return int(v.value), int(b.value)

    # mtp.zig:187-242
    def mtp_draft(self, token: int, hidden, cache_pos: int) -> int:
        from .device import ptr

        d = C.c_uint32(0)
        call("prg_model_mtp_draft", self.model.handle, self.handle, token, ptr(hidden), cache_pos, cache_pos,
             cache_pos + 1, C.byref(d))
        return int(d.value)

    # mtp.zig:137-185
    def mtp_prefill(self, tokens, hidden_rows, start: int) -> None:
        from .device import ptr

        tokens = np.ascontiguousarray(tokens, np.uint32)
        call("prg_model_mtp_prefill", self.model.handle, self.handle, tokens.ctypes.data_as(C.c_void_p), len(tokens),
             ptr(hidden_rows), start)

    def close(self) -> None:
        if self.handle:
            lib.prg_model_state_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
