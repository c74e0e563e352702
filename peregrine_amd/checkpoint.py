"""Python handle on the checkpoint C ABI (include/peregrine_model.h).

Mirrors the reference's safetensors Repository (src/model/safetensors.zig:17-220)
and config checks (src/model/config.zig:34-73, src/model/mtp.zig:318-345). The
parsing and reading run in libperegrine_hip.so; nothing here needs a GPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import call, lib

_NP_DTYPES = {"U32": np.uint32, "BF16": np.uint16, "F32": np.float32, "F16": np.float16, "U8": np.uint8,
              "I32": np.int32, "I64": np.int64, "U64": np.uint64, "F64": np.float64, "I8": np.int8,
              "U16": np.uint16, "I16": np.int16, "BOOL": np.uint8}


@dataclass
class TensorInfo:
    dtype: str
    shape: tuple[int, ...]
    nbytes: int
    shard: int


class Safetensors:
    """A checkpoint directory of safetensors shards (Repository.open)."""

    def __init__(self, path: str) -> None:
        h = C.c_void_p(0)
        call("prg_safetensors_open", str(path).encode(), C.byref(h))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib.prg_safetensors_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def shards(self) -> list[str]:
        buf = C.create_string_buffer(4096)
        out = []
        for i in range(int(lib.prg_safetensors_shard_count(self.handle))):
            call("prg_safetensors_shard_name", self.handle, i, buf, len(buf))
            out.append(buf.value.decode())
        return out

    def names(self) -> list[str]:
        buf = C.create_string_buffer(4096)
        out = []
        for i in range(int(lib.prg_safetensors_tensor_count(self.handle))):
            call("prg_safetensors_tensor_name", self.handle, i, buf, len(buf))
            out.append(buf.value.decode())
        return out

    def info(self, name: str) -> TensorInfo:
        dt = C.create_string_buffer(16)
        shape = (C.c_uint64 * 8)()
        nd, nb, sh = C.c_uint32(0), C.c_uint64(0), C.c_uint32(0)
        call("prg_safetensors_tensor_info", self.handle, name.encode(), dt, len(dt), shape, 8, C.byref(nd),
             C.byref(nb), C.byref(sh))
        return TensorInfo(dt.value.decode(), tuple(int(shape[k]) for k in range(nd.value)), int(nb.value),
                          int(sh.value))

    def read(self, name: str) -> np.ndarray:
        """Raw bytes of a tensor as a numpy array of its dtype and shape."""
        ti = self.info(name)
        raw = np.empty(ti.nbytes, np.uint8)
        call("prg_safetensors_read", self.handle, name.encode(), raw.ctypes.data_as(C.c_void_p),
             C.c_uint64(ti.nbytes))
        dt = _NP_DTYPES.get(ti.dtype)
        return raw.view(dt).reshape(ti.shape) if dt is not None else raw


def verify_config(path: str) -> None:
    """config.verifyFingerprint: raises PrgError unless the exact 9B checkpoint."""
    call("prg_checkpoint_verify_config", str(path).encode())


def verify_mtp_config(path: str) -> None:
    call("prg_checkpoint_verify_mtp_config", str(path).encode())


def read_config(path: str):
    from .model import ModelConfig, PrgModelConfig

    c = PrgModelConfig()
    call("prg_checkpoint_read_config", str(path).encode(), C.byref(c))
    return ModelConfig(c.num_layers, c.hidden, c.intermediate, c.vocab, c.full_attention_interval, c.rms_eps,
                       c.mtp_layers)
