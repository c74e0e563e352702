"""Python handle on the prompt-prefix cache and its PRGPFXS1 file
(include/peregrine_model.h; reference src/server/prefix_state_cache.zig,
src/server/prefix_persist.zig). All logic runs in libperegrine_hip.so."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import PrgPrefixMatch, call, lib


class PrgPrefixCacheStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("hits", "misses", "hit_tokens", "computed_tokens", "reserved_tokens",
                                           "resident_tokens", "max_tokens", "entry_count", "evictions")]


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.uint32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class PrefixCache:
    """Cache.init(max_cache_tokens, prefill_chunk_tokens); model=None keeps
    tokens and accounting only."""

    def __init__(self, model, max_tokens: int, prefill_chunk_tokens: int) -> None:
        h = C.c_void_p(0)
        call("prg_prefix_cache_create", model.handle if model is not None else None, max_tokens,
             prefill_chunk_tokens, C.byref(h))
        self.handle = h
        self.model = model

    def close(self) -> None:
        if self.handle:
            lib.prg_prefix_cache_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    # -- queries ---------------------------------------------------------
    def entry_count(self) -> int:
        return int(lib.prg_prefix_cache_entry_count(self.handle))

    def pinned_count(self) -> int:
        return int(lib.prg_prefix_cache_pinned_count(self.handle))

    def active_tokens(self) -> int:
        return int(lib.prg_prefix_cache_active_tokens(self.handle))

    def stats(self) -> dict:
        s = PrgPrefixCacheStats()
        call("prg_prefix_cache_stats", self.handle, C.byref(s))
        return {n: int(getattr(s, n)) for n, _ in s._fields_}

    def find(self, prompt) -> PrgPrefixMatch | None:
        p = _u32(prompt)
        m = PrgPrefixMatch()
        call("prg_prefix_cache_find", self.handle, _ptr(p), len(p), C.byref(m))
        return m if m.len else None

    def contains(self, prompt, prefix_len: int) -> bool:
        p = _u32(prompt)
        return bool(lib.prg_prefix_cache_contains(self.handle, _ptr(p), len(p), prefix_len))

    def cached_next_token(self, m: PrgPrefixMatch) -> tuple[int, bool]:
        t, v = C.c_uint32(0), C.c_int(0)
        call("prg_prefix_cache_cached_next_token", self.handle, m, C.byref(t), C.byref(v))
        return int(t.value), bool(v.value)

    def entry_info(self, index: int) -> dict:
        n, cap, pin, hits = C.c_uint32(0), C.c_uint32(0), C.c_int(0), C.c_uint64(0)
        call("prg_prefix_cache_entry_info", self.handle, index, C.byref(n), C.byref(cap), C.byref(pin),
             C.byref(hits))
        return {"tokens": n.value, "capacity": cap.value, "pinned": bool(pin.value), "hits": hits.value}

    def entry_tokens(self, index: int) -> np.ndarray:
        n = self.entry_info(index)["tokens"]
        out = np.empty(n, np.uint32)
        call("prg_prefix_cache_entry_tokens", self.handle, index, _ptr(out), n)
        return out

    def entry_state_handle(self, index: int) -> C.c_void_p:
        h = C.c_void_p(0)
        call("prg_prefix_cache_entry_state", self.handle, index, C.byref(h))
        return h

    # -- mutators ----------------------------------------------------------
    def touch(self, m: PrgPrefixMatch) -> None:
        call("prg_prefix_cache_touch", self.handle, m)

    def remove(self, index: int) -> None:
        call("prg_prefix_cache_remove", self.handle, index)

    def clear(self) -> None:
        call("prg_prefix_cache_clear", self.handle)

    def record_hit(self, reused: int) -> None:
        lib.prg_prefix_cache_record_hit(self.handle, reused)

    def record_miss(self) -> None:
        lib.prg_prefix_cache_record_miss(self.handle)

    def record_computed(self, n: int) -> None:
        lib.prg_prefix_cache_record_computed(self.handle, n)

    def start_direct(self, ids, pinned: bool = False) -> PrgPrefixMatch:
        p = _u32(ids)
        m = PrgPrefixMatch()
        call("prg_prefix_cache_start_direct", self.handle, _ptr(p), len(p), int(pinned), C.byref(m))
        return m

    def finish_direct(self, m: PrgPrefixMatch, next_token: int) -> None:
        call("prg_prefix_cache_finish_direct", self.handle, m, next_token)

    def store(self, ids, work=None, reuse: PrgPrefixMatch | None = None, next_token: int | None = None,
              pinned: bool = False, work_hidden: int | None = None, hidden_base_rows: int = 0) -> PrgPrefixMatch:
        """storePrefixFromWork. work: a ModelState (or None without a model);
        work_hidden: device pointer of bf16 hidden rows."""
        p = _u32(ids)
        m = PrgPrefixMatch()
        nt = C.c_uint32(next_token) if next_token is not None else None
        call("prg_prefix_cache_store", self.handle, _ptr(p), len(p), C.byref(reuse) if reuse is not None else None,
             work.handle if work is not None else None, C.c_void_p(work_hidden) if work_hidden else None,
             hidden_base_rows, C.byref(nt) if nt is not None else None, int(pinned), C.byref(m))
        return m

    def restore(self, m: PrgPrefixMatch, work) -> None:
        call("prg_prefix_cache_restore", self.handle, m, work.handle)

    def enable_hidden(self) -> None:
        call("prg_prefix_cache_enable_hidden", self.handle)

    def entry_hidden(self, m: PrgPrefixMatch) -> tuple[int, bool]:
        p, v = C.c_void_p(0), C.c_int(0)
        call("prg_prefix_cache_entry_hidden", self.handle, m, C.byref(p), C.byref(v))
        return (p.value or 0), bool(v.value)

    def set_entry_hidden(self, m: PrgPrefixMatch, rows_ptr: int) -> None:
        call("prg_prefix_cache_set_entry_hidden", self.handle, m, C.c_void_p(rows_ptr))

    # -- persistence (PRGPFXS1 v3) ---------------------------------------
    def save(self, path: str, fingerprint: int) -> None:
        call("prg_prefix_cache_save", self.handle, str(path).encode(), C.c_uint64(fingerprint))

    def load(self, path: str, fingerprint: int) -> int:
        n = C.c_uint32(0)
        call("prg_prefix_cache_load", self.handle, str(path).encode(), C.c_uint64(fingerprint), C.byref(n))
        return int(n.value)


def model_fingerprint(model_dir: str) -> int:
    out = C.c_uint64(0)
    call("prg_model_fingerprint", str(model_dir).encode(), C.byref(out))
    return int(out.value)


def wyhash(data: bytes, seed: int) -> int:
    out = C.c_uint64(0)
    buf = C.create_string_buffer(data, len(data)) if data else None
    call("prg_wyhash", buf, C.c_size_t(len(data)), C.c_uint64(seed), C.byref(out))
    return int(out.value)


def file_bytes(cfg, token_count: int) -> int:
    out = C.c_uint64(0)
    call("prg_prefix_state_file_bytes", C.byref(cfg.c()), C.c_uint64(token_count), C.byref(out))
    return int(out.value)


def default_path() -> str:
    buf = C.create_string_buffer(4096)
    call("prg_prefix_state_default_path", buf, len(buf))
    return buf.value.decode()
