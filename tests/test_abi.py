"""The C-ABI library loads, exports every prototype declared in include/*.h,
and rejects contract violations on the host before touching a GPU. CPU only
(no compute calls)."""
import ctypes as C
import subprocess

import pytest

from peregrine_amd._lib import LIB_PATH, declared_symbols, lib


def test_headers_declare_entry_points():
    protos = declared_symbols()
    assert len(protos) > 20
    for name in ["prg_q4_gemv_bf16", "prg_argmax_pairs_f32_u32", "prg_hip_alloc_device", "prg_last_error"]:
        assert name in protos


def test_library_exports_every_declared_symbol():
    assert LIB_PATH.exists(), "build the library first (python -m peregrine_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = sorted(set(declared_symbols()) - exported)
    assert not missing, f"declared but not exported: {missing}"
    d = lib.load()
    for name in declared_symbols():
        assert getattr(d, name) is not None


def test_version_and_error_string():
    assert b"gfx950" in lib.prg_version()
    assert isinstance(lib.prg_last_error(), bytes)


@pytest.mark.parametrize("in_dim,out_dim,tokens,code", [
    (100, 8, 1, 1),    # in_dim % 512 != 0
    (512, 12, 1, 1),   # out_dim % 8 != 0
    (512, 8, 0, 7),    # token_count == 0 -> EmptyInput (linear_q4.zig:85)
])
def test_gemv_contract_rejected_on_host(in_dim, out_dim, tokens, code):
    dummy = C.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc = lib.prg_q4_gemv_bf16(None, dummy, dummy, dummy, dummy, dummy, tokens, out_dim, in_dim)
    assert rc == code
    assert lib.prg_last_error()


def test_null_pointer_rejected():
    rc = lib.prg_q4_gemv_bf16(None, None, None, None, None, None, 1, 8, 512)
    assert rc == 1


@pytest.mark.parametrize("x,out_dim,in_dim,tokens,code", [
    (0x1000, 40, 4096, 1, 1),    # out_dim % 16 != 0
    (0x1000, 64, 2048, 1, 1),    # in_dim % 1024 != 0
    (0x1002, 64, 4096, 1, 1),    # x not 16-byte aligned
    (0x1000, 64, 4096, 0, 7),    # token_count == 0 -> EmptyInput (linear_q4.zig:85)
])
def test_decode_layout_gemv_contract_rejected_on_host(x, out_dim, in_dim, tokens, code):
    dummy = C.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc = lib.prg_q4_gemv_t16_bf16(None, C.c_void_p(x), dummy, dummy, dummy, dummy, tokens, out_dim, in_dim)
    assert rc == code
    assert lib.prg_last_error()
