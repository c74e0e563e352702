"""ctypes binding of libperegrine_hip.so, generated from include/*.h.

The C headers are the single source of truth for the ABI: every
`<ret> prg_<name>(<args>);` prototype is parsed and bound with matching
ctypes argtypes/restype, so the Python layer can never drift from the C ABI.
Loading fails loudly when the library has not been built — there is no
fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
LIB_PATH = PKG / "libperegrine_hip.so"

_SCALARS = {
    "int": C.c_int,
    "unsigned": C.c_uint,
    "uint32_t": C.c_uint32,
    "int32_t": C.c_int32,
    "uint64_t": C.c_uint64,
    "int64_t": C.c_int64,
    "size_t": C.c_size_t,
    "float": C.c_float,
    "double": C.c_double,
    "void": None,
}

class PrgPrefixMatch(C.Structure):
    """struct PrgPrefixMatch (passed by value)."""
    _fields_ = [("index", C.c_uint32), ("len", C.c_uint32)]


# Structs passed by value in the C ABI.
_STRUCTS = {"PrgPrefixMatch": PrgPrefixMatch}

_PROTO = re.compile(r"^\s*([A-Za-z_][\w\s\*]*?)\s*\b(prg_\w+)\s*\(([^;]*?)\)\s*;", re.M | re.S)


def _ctype(decl: str):
    decl = decl.replace("const", " ").strip()
    if "*" in decl:
        base = decl.replace("*", " ").split()
        if base and base[0] == "char" and decl.count("*") == 1:
            return C.c_char_p
        return C.c_void_p
    toks = decl.split()
    if not toks:
        return None
    if toks[0] in _STRUCTS:
        return _STRUCTS[toks[0]]
    return _SCALARS[toks[-1] if toks[-1] in _SCALARS else toks[0]]


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def parse_header(path: Path) -> dict[str, tuple[object, list[object]]]:
    """Return {name: (restype, [argtypes])} for every prg_* prototype."""
    text = _strip_comments(path.read_text())
    out: dict[str, tuple[object, list[object]]] = {}
    for m in _PROTO.finditer(text):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        restype = _ctype(ret)
        argtypes = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name
                mm = re.match(r"^(.*?)([A-Za-z_]\w*)$", a)
                decl = mm.group(1) if mm and mm.group(1).strip() else a
                argtypes.append(_ctype(decl))
        out[name] = (restype, argtypes)
    return out


def declared_symbols() -> dict[str, tuple[object, list[object]]]:
    protos: dict[str, tuple[object, list[object]]] = {}
    for h in sorted(INCLUDE.glob("*.h")):
        protos.update(parse_header(h))
    return protos


class _Lib:
    def __init__(self) -> None:
        self._dll = None
        self.protos = declared_symbols()

    def load(self) -> C.CDLL:
        if self._dll is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m peregrine_amd.build` "
                    "(the HIP path has no fallback)")
            dll = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
            for name, (res, args) in self.protos.items():
                fn = getattr(dll, name)
                fn.restype = res
                fn.argtypes = args
            self._dll = dll
        return self._dll

    def __getattr__(self, name: str):
        if name.startswith("prg_"):
            return getattr(self.load(), name)
        raise AttributeError(name)


lib = _Lib()


class PrgError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str) -> None:
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


def check(fn_name: str, rc: int) -> None:
    if rc != 0:
        msg = lib.prg_last_error()
        raise PrgError(fn_name, rc, msg.decode() if msg else "")


def call(fn_name: str, *args) -> None:
    check(fn_name, getattr(lib, fn_name)(*args))
