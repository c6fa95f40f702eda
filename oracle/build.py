"""Build recipe of the C oracle (test infrastructure only): oracle/libffn_ref.so.

    gcc -O2 -shared -fPIC oracle/ffn_ref.c -lm -o oracle/libffn_ref.so

There is no C/C++ reference implementation to build: the reference's golden
path is Python (validation/reference.py), so oracle/_ref/ stays empty.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

ORACLE = Path(__file__).resolve().parent
SOURCE = ORACLE / "ffn_ref.c"
LIBRARY = ORACLE / "libffn_ref.so"


def build() -> Path:
    tmp = LIBRARY.with_name(LIBRARY.name + ".tmp")
    subprocess.run(["gcc", "-O2", "-std=c11", "-shared", "-fPIC", str(SOURCE), "-lm", "-o", str(tmp)],
                   check=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


def load():
    import ctypes
    if not LIBRARY.exists():
        build()
    lib = ctypes.CDLL(str(LIBRARY))
    f, i, sz = ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_size_t
    lib.ffn_ref_run.argtypes = [f, f, f, f, f, i, i, i, i, i, i]
    lib.ffn_ref_run.restype = None
    lib.ffn_ref_round.argtypes = [f, f, sz, i]
    lib.ffn_ref_round.restype = None
    lib.ffn_ref_gelu_rational.argtypes = [ctypes.c_float]
    lib.ffn_ref_gelu_rational.restype = ctypes.c_float
    lib.ffn_ref_gelu_erf.argtypes = [ctypes.c_double]
    lib.ffn_ref_gelu_erf.restype = ctypes.c_double
    return lib


if __name__ == "__main__":
    print(build())
