"""Build recipe of ``libffn_mi355x.so`` for gfx950 (MI355X).

The library is compiled ahead of time, in-tree, with ``hipcc``: one object per
(storage type, tile variant) pair from ``csrc/ffn_kernels.hip``, one per (storage
type, single-launch tile pair) from ``csrc/ffn_fused.hip``, plus the host object
``csrc/ffn_mi355x.hip``, linked into ``ffn_optim_amd/libffn_mi355x.so``.
It replaces the reference's just-in-time ``tla.compile`` of ``ops/kernel/ffn.py``
(ops/host/dispatch.py:97-116).

Run ``python -m ffn_optim_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
REPO = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = REPO / "_build"
LIBRARY = PACKAGE / "libffn_mi355x.so"
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 are generated from scalar float code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError(f"hipcc not found ({path}); the HIP library cannot be built")
    return path


def variant_ids() -> list[int]:
    text = (CSRC / "ffn_variants.hpp").read_text()
    ids = [int(m) for m in re.findall(r"^\s*X\((\d+),", text, re.M)]
    if not ids:
        raise RuntimeError("no tile variants found in ffn_variants.hpp")
    return ids


def fused_pairs() -> list[tuple[int, int]]:
    """(up, down) variant pairs compiled as a single-launch FFN (FFN_FUSED_PAIRS)."""
    text = (CSRC / "ffn_variants.hpp").read_text()
    m = re.search(r"^#define FFN_FUSED_PAIRS\(X\)(.*)$", text, re.M)
    return [(int(a), int(b)) for a, b in re.findall(r"X\((\d+),\s*(\d+)\)", m.group(1))] if m else []


def source_revision() -> str:
    digest = hashlib.sha256()
    for path in sorted(CSRC.glob("*")) + sorted(INCLUDE.glob("*.h")):
        digest.update(path.name.encode())
        digest.update(path.read_bytes())
    return digest.hexdigest()[:16]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(map(str, cmd)), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(map(str, cmd))}\n"
                           f"{proc.stdout}\n{proc.stderr}")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every kernel object and link the library; returns its path."""
    cc = hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    rev = source_revision()
    inc = ["-I", str(CSRC), "-I", str(INCLUDE)]
    units = []
    for dt in (0, 1):
        for vid in variant_ids():
            obj = BUILD_DIR / f"ffn_kernels_d{dt}_v{vid}.o"
            units.append([cc, *DEVICE_FLAGS, *inc, f"-DFFN_DT={dt}", f"-DFFN_VARIANT={vid}",
                          "-c", str(CSRC / "ffn_kernels.hip"), "-o", str(obj)])
        for up, down in fused_pairs():
            obj = BUILD_DIR / f"ffn_fused_d{dt}_u{up}_n{down}.o"
            units.append([cc, *DEVICE_FLAGS, *inc, f"-DFFN_DT={dt}", f"-DFFN_UPV={up}", f"-DFFN_DNV={down}",
                          "-c", str(CSRC / "ffn_fused.hip"), "-o", str(obj)])
    host_obj = BUILD_DIR / "ffn_mi355x.o"
    units.append([cc, *DEVICE_FLAGS, *inc, f'-DFFN_MI355X_REVISION="{rev}"',
                  "-c", str(CSRC / "ffn_mi355x.hip"), "-o", str(host_obj)])
    jobs = jobs or min(16, os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, u, verbose) for u in units]:
            fut.result()
    objects = [u[u.index("-o") + 1] for u in units]
    tmp = LIBRARY.with_name(LIBRARY.name + ".tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objects], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
