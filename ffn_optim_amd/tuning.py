"""Measured tile choices: a table from problem key to (up variant, down variant).

The library's planner picks tile variants from a cost model; the search harness
(``python -m ffn_optim_amd.performance.run --mode tune --execute-gpu``) times every
applicable variant pair on the device and can record the fastest in
``configs/tuned_plans.json``.  ``prepare_ffn`` consults that table when the caller
forces no variant, so measured choices win over modelled ones for the shapes that
were tuned, and every other shape falls back to the planner.

A key is the padded problem plus everything that changes which kernels run:
(m, mp, kp, hp, np, dtype, down_impl, gelu, block_num).
"""
from __future__ import annotations

import json
import threading
from pathlib import Path

TABLE_PATH = Path(__file__).resolve().parent / "configs" / "tuned_plans.json"
SCHEMA_VERSION = 1
KEY_FIELDS = ("m", "mp", "kp", "hp", "np", "dtype", "down_impl", "gelu", "block_num")

_lock = threading.Lock()
_cache: dict[Path, dict] = {}


def make_key(m, mp, kp, hp, np_, dtype, down_impl, gelu, block_num) -> dict:
    """Key of one planned FFN: logical rows, padded extents, storage type name
    ('float16'/'bfloat16'), down implementation, GELU form and workgroup count."""
    return {"m": int(m), "mp": int(mp), "kp": int(kp), "hp": int(hp), "np": int(np_),
            "dtype": str(dtype), "down_impl": str(down_impl), "gelu": str(gelu),
            "block_num": int(block_num)}


def _key_tuple(key: dict) -> tuple:
    missing = [f for f in KEY_FIELDS if f not in key]
    if missing:
        raise ValueError(f"tuning key lacks {missing}")
    return tuple(key[f] for f in KEY_FIELDS)


def load(path: Path | str | None = None) -> dict:
    """{key tuple: entry} of a table file; an absent file is an empty table."""
    path = Path(path or TABLE_PATH)
    with _lock:
        mtime = path.stat().st_mtime if path.exists() else None
        cached = _cache.get(path)
        if cached is not None and cached["mtime"] == mtime:
            return cached["entries"]
        entries = {}
        if mtime is not None:
            data = json.loads(path.read_text())
            if data.get("schema_version") != SCHEMA_VERSION:
                raise ValueError(f"{path}: expected schema_version {SCHEMA_VERSION}")
            for entry in data.get("entries", []):
                for field in ("up_variant", "down_variant"):
                    if type(entry.get(field)) is not int or entry[field] < 0:
                        raise ValueError(f"{path}: {field} must be a non-negative integer")
                entries[_key_tuple(entry["key"])] = entry
        _cache[path] = {"mtime": mtime, "entries": entries}
        return entries


def lookup(key: dict, path: Path | str | None = None):
    """(up_variant, down_variant) recorded for key, or None."""
    entry = load(path).get(_key_tuple(key))
    if entry is None:
        return None
    return entry["up_variant"], entry["down_variant"]


def record(key: dict, up_variant: int, down_variant: int, *, device_median_us=None, source=None,
           path: Path | str | None = None) -> None:
    """Insert or replace the entry for key and rewrite the table atomically."""
    path = Path(path or TABLE_PATH)
    entries = dict(load(path))
    entries[_key_tuple(key)] = {"key": dict(key), "up_variant": int(up_variant),
                                "down_variant": int(down_variant),
                                "device_median_us": device_median_us, "source": source}
    data = {"schema_version": SCHEMA_VERSION,
            "description": "Fastest measured (up, down) tile variants per problem on gfx950; "
                           "written by ffn_optim_amd.performance.run --mode tune --write-tuned",
            "entries": sorted(entries.values(), key=lambda e: _key_tuple(e["key"]))}
    tmp = path.with_suffix(path.suffix + ".tmp")
    tmp.write_text(json.dumps(data, indent=1) + "\n")
    tmp.replace(path)
    with _lock:
        _cache.pop(path, None)
