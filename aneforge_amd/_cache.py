"""Content-addressed cache of host weight encodings.

The reference keeps every compiled program (MIL + weight blob) in a content-addressed directory,
sha256 of its inputs, under ANEFORGE_CACHE_DIR (aneforge/_compile.py:898-923), so an identical
model compiles once.  Here kernels are prebuilt and the slow host step is encoding the weights:
per-row int8 (`quantize_per_row`), 32-weight blocks (`quantize_blockwise`), the 16-entry codebook's
Lloyd iterations (`palettize_lut4`) and Q4_0 blocks (`quantize_q4_0`).  With ANEFORGE_CACHE_DIR set,
each encoding is stored under `<dir>/encodings/<key>.npz`, the key being sha256 of the encoder's
name, its parameters and the weight's dtype, shape and bytes, and served from there on the next
load.  Unlike the reference (which always caches, by default under ~/Models/.aneforge-cache), the
cache is off unless the variable is set: a 7B model's codes are several GB of files.
Files are written to a temporary name and renamed, so a reader never sees a partial file; they are
read with numpy's loader without pickles."""
from __future__ import annotations

import hashlib
import os
from pathlib import Path

import numpy as np

_VERSION = "1"          # bump when an encoder's output layout changes


def cache_root() -> Path | None:
    root = os.environ.get("ANEFORGE_CACHE_DIR")
    if not root:
        return None
    p = Path(root) / "encodings"
    p.mkdir(parents=True, exist_ok=True)
    return p


def key(name: str, W: np.ndarray, params: tuple) -> str:
    W = np.ascontiguousarray(W)
    h = hashlib.sha256(f"{_VERSION}|{name}|{W.dtype.str}|{W.shape}|{params!r}".encode())
    h.update(memoryview(W.reshape(-1)).cast("B"))
    return h.hexdigest()[:32]


def cached(name: str, fn, W, *params):
    """fn(W, *params), through the cache when ANEFORGE_CACHE_DIR is set.  fn returns an array or a
    tuple of arrays and Python scalars; the same structure comes back from the cache."""
    root = cache_root()
    if root is None:
        return fn(W, *params)
    W = np.ascontiguousarray(W)
    path = root / f"{key(name, W, params)}.npz"
    if path.is_file():
        try:
            with np.load(path, allow_pickle=False) as z:
                n, single = int(z["n"]), bool(z["single"])
                out = [z[f"a{i}"] for i in range(n)]
                scalar = z["scalar"]
            out = [o.item() if scalar[i] else o for i, o in enumerate(out)]
            return out[0] if single else tuple(out)
        except (OSError, KeyError, ValueError):
            pass                                   # unreadable entry: recompute and replace it
    res = fn(W, *params)
    single = not isinstance(res, tuple)
    items = [res] if single else list(res)
    arrays = {f"a{i}": np.asarray(o) for i, o in enumerate(items)}
    scalar = np.array([not isinstance(o, np.ndarray) for o in items], bool)
    tmp = path.with_name(f"{path.stem}.{os.getpid()}.tmp.npz")
    np.savez(tmp, n=np.int64(len(items)), single=np.bool_(single), scalar=scalar, **arrays)
    os.replace(tmp, path)
    return res
