"""The content-addressed encoding cache (ANEFORGE_CACHE_DIR; the reference's compile cache is
aneforge/_compile.py:898-923): an encoding is stored once and served again without re-running the
encoder, the key follows the weight bytes and the encoder's parameters, and nothing is written
without the variable."""
import numpy as np
import pytest

from aneforge_amd import _blob, _cache
from aneforge_amd import _engine as E


def _w(seed, shape=(64, 128)):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("compress,fn", [("int8", "quantize_per_row"), ("blockwise", "quantize_blockwise"),
                                         ("int4", "palettize_lut4"), ("q4_0", "quantize_q4_0")])
def test_encoding_is_served_from_the_cache(tmp_path, monkeypatch, compress, fn):
    monkeypatch.setenv("ANEFORGE_CACHE_DIR", str(tmp_path))
    W = _w(1)
    first = E.encode(W, compress)
    files = list((tmp_path / "encodings").glob("*.npz"))
    assert len(files) == 1

    def boom(*a, **k):
        raise AssertionError("encoder ran although the cache holds its output")
    monkeypatch.setattr(_blob, fn, boom)
    again = E.encode(W, compress)
    assert again[0] == first[0]
    for a, b in zip(first[1:], again[1:]):
        assert (a is None and b is None) or (a.dtype == b.dtype and np.array_equal(a, b))


def test_key_follows_weights_and_parameters(tmp_path, monkeypatch):
    monkeypatch.setenv("ANEFORGE_CACHE_DIR", str(tmp_path))
    W = _w(2)
    q32, s32, bs32 = _cache.cached("quantize_blockwise", _blob.quantize_blockwise, W, 32)
    q64, s64, bs64 = _cache.cached("quantize_blockwise", _blob.quantize_blockwise, W, 64)
    assert (bs32, bs64) == (32, 64) and isinstance(bs32, int)       # scalars come back as scalars
    W2 = W.copy()
    W2[3, 5] += 1.0
    _cache.cached("quantize_blockwise", _blob.quantize_blockwise, W2, 32)
    assert len(list((tmp_path / "encodings").glob("*.npz"))) == 3
    q, s, bs = _cache.cached("quantize_blockwise", _blob.quantize_blockwise, W, 32)
    ref = _blob.quantize_blockwise(W, 32)
    assert bs == ref[2] and np.array_equal(q, ref[0]) and np.array_equal(s, ref[1])


def test_unreadable_entry_is_recomputed(tmp_path, monkeypatch):
    monkeypatch.setenv("ANEFORGE_CACHE_DIR", str(tmp_path))
    W = _w(3)
    _cache.cached("quantize_per_row", _blob.quantize_per_row, W)
    (f,) = list((tmp_path / "encodings").glob("*.npz"))
    f.write_bytes(b"not an npz")
    q, s = _cache.cached("quantize_per_row", _blob.quantize_per_row, W)
    ref = _blob.quantize_per_row(W)
    assert np.array_equal(q, ref[0]) and np.array_equal(s, ref[1])


def test_no_cache_without_the_variable(tmp_path, monkeypatch):
    monkeypatch.delenv("ANEFORGE_CACHE_DIR", raising=False)
    monkeypatch.chdir(tmp_path)
    E.encode(_w(4), "int8")
    assert _cache.cache_root() is None and not list(tmp_path.rglob("*.npz"))
