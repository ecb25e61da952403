"""The C-ABI library loads and exports every symbol include/hc.h declares.

CPU only: nothing here launches a kernel.
"""
import ctypes
import os
import re

import pytest

from heterocache_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "hc.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(hc_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_symbols()
    for required in ("hc_decode_attn", "hc_gather_store", "hc_append", "hc_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhc.so not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"symbols declared in hc.h but not exported: {missing}"


def test_python_mirror_matches_header():
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_constants_and_error_reporting_without_gpu():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhc.so not built")
    lib = _lib.load()
    assert lib.hc_version() == 2
    assert lib.hc_tile_tokens() == 32
    assert lib.hc_head_dim() == 128
    # Argument validation happens before any HIP call, so it runs on the CPU.
    rc = lib.hc_decode_attn(2, None, None, None, None, None, None, None, 4, 0, 1.0, None, None, None, None, 0, 1, 4,
                            None, None)
    assert rc == _lib.HC_ERR_INVALID
    assert b"group" in lib.hc_last_error()
    # A fused append without row capacities is refused.
    fake = 16  # never dereferenced: validation fails first
    rc = lib.hc_decode_attn(2, fake, fake, fake, fake, fake, None, None, 4, 4, 1.0, fake, fake, fake, fake, 1 << 20, 4,
                            4, None, None)
    assert rc == _lib.HC_ERR_INVALID
    assert b"row_cap" in lib.hc_last_error()
    assert lib.hc_read_status(None, 1, None, None) == _lib.HC_ERR_INVALID
    rc = lib.hc_gather_store(2, None, None, 0, None, 128, 16, None, None, None, None, None, None, None, 1, 4, None, None,
                             0, None, None)
    assert rc == _lib.HC_ERR_INVALID
    assert b"null pointer" in lib.hc_last_error()
    assert lib.hc_decode_num_parts(None, 1, 4) == -1


def test_num_parts_matches_chunking():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhc.so not built")
    from heterocache_amd import ops
    # chunk_tiles tiles of 32 tokens per part; an empty row still takes one
    # part (it writes the row's zero output).
    assert ops.decode_num_parts([0, 1, 512, 513], chunk_tiles=16) == 1 + 1 + 1 + 2
    assert ops.decode_num_parts([131072], chunk_tiles=32) == 131072 // 1024
    assert ops.decode_num_parts([100, 4097], chunk_tiles=5) == 1 + 26


def test_rounding_flags_are_checked_before_any_launch():
    """hc_decode_attn_stats and hc_score_given_stats take the cast chain's
    rounding flag (HC_SCORE_ROUND_BF16 / _F16, or 0) and refuse any other
    value before a HIP call; hc_stream_read refuses sizes that are not
    16-byte multiples and out-of-range workgroup counts."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhc.so not built")
    lib = _lib.load()
    fake = 16  # never dereferenced: validation fails first
    for bad in (1, 3, _lib.HC_SCORE_ROUND_BF16 | _lib.HC_SCORE_ROUND_F16, _lib.HC_SCORE_SUM_WINDOW):
        rc = lib.hc_decode_attn_stats(2, fake, fake, fake, fake, fake, None, None, 4, 4, 1.0, None, None, fake, fake,
                                      1 << 20, 4, 4, None, 1000, fake, 8, 2, bad, None)
        assert rc == _lib.HC_ERR_INVALID and b"stat_flags" in lib.hc_last_error(), bad
        rc = lib.hc_score_given_stats(2, fake, fake, 640, 128, fake, fake, fake, 2, 1000, 4, 5, bad, 0, 5, 0.088,
                                      fake, fake, fake, None)
        assert rc == _lib.HC_ERR_INVALID and b"flags" in lib.hc_last_error(), bad
    assert lib.hc_stream_read(fake, 24, fake, 8, None) == _lib.HC_ERR_INVALID
    assert lib.hc_stream_read(fake, 4096, fake, 0, None) == _lib.HC_ERR_INVALID
    assert lib.hc_stream_read(None, 4096, fake, 8, None) == _lib.HC_ERR_INVALID
