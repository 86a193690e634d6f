"""The C ABI library loads and exports every entry point include/*.h declares
(no compute: this runs on machines without a GPU)."""
import ctypes
import glob
import os
import re

from gomlx_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(ghip_\w+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    for n in ["ghip_softmax_rows", "ghip_rmsnorm_rows", "ghip_layernorm_rows",
              "ghip_gemm_batched", "ghip_gather_rows", "ghip_argminmax", "ghip_iota"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"


def test_python_signatures_cover_header():
    # Every declared entry point has a ctypes signature, so no call goes untyped.
    from gomlx_hip import backend
    sigs = set(_lib.SIGNATURES) | set(_lib.SIGNATURES_I64) | set(backend._GRAPH_SIGS) | {"ghip_version",
                                                                                          "ghip_error_clear"}
    extra = declared_symbols() - sigs
    assert not extra, f"no ctypes signature for {sorted(extra)}"


def test_version_string():
    assert b"gfx950" in _lib.load().ghip_version()


def test_error_path_without_gpu():
    # Argument validation happens on the host before any HIP call.
    import pytest
    with pytest.raises(_lib.BackendError) as ei:
        _lib.call("ghip_gemm_batched", _lib.DT_FLOAT32, _lib.DT_FLOAT32, 1, 4, 4, 4,
                  None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 2, None)
    assert ei.value.code == 1 and "sc_n" in str(ei.value)
    with pytest.raises(_lib.BackendError) as ei:
        _lib.call("ghip_softmax_rows", 99, None, None, 4, 4, 0, None)
    assert ei.value.code in (1, 2)


def test_sdpa_workspace_policy():
    """Host-side policy of the split key range (no GPU call): a workspace only for
    16-bit grids of few workgroups with at least 8 key tiles, its size covering
    every split's partial rows (D + 1 floats a row).  Without a causal mask,
    grouped-query heads of one kv head share workgroups when Sq < 128 (decoding):
    B8 H32 Hkv8 Sq1 is 64 workgroups, so 12 splits.  Grids of several row blocks
    per (b, h) split only with 64 key tiles or more (counted to the causal bound)."""
    L = _lib.load()
    ws = L.ghip_sdpa_workspace_bytes
    BF16, F32 = _lib.DT_BFLOAT16, _lib.DT_FLOAT32
    assert ws(BF16, 8, 32, 8, 1, 8192, 128, 0) == 12 * 8 * 32 * 1 * 129 * 4
    assert ws(BF16, 8, 32, 8, 1, 8192, 128, 1) == 0        # causal, one query: it sees key 0 only
    assert ws(BF16, 1, 16, 16, 2048, 2048, 128, 0) == 0    # prefill, 32 key tiles: no split
    assert ws(BF16, 2, 8, 8, 1024, 8192, 128, 0) == 6 * 2 * 8 * 1024 * 129 * 4  # 128 tiles: 6 splits
    assert ws(BF16, 1, 16, 16, 512, 8192, 64, 1) == 0      # causal: its queries see 512 keys
    assert ws(BF16, 8, 32, 32, 1, 8192, 128, 0) == 3 * 8 * 32 * 1 * 129 * 4  # no GQA: 256 workgroups
    assert ws(BF16, 1, 32, 8, 1, 32768, 128, 0) == 64 * 32 * 1 * 129 * 4     # 8 workgroups, at most 64 splits
    assert ws(BF16, 4, 16, 16, 2048, 2048, 128, 1) == 0     # the config: 1024 workgroups
    assert ws(F32, 1, 2, 2, 1, 8192, 128, 0) == 0           # fp32 never splits
    assert ws(BF16, 1, 2, 2, 1, 448, 128, 0) == 0           # fewer than 8 key tiles
    assert ws(BF16, 1, 4, 4, 1, 777, 128, 0) == 3 * 4 * 1 * 129 * 4
    assert ws(BF16, 0, 4, 4, 1, 777, 128, 0) == 0


def test_gemm_workspace_policy():
    """Host-side policy of the contraction split (no GPU call): batch 1, at most 256
    (16-bit) or 128 (fp32) tiles of 128 x 128, K >= 1024 with K / s a multiple of 64
    and at least 128 steps a range, and a modelled saving of 15% or more; the
    workspace holds s fp32 partials [M, N]."""
    L = _lib.load()
    ws = L.ghip_gemm_workspace_bytes
    BF16, F16, F32 = _lib.DT_BFLOAT16, _lib.DT_FLOAT16, _lib.DT_FLOAT32
    assert ws(BF16, BF16, 1, 16, 4096, 4096) == 16 * 16 * 4096 * 4     # decoding-size rows: 16 ranges of 256
    assert ws(F16, F32, 1, 16, 4096, 4096) == 16 * 16 * 4096 * 4
    assert ws(BF16, BF16, 1, 256, 4096, 4096) == 4 * 256 * 4096 * 4   # 64 tiles: the partials' traffic caps it at 4
    assert ws(BF16, BF16, 1, 4, 2048, 1024) == 8 * 4 * 2048 * 4       # ranges of 128 steps
    assert ws(BF16, BF16, 1, 1024, 1024, 8192) == 8 * 1024 * 1024 * 4  # 64 tiles: 8 ranges
    assert ws(BF16, BF16, 1, 2048, 2048, 8192) == 2 * 2048 * 2048 * 4  # 256 tiles: 2 ranges
    # 14 ranges of 1024: reading W bounds 14 and 16 ranges alike, and 14 write fewer partials
    assert ws(BF16, BF16, 1, 16, 4096, 14336) == 14 * 16 * 4096 * 4
    assert ws(BF16, BF16, 1, 2048, 4096, 4096) == 0   # 512 tiles: one full round already
    assert ws(BF16, BF16, 1, 2048, 2048, 2048) == 0   # the partials' traffic would eat the saving
    assert ws(BF16, BF16, 2, 16, 4096, 4096) == 0     # batched products never split
    assert ws(BF16, BF16, 1, 16, 4096, 1000) == 0     # short contraction
    assert ws(BF16, BF16, 1, 16, 4096, 1096) == 0     # no split of K into multiples of 64
    # fp32: one 128 x 128 tile per CU already runs near the CU's fp32 MFMA rate, so a
    # split only fills idle CUs (t x s <= 256)
    assert ws(F32, F32, 1, 16, 4096, 4096) == 8 * 16 * 4096 * 4
    assert ws(F32, BF16, 1, 1024, 1024, 8192) == 4 * 1024 * 1024 * 4
    assert ws(F32, F32, 1, 2048, 2048, 2048) == 0    # 256 tiles: every CU busy
    assert ws(F32, F32, 1, 2048, 4096, 4096) == 0
    assert ws(_lib.DT_FLOAT64, _lib.DT_FLOAT64, 1, 16, 4096, 4096) == 0
    assert ws(BF16, BF16, 1, 0, 4096, 4096) == 0
