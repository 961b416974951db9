"""CPU checks of the C ABI: the library loads, exports exactly the entry
points that include/gptq_hip.h declares, and the ctypes signatures cover
them.  No compute calls (there is no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gptq_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(gptq_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    names = declared()
    assert "gptq_hessian_accumulate" in names and "gptq_linear" in names
    assert len(names) >= 15


def test_library_exports_every_declared_symbol():
    from distributed_gptq_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    h = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(declared()) if not hasattr(h, n)]
    assert not missing, missing


def test_ctypes_signatures_match_header():
    from distributed_gptq_amd import _lib
    assert set(_lib.SIGNATURES) == declared()
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def test_library_loads_and_reports_version():
    from distributed_gptq_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    h = _lib.load()
    assert h.gptq_abi_version() == 1
    assert h.gptq_last_error() == b""
    # workspace queries are host-only arithmetic
    assert h.gptq_hessian_workspace_size(65536, 768) > 0
    assert h.gptq_factor_workspace_size(4096) >= 4096 * 4096 * 4
    # errors of one run of >= 512 columns (4 blocks of 128; one block of 1024)
    assert h.gptq_sweep_workspace_size(4096, 4096, 128) == 4096 * 512 * 4
    assert h.gptq_sweep_workspace_size(4096, 4096, 1024) == 4096 * 1024 * 4
    # linear: the act-order gather (rounded to 256 B) + split-K partials when
    # 16 < M <= 128 on a layer of < 192 x 128 rows (4096 rows: 32 x 8 splits)
    bf16 = 2
    assert h.gptq_linear_workspace_size(128, 4096, 4096, 4, 128, bf16, 0) == 8 * 128 * 4096 * 4
    assert h.gptq_linear_workspace_size(100, 4096, 4096, 4, 128, bf16, 1) == \
        (100 * 4096 * 2 + 255) // 256 * 256 + 8 * 100 * 4096 * 4
    # 11 blocks of 128 over 6 splits at 5120 rows (40 workgroups)
    assert h.gptq_linear_workspace_size(128, 5120, 1408, 3, 64, bf16, 0) == 6 * 128 * 5120 * 4
    # 64 < M <= 128 at 28672 rows: 128 workgroups of 224 rows, K in 2 ranges
    assert h.gptq_linear_workspace_size(128, 28672, 4096, 4, 128, bf16, 0) == 2 * 128 * 28672 * 4
    assert h.gptq_linear_workspace_size(64, 28672, 4096, 4, 128, bf16, 0) == 0    # unsplit, 7 waves
    assert h.gptq_linear_workspace_size(64, 4096, 14336, 4, 128, bf16, 0) == 8 * 64 * 4096 * 4
    assert h.gptq_linear_workspace_size(17, 4096, 14336, 3, 128, bf16, 0) == 8 * 17 * 4096 * 4
    assert h.gptq_linear_workspace_size(32, 4096, 4096, 4, 128, bf16, 0) == 0     # M <= 32 on 2^24 weights
    # 8 < M <= 16 on 3072-4096 rows with K >= 10240: K in 2 ranges
    assert h.gptq_linear_workspace_size(16, 4096, 14336, 4, 128, bf16, 0) == 2 * 16 * 4096 * 4
    assert h.gptq_linear_workspace_size(9, 3072, 10240, 3, 128, bf16, 0) == 2 * 9 * 3072 * 4
    assert h.gptq_linear_workspace_size(8, 4096, 14336, 4, 128, bf16, 0) == 0     # M <= 8
    assert h.gptq_linear_workspace_size(16, 4096, 8192, 4, 128, bf16, 0) == 0     # K < 10240
    assert h.gptq_linear_workspace_size(16, 2048, 14336, 4, 128, bf16, 0) == 0    # < 3072 rows
    assert h.gptq_linear_workspace_size(16, 4094, 14336, 4, 128, bf16, 0) == 0    # N % 4
    # M > 128: the grid counts two activation tiles (4096 rows: 4 splits)
    assert h.gptq_linear_workspace_size(256, 4096, 4096, 4, 128, bf16, 0) == 4 * 256 * 4096 * 4
    assert h.gptq_linear_workspace_size(256, 28672, 4096, 4, 128, bf16, 0) == 0
    assert h.gptq_linear_workspace_size(400, 4096, 4096, 4, 128, bf16, 0) == 0    # M > 384
    # 1 < M <= 16 on 4097-8191 rows with K >= 8192: K in 3 ranges
    assert h.gptq_linear_workspace_size(16, 5120, 13824, 4, 128, bf16, 0) == 3 * 16 * 5120 * 4
    assert h.gptq_linear_workspace_size(5, 5120, 13824, 3, 128, bf16, 0) == 3 * 5 * 5120 * 4
    assert h.gptq_linear_workspace_size(5, 5120, 13824, 3, 32, bf16, 0) == 0      # > 128 groups
    assert h.gptq_linear_workspace_size(16, 5120, 5120, 4, 128, bf16, 0) == 0     # K < 8192
    assert h.gptq_linear_workspace_size(2, 5120, 13824, 4, 128, bf16, 0) == 3 * 2 * 5120 * 4
    assert h.gptq_linear_workspace_size(1, 5120, 13824, 4, 128, bf16, 0) == 0     # M = 1: the GEMV
    # 1 < M <= 16 at 8192 rows: 128 workgroups of 64 rows, K in 2 ranges
    assert h.gptq_linear_workspace_size(16, 8192, 8192, 4, 128, bf16, 0) == 2 * 16 * 8192 * 4
    assert h.gptq_linear_workspace_size(16, 14336, 4096, 4, 128, bf16, 0) == 0
    assert h.gptq_linear_workspace_size(16, 5122, 13824, 4, 128, bf16, 0) == 0    # N % 4
    assert h.gptq_linear_workspace_size(128, 4098, 4096, 4, 128, bf16, 0) == 0    # N % 4
    assert h.gptq_linear_workspace_size(128, 4096, 4096, 8, 128, bf16, 0) == 0    # 8-bit
    assert h.gptq_linear_workspace_size(16, 4096, 4096, 4, 128, bf16, 1) == 16 * 4096 * 2


def test_entry_points_reject_bad_arguments_without_gpu():
    """Argument checks run on the host before any launch."""
    from distributed_gptq_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    h = _lib.load()
    null = ctypes.c_void_p(0)
    rc = h.gptq_hessian_accumulate(null, null, 16, 8, 8, 0, null, 0, null)
    assert rc == _lib.ERR_ARG
    assert b"null" in h.gptq_last_error()
    dummy = ctypes.c_void_p(16)
    rc = h.gptq_pack(dummy, 4, 8, 5, dummy, null)
    assert rc == _lib.ERR_ARG and b"bits" in h.gptq_last_error()
    rc = h.gptq_pack_reference_layout(dummy, 3, 8, 4, dummy, null)
    assert rc == _lib.ERR_SHAPE
    rc = h.gptq_damp_factor(dummy, 8, ctypes.c_float(1.0), ctypes.c_float(0.01), null, 7, null, dummy, null, dummy,
                            dummy, 10 ** 9, null)
    assert rc == _lib.ERR_ARG and b"mode" in h.gptq_last_error()
    rc = h.gptq_damp_factor(dummy, 64, ctypes.c_float(1.0), ctypes.c_float(0.01), null, 1, null, dummy, null, dummy,
                            dummy, 16, null)
    assert rc == _lib.ERR_WORKSPACE
