"""The C-ABI library loads without a GPU and exports exactly what include/forgeserve_amd.h declares.
Only argument checking runs here (it returns before any HIP call); no kernel is launched."""

import ctypes
import os
import re

import pytest

from forgeserve_amd import _lib
from forgeserve_amd.build import LIB, exported_symbols

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "forgeserve_amd.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fs_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("library not built (python -m forgeserve_amd.build)")
    return _lib.load()


def test_header_and_library_agree(lib):
    names = declared()
    assert len(names) >= 15
    exported = set(exported_symbols())
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(lib, n)


def test_python_binding_covers_the_header(lib):
    assert sorted(_lib.SIGNATURES) == declared()


def test_abi_version(lib):
    assert lib.fs_abi_version() == 3   # fs_kv_layout gained k_group


def test_argument_errors_are_reported_not_launched(lib):
    rc = lib.fs_gemm(None, 0, None, 0, None, 0, None, 0, 4, 4, 4, 1, None, 0, None)
    assert rc == -1 and b"null" in lib.fs_last_error()
    rc = lib.fs_spec_accept(None, 0, 0, None, 0, 0, 1, 1, 10, 1, None, None, None, None, None, 0, None, None, None,
                            None, None, None, None, 0, None)
    assert rc == -1
    rc = lib.fs_keyed_noise(None, 1, 0, 1, 10, 1, None, 10, 10, None)
    assert rc == -1 and b"keyed_noise" in lib.fs_last_error()
    # a debug output without its two companions is refused before anything is launched
    rc = lib.fs_spec_accept(1, 0, 0, 1, 0, 0, 1, 1, 10, 1, 1, None, 1, 1, 1, 10, 1, 1, None, 1, None, None, 1, 1 << 20,
                            None)
    assert rc == -1 and b"together" in lib.fs_last_error()
    lay = _lib.KVLayout()
    rc = lib.fs_paged_attention(None, 0, 0, 0, ctypes.byref(lay), None, 0, 1, None, 1, 1, 1, 1.0, None, 0, 0, 0, None,
                                0, None)
    assert rc == -1 and b"paged_attention" in lib.fs_last_error()
    # grouped keys need k_dim == 1: refused before anything is launched
    bad = _lib.KVLayout(1, 1, 4096, 2048, 8, 2, 64, 16, 1, 16, 16, 2, 128, 1, 8, 128)
    rc = lib.fs_paged_attention(1, 0, 0, 0, ctypes.byref(bad), 1, 1, 1, 1, 1, 1, 2, 1.0, 1, 0, 0, 0, 1, 1 << 30, None)
    assert rc == -1 and b"grouped keys" in lib.fs_last_error()
    rc = lib.fs_paged_kv_write(1, 1, 0, 0, 0, 1, 1, 1, 1, 1, 1, ctypes.byref(bad), None)
    assert rc == -1 and b"grouped keys" in lib.fs_last_error()


def test_workspace_sizes_are_positive(lib):
    assert lib.fs_paged_attention_workspace_size(64, 7, 32, 128, 600, 16) > 64 * 7 * 32 * 128 * 4
    assert lib.fs_spec_accept_workspace_size(64, 6, 128256) > 0
    assert lib.fs_paged_attention_split() == int(os.environ.get("FS_ATTN_SPLIT", 16384))
    assert lib.fs_sampling_workspace_size(64, 128256) > 0
    assert lib.fs_paged_attention_workspace_size(0, 1, 1, 1, 1, 1) == 0
    # split-K partials: a function of (N, K) only, sized for M rows
    assert lib.fs_gemm_workspace_size(448, 4096, 4096, 1) == 4 * 448 * 4096 * 4
    assert lib.fs_gemm_workspace_size(64, 28672, 4096, 1) == 0
    assert lib.fs_gemm_workspace_size(64, 4096, 4096, 0) == 0
    # a long batch runs the splits one after the other in each workgroup: no partials
    assert lib.fs_gemm_serial(448, 4096, 4096, 1) == 0 and lib.fs_gemm_serial(4096, 4096, 4096, 1) == 1
    assert lib.fs_gemm_workspace_size(4096, 4096, 4096, 1) == 0
    assert lib.fs_gemm_serial(32768, 28672, 4096, 1) == 0   # not split
    assert lib.fs_gemm_serial(32768, 4096, 14336, 1) == 0   # 3584-k splits keep their partials
    assert lib.fs_gemm_serial(4096, 4096, 4096, 0) == 0 and lib.fs_gemm_serial(0, 4096, 4096, 1) == 0
