"""The C-ABI library loads on a CPU-only host, exports every function that
include/*.h declares, and rejects bad arguments before any launch."""

import ctypes
import re
from pathlib import Path

import pytest

from yapd_amd import kernels

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(yapd_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    assert "yapd_score_cfg_pmi_unmask" in names and "yapd_last_error" in names


def test_library_exports_every_declared_symbol():
    lib = kernels.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_signatures_cover_header():
    assert set(declared_functions()) <= set(kernels._SIGNATURES)


def test_abi_version_and_empty_error():
    lib = kernels.load_library()
    assert lib.yapd_abi_version() >= 1
    assert isinstance(lib.yapd_last_error(), bytes)


def test_score_rejects_bad_arguments_without_launch():
    lib = kernels.load_library()
    fn = lib.yapd_score_cfg_pmi_unmask
    nul = None
    # bl = 0 is invalid; every pointer NULL: validation fails first, no GPU call.
    rc = fn(nul, 8194, 8194, 1, 0, 8194, 0, 1, 0, 0, nul, nul, nul, nul, nul, nul, 10, 0.5, 1, 8194, 6562,
            0.0, 0, 0, 0, nul, nul, nul, nul, nul, nul, nul)
    assert rc == 1
    rc = fn(ctypes.c_void_p(16), 8194, 8194, 1, 65, 8194, 0, 1, 0, 0, nul, nul, nul, nul, nul, nul, 10, 0.5, 1,
            8194, 6562, 0.0, 0, 0, 0, nul, nul, nul, nul, nul, nul, nul)
    assert rc == 1 and b"bl" in lib.yapd_last_error()
    with pytest.raises(ValueError):
        kernels.check(1)
