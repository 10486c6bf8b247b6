"""Host logic of the ``hip`` backend selection (engines/__init__.py:53-135
semantics) and of the native structs, without a GPU."""

import ctypes
import subprocess
from pathlib import Path

import pytest

import yapd_amd.engines as E
from yapd_amd import kernels


def test_resolve_env_overrides(monkeypatch):
    monkeypatch.setattr(E, "_hip_available", lambda: True)
    monkeypatch.setenv("CHATTERBOX_FLASH_ENGINE", "hip")
    assert E._resolve_backend("auto") == "hip"
    monkeypatch.setenv("CHATTERBOX_FLASH_ENGINE", "torch")
    with pytest.raises(ImportError):
        E._resolve_backend("hip")  # the env var wins, and torch lives in chatterbox_flash
    monkeypatch.delenv("CHATTERBOX_FLASH_ENGINE")
    assert E._resolve_backend("hip") == "hip"
    with pytest.raises(ValueError):
        E._resolve_backend("cuda")


def test_unavailable_raises_import_error(monkeypatch):
    monkeypatch.delenv("CHATTERBOX_FLASH_ENGINE", raising=False)
    monkeypatch.setattr(E, "_hip_available", lambda: False)
    with pytest.raises(ImportError):
        E._resolve_backend("hip")
    with pytest.raises(ImportError):
        E._resolve_backend("auto")


def test_shim_exports():
    import yapd_amd.attention_hip as shim
    assert hasattr(shim, "HipEngine") and callable(shim.hip_available)
    from yapd_amd.engines.base import InferenceEngine
    assert "block_forward_graph" in dir(InferenceEngine)


def test_ctypes_structs_match_c_header(tmp_path):
    """Field offsets of the ctypes mirrors equal the C compiler's (gcc on the header)."""
    header = Path(__file__).resolve().parents[1] / "include" / "yapd_t3.h"
    structs = {"yapd_t3_layer": kernels.T3Layer, "yapd_t3_model": kernels.T3Model,
               "yapd_t3_workspace": kernels.T3Workspace}
    lines = [f'#include "{header}"', "#include <stdio.h>", "#include <stddef.h>", "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'  printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for cname, py in structs.items():
        assert int(got[cname]) == ctypes.sizeof(py)
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, (cname, fname)
