"""The C-ABI library loads and exports every entry point include/*.h declares
(no compute calls: this runs without a GPU)."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(cwen_\w+)\s*\(", re.M)


def declared(headers=None):
    names = set()
    for h in headers or (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(DECL.findall(text))
    return sorted(names)


HOST_H = [ROOT / "cwen_amd" / "host" / "cwen_host.h"]


def test_header_declares_entry_points():
    names = declared()
    for must in ("cwen_ctx_create", "cwen_weight_upload", "cwen_gemvb", "cwen_gemvb_swiglu"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from cwen_amd import gpu
    if not gpu.LIB_PATH.exists():
        pytest.fail("libcwen_gpu.so is not built (python -m cwen_amd.build)")
    L = C.CDLL(str(gpu.LIB_PATH))
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    from cwen_amd import gpu
    bound = {name for name, _, _ in gpu.SIGNATURES}
    assert set(declared()) <= bound, set(declared()) - bound


def test_host_library_exports_and_bindings():
    """libcwen_host.so (host drivers, GGUF reader) exports what cwen_host.h
    declares, and the Python binding covers it."""
    from cwen_amd import gpu
    if not gpu.HOST_LIB_PATH.exists():
        pytest.fail("libcwen_host.so is not built (python -m cwen_amd.build)")
    L = gpu.host_lib()
    names = declared(HOST_H)
    assert "cwen_gguf_open" in names and "cwen_model_load_gguf" in names
    assert not [n for n in names if not hasattr(L, n)]
    assert set(names) <= {name for name, _, _ in gpu.HOST_SIGNATURES}


def test_version_string():
    from cwen_amd import gpu
    assert b"gfx950" in gpu.lib().cwen_version()


def test_ctx_create_rejects_bad_device_without_gpu():
    """Argument checking happens before any compute (no GPU needed)."""
    from cwen_amd import gpu
    h = C.c_void_p()
    assert gpu.lib().cwen_ctx_create(-1, C.byref(h)) != 0
    assert gpu.lib().cwen_ctx_create(0, None) == -1
