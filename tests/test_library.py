"""The C-ABI library: it loads without a GPU, exports every entry point that
include/l3p.h declares, and the Python layer refuses to run without it."""
import ctypes
import os
import re
import subprocess
import sys

import llama3pure_amd as l3p

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "l3p.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(l3p_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_bound_entry_points():
    assert sorted(l3p.EXPORTS) == declared()


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(l3p.LIB_PATH)
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_error_paths_without_a_device():
    """Calls that fail before touching a device report errors, not crashes."""
    L = l3p.lib()
    assert L.l3p_row_bytes(l3p.Q8_0, 4096) == 4096 // 32 * 34
    assert L.l3p_row_bytes(l3p.Q4_K, 4096) == 4096 // 256 * 144
    assert L.l3p_create(0, None) != 0
    assert L.l3p_synchronize(None) != 0
    assert L.l3p_profile(None, 1) != 0


def test_missing_library_fails_loudly(tmp_path):
    code = ("import llama3pure_amd as l3p\n"
            f"l3p.LIB_PATH = {str(tmp_path / 'nope.so')!r}\n"
            "try:\n    l3p.lib()\nexcept ImportError as e:\n    print('ImportError', e)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert "ImportError" in r.stdout and "build" in r.stdout
