"""CPU checks of the drop-in boundary: libdaiza_hip.so loads, exports every entry point that
include/*.h declares, and the Python mirror neither reaches the oracle nor falls back to the CPU.
No compute call is made (there is no GPU here)."""
import ctypes
import glob
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        if os.path.basename(h) == "daiza_synth.h":  # header-only generator, no exported symbols
            continue
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(dz_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def so():
    import daiza_amd
    if not os.path.exists(daiza_amd.LIB_PATH):
        pytest.fail("libdaiza_hip.so is not built; run __graft_entry__.build()")
    return ctypes.CDLL(daiza_amd.LIB_PATH)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("dz_q1_0_upload", "dz_q1_0_matvec", "dz_q1_0_matvec_multi", "dz_q1_0_dequant_rows",
                 "dz_model_create", "dz_ctx_create", "dz_forward_token", "dz_forward_batch",
                 "dz_decode_greedy", "dz_kv_truncate", "dz_ctx_reset"):
        assert must in names


def test_library_exports_every_declared_symbol(so):
    missing = [n for n in sorted(declared_functions()) if not hasattr(so, n)]
    assert not missing, missing


def test_python_mirror_binds_every_symbol(so):
    import daiza_amd
    assert set(daiza_amd.EXPORTED_SYMBOLS) <= declared_functions()
    assert declared_functions() <= set(daiza_amd.EXPORTED_SYMBOLS)


def test_exports_are_c_linkage(so):
    """nm shows the dz_ symbols unmangled and defined."""
    import daiza_amd
    out = subprocess.run(["nm", "-D", "--defined-only", daiza_amd.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert declared_functions() <= syms


def test_product_never_imports_oracle():
    """The product package must not reach oracle/ (test infrastructure)."""
    for path in glob.glob(os.path.join(ROOT, "daiza_amd", "**", "*.py"), recursive=True):
        src = open(path).read()
        assert not re.search(r"^\s*(import|from)\s+oracle\b", src, flags=re.M), path
    for path in glob.glob(os.path.join(ROOT, "daiza_amd", "csrc", "*")):
        assert "oracle" not in open(path, errors="ignore").read().lower() or path.endswith(".md"), path


def test_missing_library_fails_loudly(tmp_path):
    """With the shared library absent the mirror raises instead of computing anything."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import daiza_amd\n"
        "daiza_amd.LIB_PATH = %r\n"
        "try:\n"
        "    daiza_amd.lib()\n"
        "except daiza_amd.DaizaError as e:\n"
        "    print('raised', e.code)\n"
    ) % (ROOT, str(tmp_path / "nope.so"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "raised -4" in r.stdout, r.stdout + r.stderr


def test_config_matches_bonsai27b_abi(so):
    """dz_config_bonsai27b (C) and Config.bonsai27b (Python) agree field by field."""
    import daiza_amd
    c = daiza_amd.Config()
    so.dz_config_bonsai27b(ctypes.byref(c), 1234)
    p = daiza_amd.Config.bonsai27b(max_ctx=1234)
    for name, _ in daiza_amd.Config._fields_:
        assert getattr(c, name) == pytest.approx(getattr(p, name)), name
    assert [p.is_full_attention(i) for i in range(8)] == [False, False, False, True] * 2
