"""The C-ABI library (libuocr_hip.so) loads on a CPU-only host and exports
every entry point include/uocr_hip/*.h declares; argument checks that need no
device return their documented codes."""
import ctypes as C
import glob
import os
import re
import subprocess

import pytest

from uocr_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "uocr_hip", "*.h")))


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        names += re.findall(r"\b(uocr_hip_\w+)\s*\(", text)
    return sorted(set(names))


def test_headers_declare_entry_points():
    names = declared_functions()
    assert "uocr_hip_moe_layer_forward" in names and "uocr_hip_moe_router_topk" in names


def test_library_exports_every_declared_symbol():
    path = _lib.lib_path()
    assert os.path.exists(path), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (uocr_hip_\w+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    # and the Python binding declares exactly the header's set
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_library_loads_and_validates_without_gpu():
    lib = _lib.load()
    assert lib.uocr_hip_version().decode()
    out = C.c_void_p()
    assert lib.uocr_hip_moe_layer_create(None, C.byref(out)) == _lib.EINVAL
    assert b"null" in lib.uocr_hip_last_error().lower()
    assert lib.uocr_hip_moe_layer_forward(None, None, 1, 1, None, None, None, None, 0, None) == _lib.EINVAL
    assert lib.uocr_hip_moe_layer_destroy(None) in (_lib.OK, _lib.EINVAL)
    assert lib.uocr_hip_moe_layer_workspace_size(None, 16) == 0


def test_no_cpu_fallback_in_product_sources():
    """The product library never links or loads the oracle."""
    csrc = os.path.join(ROOT, "unlimited-ocr.cpp_amd")
    for dirpath, _, files in os.walk(csrc):
        for f in files:
            if f.endswith((".hip", ".hpp", ".h", ".py", ".cpp", ".c")):
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert "liboracle" not in text and "import oracle" not in text, f


def test_upload_rejects_non_integer_zero_points():
    """Zeros must be integers in [0, 15] (what quantize_int4_awq and the GPTQ
    files produce); anything else is refused at upload, before any device call."""
    import numpy as np
    from uocr_hip import MoELayerInt4, synth
    from uocr_hip._lib import HipError

    L = synth.random_layer(5, hidden=256, inter=128, n_experts=4, top_k=2, n_shared=0, group=32)
    L.up[2].zeros = L.up[2].zeros.copy()
    L.up[2].zeros[3, 1] = 7.5
    with pytest.raises(HipError) as ei:
        MoELayerInt4(L)
    assert ei.value.code == _lib.EUNSUPPORTED and "integers in [0, 15]" in str(ei.value)
    L.up[2].zeros[3, 1] = 16.0
    with pytest.raises(HipError) as ei:
        MoELayerInt4(L)
    assert ei.value.code == _lib.EUNSUPPORTED
