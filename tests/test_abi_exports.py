"""The C-ABI library exports every entry point include/hos_hip.h declares, and the ctypes mirror
(hos_amd/_lib.py) binds each one. Loads the library only; no compute calls (runs without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hos_hip.h")
LIB = os.path.join(ROOT, "hos_amd", "libhos_hip.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hos_(?:hip|peft|gguf|format|ft)_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("hos_hip_create", "hos_hip_matmul_f32_keyed", "hos_hip_matmul_abt_keyed", "hos_hip_matmul_atb_keyed",
                 "hos_hip_evict", "hos_hip_clear_cache", "hos_hip_upload_quant", "hos_hip_qgemm_fwd",
                 "hos_hip_qgemm_dx", "hos_hip_dequant", "hos_peft_loss_grad", "hos_peft_adamw"):
        assert must in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="libhos_hip.so not built (run __graft_entry__.build())")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"declared in hos_hip.h but not exported: {missing}"


@pytest.mark.skipif(not os.path.exists(LIB), reason="libhos_hip.so not built (run __graft_entry__.build())")
def test_ctypes_mirror_binds_every_symbol():
    from hos_amd import _lib
    assert set(declared()) <= set(_lib.SIGNATURES), sorted(set(declared()) - set(_lib.SIGNATURES))
    _lib.lib()  # binds argtypes/restype for every symbol


def test_bytes_for_matches_the_oracle_without_a_device():
    """hos_hip_bytes_for is pure arithmetic (src/gguf.rs:548-561): callable with no GPU present."""
    if not os.path.exists(LIB):
        pytest.skip("libhos_hip.so not built")
    from hos_amd import _lib
    from oracle import binding as o
    lib = _lib.lib()
    for t, n in ((8, 4096), (12, 4096), (14, 4096), (0, 10)):
        assert lib.hos_hip_bytes_for(t, n) == o.bytes_for(t, n)
