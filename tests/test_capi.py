"""The C-ABI library loads and exports every symbol include/ditk.h declares (no GPU calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ditk.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\*]+\s+\**(ditk_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "ditk_flash_attn_varlen" in syms and "ditk_gemm" in syms and len(syms) >= 15


def test_library_exports_every_declared_symbol():
    from ditserve_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libditk.so not built (run python -m ditserve_amd.build)")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python binding table covers exactly the declared ABI
    assert sorted(_lib.SIGNATURES) == declared_symbols()
    assert lib.ditk_version() == 1


def test_ops_reject_cpu_tensors_before_launch():
    import torch
    from ditserve_amd import ops
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.adaln(x)
    with pytest.raises(ValueError):
        ops.linear(x, torch.zeros(8, 64, dtype=torch.bfloat16))
