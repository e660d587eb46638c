"""The C-ABI library loads, exports every symbol include/jangq_amd.h declares, and rejects
bad arguments on the host before any launch (no compute without a GPU). CPU only."""
import ctypes
import re
from pathlib import Path

import pytest

HEADER = Path(__file__).resolve().parent.parent / "include" / "jangq_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path_entry_points():
    names = declared_functions()
    for n in ("jq_unpack", "jq_dequantize", "jq_quantize", "jq_quantized_matmul",
              "jq_gather_qmm", "jq_moe_route", "jq_switch_glu"):
        assert n in names


def test_library_exports_every_declared_symbol(native_lib):
    from jangq_amd import _lib

    for name in declared_functions():
        assert hasattr(native_lib, name), f"{name} declared but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_status_strings(native_lib):
    assert native_lib.jq_abi_version() == 2
    from jangq_amd import _lib

    assert _lib.status_string(0) == "ok"
    assert "bits" in _lib.status_string(-1)
    assert "group_size" in _lib.status_string(-2)


def test_entry_points_validate_before_launch(native_lib):
    """Invalid bits / group sizes / dtypes / shapes / null pointers return negative codes."""
    L = native_lib
    # bits 7
    assert L.jq_quantized_matmul(None, 1, None, None, None, 1, 7, 64, 1, 8, 64, None, 1, None) == -1
    # group size 48
    assert L.jq_quantized_matmul(None, 1, None, None, None, 1, 4, 48, 1, 8, 96, None, 1, None) == -2
    # K not a multiple of gs
    assert L.jq_dequantize(None, None, None, 1, 4, 64, 4, 96, None, 1, None) == -2
    # dtype code 9
    assert L.jq_quantized_matmul(None, 9, None, None, None, 1, 4, 64, 1, 8, 64, None, 1, None) == -4
    # non-empty operand with null pointers
    assert L.jq_quantized_matmul(None, 1, None, None, None, 1, 4, 64, 1, 8, 64, None, 1, None) == -5
    # empty problem is a no-op
    assert L.jq_quantized_matmul(None, 1, None, None, None, 1, 4, 64, 0, 8, 64, None, 1, None) == 0
    assert L.jq_unpack(None, 4, 0, 64, None, None) == 0
    # routing: k > E
    assert L.jq_moe_route(None, 1, 4, 5, 1, None, None, None) == -3
    # gather workspace query is host-only
    assert L.jq_gather_workspace_size(64, 128, 1) > 0
    assert L.jq_gather_workspace_size(-1, 128, 1) == -1
    # gather without workspace
    one = ctypes.c_void_p(1)
    assert L.jq_gather_qmm(one, 1, 4, 1, one, one, one, 1, 4, 64, 8, 128, 128, None, one, 4, 0,
                           one, 1, None, 0, None) == -7


def test_newer_entry_points_validate_before_launch(native_lib):
    """MX modes, the fused MoE calls and the K-split workspace query reject bad arguments on
    the host (no launch)."""
    L = native_lib
    assert L.jq_mx_dequantize(None, None, 5, 1, 32, None, 0, None) == -1     # mode
    assert L.jq_mx_dequantize(None, None, 4, 1, 48, None, 0, None) == -2     # K % 32
    assert L.jq_mx_dequantize(None, None, 4, 1, 32, None, 0, None) == -5     # null
    assert L.jq_mx_dequantize(None, None, 8, 0, 32, None, 0, None) == 0      # empty
    assert L.jq_mx_quantized_matmul(None, 1, None, None, 4, 1, 8, 32 * 64 * 8 + 32, None, 1,
                                    None) == -3                               # K too long
    assert L.jq_mx_quantized_matmul(None, 0, None, None, 8, 1, 8, 64, None, 1, None) == -4
    # routed experts: k > E, and missing logits with tokens to route
    args = [None, 1, 1, 256, 128, 4, None, 5, 1, None, None,
            None, None, None, None, None, None, 2, None, None, None, 2, 1, 64,
            None, None, None, None, 1, None, 0, None]
    one = ctypes.c_void_p(1)
    a = list(args)
    a[6], a[9], a[10], a[27] = one, one, one, one
    assert L.jq_moe_experts(*a) == -3
    a = list(args)
    a[7] = 2
    assert L.jq_moe_experts(*a) == -5
    # fused combine: weights missing
    assert L.jq_switch_glu_combine(None, 1, 1, 256, 128, 4, None, None, 2, None, None, None,
                                   None, None, None, 2, None, None, None, 2, 1, 64, None, None,
                                   None, None, 1, None, 0, None) == -5
    # K-split workspace: 0 where the split does not apply, -1 for negative sizes
    assert L.jq_quantized_matmul_workspace_size(1, 4096, 4096, 4, 64, 1, 1) == 0
    assert L.jq_quantized_matmul_workspace_size(8, 4096, 14336, 2, 64, 1, 1) > 0
    assert L.jq_quantized_matmul_workspace_size(-1, 4096, 14336, 2, 64, 1, 1) == -1
