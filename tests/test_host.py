"""Host-side logic: bit / group-size inference from packed shapes and operator argument
checks that run before any kernel. CPU only."""
import pytest
import torch

from jangq_amd import ops
from jangq_amd.shapes import bit_inference, infer_bits_group_size, is_router_name


def test_bit_inference_swift_cases():
    # jang-runtime/Tests/JANGCoreTests/BitInferenceTests.swift:5-52
    r = bit_inference([3072, 512], [3072, 64], 64)
    assert (r.bits, r.in_features, r.out_features) == (4, 4096, 3072)
    r = bit_inference([5120, 512], [5120, 128], 64)
    assert (r.bits, r.in_features) == (2, 8192)
    r = bit_inference([128, 1024, 512], [128, 1024, 64], 64)
    assert (r.bits, r.in_features, r.out_features) == (4, 4096, 128 * 1024)
    assert bit_inference([3072, 512], [64], 64) is None
    assert bit_inference([3072, 512], [3000, 64], 64) is None


def test_loader_rule_ambiguous_embedding_uses_logical_dims():
    # jang-tools/tests/test_loader_mxfp4_mode.py:29-46: (248320, 640)/(248320, 80) with a
    # module initialised at 8-bit/gs32 is 4-bit/gs64 once the logical width 5120 is known.
    assert infer_bits_group_size(640, 80, bits=8, group_size=32, logical_in=5120) == (4, 64)
    # without the logical width the module's own gs wins: 8-bit/gs32 is a valid reading
    assert infer_bits_group_size(640, 80, bits=8, group_size=32) == (8, 32)


@pytest.mark.parametrize("bits,gs,K", [(2, 64, 4096), (3, 64, 4096), (4, 64, 4096),
                                       (6, 64, 4096), (8, 64, 4096), (2, 128, 1024),
                                       (3, 64, 14336)])
def test_loader_rule_recovers_config_shapes(bits, gs, K):
    w_cols, s_cols = K * bits // 32, K // gs
    assert infer_bits_group_size(w_cols, s_cols, bits=4, group_size=gs) == (bits, gs)
    assert infer_bits_group_size(w_cols, s_cols, bits=4, group_size=gs, logical_in=K) == (bits, gs)


def test_router_names_prefer_gs64():
    assert is_router_name("model.layers.3.mlp.gate")
    assert is_router_name("model.layers.3.mlp.shared_expert_gate")
    assert not is_router_name("model.layers.3.mlp.gate_proj")
    # 8-bit gs64 router vs the 4-bit gs32 alias of the same shapes
    assert infer_bits_group_size(1024, 64, bits=4, group_size=32, is_router=True) == (8, 64)


def test_operator_argument_checks_run_before_launch():
    w = torch.zeros((8, 8), dtype=torch.int32)
    s = torch.zeros((8, 1), dtype=torch.bfloat16)
    x = torch.zeros((1, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="bits"):
        ops.quantized_matmul(x, w, s, s, bits=7)
    with pytest.raises(ValueError, match="group_size"):
        ops.quantized_matmul(x, w, s, s, group_size=48)
    with pytest.raises(ValueError, match="transpose"):
        ops.quantized_matmul(x, w, s, s, transpose=False)
    with pytest.raises(ValueError, match="affine, mxfp4 and mxfp8"):
        ops.quantized_matmul(x, w, s, s, mode="nvfp4")
    with pytest.raises(ValueError, match="group_size=32"):
        ops.quantized_matmul(x, w, s, s, mode="mxfp4")  # MX modes are group 32, bits 4 / 8
    with pytest.raises(ValueError, match="GPU"):
        ops.quantized_matmul(x, w, s, s)  # CPU tensors are refused: no CPU fallback


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from jangq_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(_lib.JangqError, match="no CPU fallback"):
        _lib.lib()
