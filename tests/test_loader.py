"""JANG v2 bundle loader on the CPU: format checks, the per-module bits / group-size fix from
tensor shapes (loader.py:1851-1982), tensor assignment, the 1-bit storage manifest and the
refused MXFP scales. No GPU work."""
import json

import numpy as np
import pytest
import torch

from jangq_amd import loader
from jangq_amd import nn as jnn
from tests.bundle_util import quantized, tensors_of, write_bundle

H, I, E, K_TOP = 256, 128, 4, 2


def _block():
    return jnn.SparseMoeBlock(H, I, E, K_TOP, shared_hidden=256, group_size=64, bits=2,
                              router_bits=8, shared_bits=8, device="cpu")


def _bundle_tensors():
    t = {}
    t.update(tensors_of("gate", *quantized(E, H, 8, 64, 1)))
    # experts stored at 3-bit g128 (gate/up) and 4-bit g64 (down), although the skeleton
    # was built at the config's 2-bit g64: the loader must fix them from the shapes
    t.update(tensors_of("switch_mlp.gate_proj", *quantized(I, H, 3, 128, 2, experts=E)))
    t.update(tensors_of("switch_mlp.up_proj", *quantized(I, H, 3, 128, 3, experts=E)))
    t.update(tensors_of("switch_mlp.down_proj", *quantized(H, I, 4, 64, 4, experts=E)))
    t.update(tensors_of("shared_expert.gate_proj", *quantized(256, H, 8, 64, 5)))
    t.update(tensors_of("shared_expert.up_proj", *quantized(256, H, 8, 64, 6)))
    t.update(tensors_of("shared_expert.down_proj", *quantized(H, 256, 8, 64, 7)))
    return t


def test_load_fixes_bits_and_assigns(tmp_path):
    t = _bundle_tensors()
    t["extra.weight"] = torch.ones(4)
    write_bundle(tmp_path, t)
    blk = _block()
    rep = loader.load_bundle_into(blk, tmp_path)
    assert rep.fixed == {"switch_mlp.gate_proj": (3, 128), "switch_mlp.up_proj": (3, 128),
                         "switch_mlp.down_proj": (4, 64)}
    assert rep.unexpected == ["extra.weight"] and rep.missing == [] and rep.expanded == []
    mods = dict(blk.named_modules())
    for key, v in t.items():
        if key == "extra.weight":
            continue
        mod, attr = key.rsplit(".", 1)
        got = getattr(mods[mod], attr)
        if attr == "weight":
            assert got.dtype == torch.int32
            assert torch.equal(got, v.view(torch.int32)), key
        else:
            assert got.dtype == v.dtype and torch.equal(got, v), key
    sw = blk.switch_mlp
    assert (sw.gate_proj.bits, sw.gate_proj.group_size) == (3, 128)
    assert (sw.down_proj.bits, sw.down_proj.group_size) == (4, 64)
    assert (blk.gate.bits, blk.gate.group_size) == (8, 64)
    with pytest.raises(ValueError, match="group sizes"):
        sw.group_size()  # 128 / 128 / 64: the SwitchGLU launches take one group size
    with pytest.raises(KeyError):
        loader.load_bundle_into(_block(), tmp_path, strict=True)


def test_missing_module_tensors(tmp_path):
    t = _bundle_tensors()
    del t["shared_expert.down_proj.biases"]
    write_bundle(tmp_path, t, shards=1)
    rep = loader.load_bundle_into(_block(), tmp_path)
    assert rep.missing == ["shared_expert.down_proj.biases"]


def test_format_checks(tmp_path):
    with pytest.raises(ValueError, match="jang_config"):
        loader.read_configs(tmp_path)
    write_bundle(tmp_path / "a", _bundle_tensors(), fmt="mlx")
    with pytest.raises(ValueError, match="not 'jang'"):
        loader.read_configs(tmp_path / "a")
    write_bundle(tmp_path / "b", _bundle_tensors(), version="1.1")
    with pytest.raises(ValueError, match="v2"):
        loader.read_configs(tmp_path / "b")
    cfg, jang = loader.read_configs(write_bundle(tmp_path / "c", _bundle_tensors()))
    assert cfg["quantization"] == {"group_size": 64, "bits": 2} and jang["format"] == "jang"
    (tmp_path / "d").mkdir()
    (tmp_path / "d" / "jang_config.json").write_text(json.dumps({"format": "jang",
                                                                 "format_version": "2.0"}))
    with pytest.raises(ValueError, match="no .safetensors"):
        loader.load_bundle_into(_block(), tmp_path / "d")


def test_mx_scales_switch_the_mode(tmp_path):
    """uint8 scales: mxfp4 / mxfp8 chosen from the shapes, biases dropped (loader.py:1877-1912),
    for dense modules and expert stacks alike."""
    rng = np.random.default_rng(4)
    t = _bundle_tensors()
    # router as mxfp8 (4 elements per word), shared down as mxfp4 (8 per word)
    t["gate.weight"] = torch.from_numpy(
        rng.integers(0, 2**32, (E, H // 4), dtype=np.uint64).astype(np.uint32).view(np.int32)).view(torch.uint32)
    t["gate.scales"] = torch.full((E, H // 32), 120, dtype=torch.uint8)
    del t["gate.biases"]
    t["shared_expert.down_proj.weight"] = torch.from_numpy(
        rng.integers(0, 2**32, (H, 256 // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)).view(torch.uint32)
    t["shared_expert.down_proj.scales"] = torch.full((H, 256 // 32), 127, dtype=torch.uint8)
    write_bundle(tmp_path, t)
    blk = _block()
    rep = loader.load_bundle_into(blk, tmp_path)
    assert rep.fixed["gate"] == ("mxfp8", 8, 32)
    assert rep.fixed["shared_expert.down_proj"] == ("mxfp4", 4, 32)
    assert blk.gate.mode == "mxfp8" and blk.gate.biases is None
    assert blk.shared_expert.down_proj.mode == "mxfp4"
    t["switch_mlp.down_proj.scales"] = torch.zeros((E, H, I // 32), dtype=torch.uint8)
    t["switch_mlp.down_proj.weight"] = torch.zeros((E, H, I // 8), dtype=torch.uint32)
    del t["switch_mlp.down_proj.biases"]
    write_bundle(tmp_path / "x", t)
    blk = _block()
    rep = loader.load_bundle_into(blk, tmp_path / "x")
    dn = blk.switch_mlp.down_proj
    assert rep.fixed["switch_mlp.down_proj"] == ("mxfp4", 4, 32) and not rep.missing
    assert (dn.mode, dn.bits, dn.group_size, dn.biases) == ("mxfp4", 4, 32, None)
    assert tuple(dn.weight.shape) == (E, H, I // 8) and dn.scales.dtype == torch.uint8
    assert not blk.switch_mlp.is_affine()
    # an MX stack whose scale columns do not give the module's input width
    t["switch_mlp.down_proj.scales"] = torch.zeros((E, H, I // 64), dtype=torch.uint8)
    t["switch_mlp.down_proj.weight"] = torch.zeros((E, H, I // 16), dtype=torch.uint32)
    write_bundle(tmp_path / "y", t)
    with pytest.raises(ValueError, match="do not fit"):
        loader.load_bundle_into(_block(), tmp_path / "y")


def test_shapes_that_fit_nothing(tmp_path):
    t = _bundle_tensors()
    # gate rows of a 3-expert router on a 4-expert skeleton
    t.update(tensors_of("gate", *quantized(E - 1, H, 8, 64, 1)))
    write_bundle(tmp_path, t)
    with pytest.raises(ValueError, match="rows"):
        loader.load_bundle_into(_block(), tmp_path)


def test_affine1_manifest(tmp_path):
    man = {"switch_mlp.down_proj": {"storage_bits": 1, "bits": 1, "group_size": 64},
           "gate": {"bits": 8, "group_size": 64},
           "shared_expert.up_proj": {"bits": 1}}
    jang = {"quantization": {"tensor_quantization_manifest": man}}
    assert loader.affine1_modules(jang) == {"switch_mlp.down_proj", "shared_expert.up_proj"}
    assert loader.affine1_modules({}) == frozenset()
    # 1-bit codes of the down stack: half the 2-bit words
    t = _bundle_tensors()
    rng = np.random.default_rng(9)
    t["switch_mlp.down_proj.weight"] = torch.from_numpy(
        rng.integers(0, 2**32, (E, H, I // 32), dtype=np.uint64).astype(np.uint32).view(np.int32)
    ).view(torch.uint32)
    t.update({k: v for k, v in tensors_of("switch_mlp.down_proj",
                                          *quantized(H, I, 2, 64, 4, experts=E)).items()
              if not k.endswith("weight")})
    write_bundle(tmp_path, t, manifest={"switch_mlp.down_proj": {"storage_bits": 1}})
    with pytest.raises(ValueError, match="GPU"):
        loader.load_bundle_into(_block(), tmp_path)


def test_dtype_policy():
    """bfloat16 for 512+ experts at hidden 4096+ and for MLA models (loader.py:536-557)."""
    assert loader.dtype_policy({"num_experts": 512, "hidden_size": 4096}) == torch.bfloat16
    assert loader.dtype_policy({"text_config": {"n_routed_experts": 1024,
                                                "hidden_size": 7168}}) == torch.bfloat16
    assert loader.dtype_policy({"num_local_experts": 512, "hidden_size": 2048}) is None
    assert loader.dtype_policy({"num_experts": 256, "hidden_size": 4096}) is None
    assert loader.dtype_policy({"model_type": "mistral4"}) == torch.bfloat16
    assert loader.dtype_policy({"kv_lora_rank": 512}) == torch.bfloat16
    assert loader.dtype_policy({"kv_lora_rank": None, "hidden_size": 8192}) is None
    assert loader.dtype_policy({}) is None


class _RouterModel(torch.nn.Module):
    """A float router and a float norm weight beside a quantized block (f16 sidecars)."""

    def __init__(self):
        super().__init__()
        self.gate = jnn.DenseRouter(H, E)
        self.norm = torch.nn.Parameter(torch.ones(H, dtype=torch.float16), requires_grad=False)
        self.proj = jnn.QuantizedLinear(H, 64, group_size=64, bits=4, dtype=torch.float16)


def test_dtype_policy_applied(tmp_path):
    t = {"gate.weight": torch.randn(E, H), "norm": torch.ones(H, dtype=torch.float16)}
    t.update(tensors_of("proj", *quantized(64, H, 4, 64, 3), sidecar="f16"))
    write_bundle(tmp_path / "a", t, config_extra={"num_experts": 512, "hidden_size": 4096})
    m = _RouterModel()
    rep = loader.load_bundle_into(m, tmp_path / "a")
    assert rep.dtype == "bfloat16" and not rep.missing and not rep.unexpected
    assert m.gate.weight.dtype == torch.bfloat16 and m.norm.dtype == torch.bfloat16
    assert m.proj.scales.dtype == torch.bfloat16 and m.proj.biases.dtype == torch.bfloat16
    assert m.proj.weight.dtype == torch.int32  # codes keep theirs
    np.testing.assert_array_equal(m.gate.weight.float().numpy(),
                                  t["gate.weight"].to(torch.bfloat16).float().numpy())
    # no policy: stored dtypes kept, the float router stays float32
    write_bundle(tmp_path / "b", t)
    m = _RouterModel()
    rep = loader.load_bundle_into(m, tmp_path / "b")
    assert rep.dtype is None and m.gate.weight.dtype == torch.float32
    assert m.proj.scales.dtype == torch.float16
    assert torch.equal(m.gate.weight, t["gate.weight"])


def test_quantized_router_gate_shape_checks(tmp_path):
    """A quantized gate for a float router must give the router's width at some bits / group
    size (the dequantization itself runs on the GPU)."""
    t = tensors_of("gate", *quantized(E, H // 4, 4, 64, 1))  # a 64-wide gate for 256 inputs
    write_bundle(tmp_path / "a", t)
    with pytest.raises(ValueError, match="fits no bits"):
        loader.load_bundle_into(_RouterModel(), tmp_path / "a")
    t = tensors_of("gate", *quantized(E + 1, H, 4, 64, 1))
    write_bundle(tmp_path / "b", t)
    with pytest.raises(ValueError, match="experts"):
        loader.load_bundle_into(_RouterModel(), tmp_path / "b")


class _FloatExperts(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.switch_mlp = torch.nn.Module()
        for name, (i, o) in {"gate_proj": (H, I), "up_proj": (H, I), "down_proj": (I, H)}.items():
            setattr(self.switch_mlp, name, jnn.SwitchLinear(i, o, E))


def test_switch_linear_upgrade(tmp_path):
    """Float expert stacks the bundle holds quantized become QuantizedSwitchLinear at the
    config's bits / group size, then take the shapes' (loader.py:1826-1848, 1851-1982); a float
    stack the bundle holds as floats stays SwitchLinear."""
    t = {}
    t.update(tensors_of("switch_mlp.gate_proj", *quantized(I, H, 3, 128, 2, experts=E)))
    t.update(tensors_of("switch_mlp.up_proj", *quantized(I, H, 2, 64, 3, experts=E)))
    t["switch_mlp.down_proj.weight"] = torch.randn(E, H, I).to(torch.bfloat16)
    write_bundle(tmp_path, t)
    m = _FloatExperts()
    rep = loader.load_bundle_into(m, tmp_path)
    assert sorted(rep.upgraded) == ["switch_mlp.gate_proj", "switch_mlp.up_proj"]
    sw = m.switch_mlp
    assert isinstance(sw.gate_proj, jnn.QuantizedSwitchLinear)
    assert isinstance(sw.down_proj, jnn.SwitchLinear)
    assert (sw.gate_proj.bits, sw.gate_proj.group_size) == (3, 128)
    assert (sw.up_proj.bits, sw.up_proj.group_size) == (2, 64)
    assert rep.fixed == {"switch_mlp.gate_proj": (3, 128)} and not rep.missing
    assert torch.equal(sw.down_proj.weight, t["switch_mlp.down_proj.weight"])
    assert torch.equal(sw.up_proj.weight, t["switch_mlp.up_proj.weight"].view(torch.int32))


def test_switch_linear_float_forward():
    """SwitchLinear's gather matmul equals the per-pair float products."""
    torch.manual_seed(0)
    lin = jnn.SwitchLinear(16, 8, 4, bias=True, dtype=torch.float32)
    with torch.no_grad():
        lin.weight.normal_()
        lin.bias.normal_()
    x = torch.randn(3, 1, 1, 16)
    idx = torch.tensor([[0, 2], [3, 3], [1, 0]])
    y = lin(x, idx)
    assert tuple(y.shape) == (3, 2, 1, 8)
    for t_ in range(3):
        for j in range(2):
            e = int(idx[t_, j])
            ref = x[t_, 0, 0] @ lin.weight[e].t() + lin.bias[e]
            torch.testing.assert_close(y[t_, j, 0], ref, rtol=1e-5, atol=1e-5)
