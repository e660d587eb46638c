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
    """uint8 scales: mxfp4 / mxfp8 chosen from the shapes, biases dropped (loader.py:1877-1912);
    MX expert stacks are refused."""
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
    write_bundle(tmp_path / "x", t)
    with pytest.raises(NotImplementedError, match="MX-mode expert"):
        loader.load_bundle_into(_block(), tmp_path / "x")


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
