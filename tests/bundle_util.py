"""Writes small synthetic JANG v2 bundles (config.json, jang_config.json, safetensors shards)
for the loader tests; weights are quantized with the CPU oracle."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
from safetensors.torch import save_file

from oracle import jangq_oracle as O
from tests._util import codes_tensor, sidecar_tensor


def quantized(rows, K, bits, gs, seed, experts=None):
    """(packed u32, scale bits, bias bits) of a seeded N(0, 0.02) matrix or expert stack."""
    rng = np.random.default_rng(seed)
    shape = (experts, rows, K) if experts else (rows, K)
    w = O.round_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
    flat = w.reshape(-1, K)
    packed, s, b, _ = O.quantize_affine(flat, bits, gs)
    lead = shape[:-1]
    return (packed.reshape(*lead, -1), np.asarray(s).reshape(*lead, -1),
            np.asarray(b).reshape(*lead, -1))


def tensors_of(prefix, packed, s, b, sidecar="bf16"):
    return {f"{prefix}.weight": codes_tensor(packed, "cpu").view(torch.uint32),
            f"{prefix}.scales": sidecar_tensor(s, sidecar, "cpu"),
            f"{prefix}.biases": sidecar_tensor(b, sidecar, "cpu")}


def write_bundle(root, tensors: dict, *, bits=2, group_size=64, manifest=None, shards=2,
                 fmt="jang", version="2.0", config_extra=None):
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    keys = sorted(tensors)
    for i in range(shards):
        part = {k: tensors[k].contiguous() for k in keys[i::shards]}
        if part:
            save_file(part, str(root / f"model-{i + 1:05d}-of-{shards:05d}.safetensors"))
    cfg = {"model_type": "synthetic_moe", "quantization": {"group_size": group_size, "bits": bits}}
    cfg.update(config_extra or {})
    (root / "config.json").write_text(json.dumps(cfg))
    q = {"profile": "JANG_2L", "block_size": group_size, "bit_widths_used": [2, 8]}
    if manifest:
        q["tensor_quantization_manifest"] = manifest
    (root / "jang_config.json").write_text(json.dumps(
        {"format": fmt, "format_version": version, "quantization": q,
         "source_model": {"name": "synthetic"}}))
    return root
