"""JANG v2 bundle loading onto this package's modules: the loader that feeds the kernels.

Restated from the reference's v2 load path (jang-tools/jang_tools/loader.py:341-560) for
torch modules on the GPU:
  - ``config.json`` carries ``quantization: {group_size, bits}`` (the COMPRESS tier) and
    ``jang_config.json`` carries ``format == "jang"`` and ``format_version`` (FORMAT.md:118-140);
  - the weights are the ``*.safetensors`` shards, read through mmap (``safe_open``), with MoE
    experts already stacked as ``switch_mlp.{gate,up,down}_proj`` [E, N, P] (FORMAT.md:170-182);
  - modules listed with storage bits 1 in ``jang_config.json``'s
    ``quantization.tensor_quantization_manifest`` are stored as 1-bit codes and expanded to
    the 2-bit runtime codes at load, losslessly, scales and biases unchanged
    (affine.py:466-545); here the expansion runs on the GPU (``jq_expand_1bit_to_2bit``);
  - every quantized module's bits and group size are then fixed from its tensor shapes
    (``_fix_quantized_bits``, loader.py:1851-1982, through :func:`shapes.infer_bits_group_size`).
A dense module whose scales are uint8 (E8M0) switches to the MX mode its shapes give, mxfp4
or mxfp8 at group size 32, and drops the affine biases (loader.py:1877-1912); expert stacks
in an MX mode raise (the gathered launches are affine only).
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path

import torch

from . import nn as jnn
from . import ops
from .shapes import infer_bits_group_size, is_router_name

AFFINE1_STORAGE_BITS = 1
AFFINE1_RUNTIME_BITS = 2
_QUANT_ATTRS = ("weight", "scales", "biases")


@dataclass
class LoadReport:
    """What a load did: tensors assigned, modules whose bits / group size changed
    ({path: (bits, group_size)}, or (mode, bits, 32) for an MX mode), modules expanded from
    1-bit storage, and the bundle keys that matched nothing / module tensors the bundle did
    not hold."""
    loaded: int = 0
    fixed: dict = field(default_factory=dict)
    expanded: list = field(default_factory=list)
    unexpected: list = field(default_factory=list)
    missing: list = field(default_factory=list)


def read_configs(path) -> tuple[dict, dict]:
    """(config.json, jang_config.json) of a bundle directory; ValueError unless it is a JANG
    v2 bundle with a quantization block (FORMAT.md:118-140)."""
    root = Path(path)
    cfg_path, jang_path = root / "config.json", root / "jang_config.json"
    if not jang_path.is_file():
        raise ValueError(f"{root}: no jang_config.json (not a JANG bundle)")
    jang = json.loads(jang_path.read_text())
    if jang.get("format") != "jang":
        raise ValueError(f"{root}: jang_config.json format is {jang.get('format')!r}, not 'jang'")
    version = str(jang.get("format_version", ""))
    if not version.startswith("2"):
        raise ValueError(f"{root}: format_version {version!r}; only v2 bundles load here "
                         "(v1 tensors go through dequantize_tensor)")
    cfg = json.loads(cfg_path.read_text()) if cfg_path.is_file() else {}
    q = cfg.get("quantization")
    if q is not None and not isinstance(q, dict):
        raise ValueError(f"{root}: config.json quantization must be an object")
    return cfg, jang


def affine1_modules(jang_config: dict) -> frozenset:
    """Module paths stored as 1-bit codes (manifest specs with storage bits 1)."""
    q = jang_config.get("quantization")
    manifest = q.get("tensor_quantization_manifest") if isinstance(q, dict) else None
    if not isinstance(manifest, dict):
        return frozenset()
    out = set()
    for path, spec in manifest.items():
        if isinstance(path, str) and isinstance(spec, dict):
            if int(spec.get("storage_bits", spec.get("bits", 0)) or 0) == AFFINE1_STORAGE_BITS:
                out.add(path)
    return frozenset(out)


def shard_paths(path) -> list:
    shards = sorted(Path(path).glob("*.safetensors"))
    if not shards:
        raise ValueError(f"{path}: no .safetensors shards")
    return shards


def _split(key: str) -> tuple[str, str]:
    mod, _, attr = key.rpartition(".")
    return mod, attr


def _fix_bits(path: str, module, w_cols: int, s_cols: int) -> tuple[int, int]:
    logical_in = getattr(module, "in_features", None) or getattr(module, "input_dims", None)
    return infer_bits_group_size(w_cols, s_cols, module.bits, module.group_size,
                                 logical_in=logical_in, is_router=is_router_name(path))


def _load_mx(mod: str, m, w: torch.Tensor, s: torch.Tensor, device, report: LoadReport):
    """uint8 E8M0 scales: mxfp4 when 32 * scale columns == 8 * word columns, mxfp8 when
    == 4 * word columns (loader.py:1877-1912); no biases."""
    if isinstance(m, jnn.QuantizedSwitchLinear):
        raise NotImplementedError(f"{mod}: MX-mode expert stacks are not implemented "
                                  "(the gathered launches are affine only)")
    w_cols, s_cols = w.shape[-1], s.shape[-1]
    if s_cols * 32 == w_cols * 8:
        mode, bits = "mxfp4", 4
    elif s_cols * 32 == w_cols * 4:
        mode, bits = "mxfp8", 8
    else:
        raise ValueError(f"{mod}: uint8 scales {tuple(s.shape)} fit no MX mode for weight "
                         f"{tuple(w.shape)}")
    if s_cols * 32 != m.in_features or tuple(w.shape[:-1]) != tuple(m.weight.shape[:-1]):
        raise ValueError(f"{mod}: {mode} shapes {tuple(w.shape)} / {tuple(s.shape)} do not fit "
                         f"the module ({m.out_features} x {m.in_features})")
    m.weight = w.view(torch.int32).to(device)
    m.scales = s.to(device)
    m.biases = None
    m.bits, m.group_size, m.mode = bits, 32, mode
    report.fixed[mod] = (mode, bits, 32)
    report.loaded += 2


def load_bundle_into(model: torch.nn.Module, path, *, device=None,
                     strict: bool = False) -> LoadReport:
    """Assign a v2 bundle's tensors to ``model``'s quantized modules (QuantizedLinear,
    QuantizedSwitchLinear) and other parameters / buffers, by name, onto ``device`` (default:
    the device of the model's first tensor). Codes stay uint32 words (held as int32), scales
    and biases keep their stored dtype. With ``strict`` a key that matches nothing, or a
    module tensor the bundle lacks, raises KeyError."""
    _, jang = read_configs(path)
    one_bit = affine1_modules(jang)
    if device is None:
        first = next(iter(model.state_dict().values()), None)
        device = first.device if first is not None else torch.device("cpu")
    device = torch.device(device)
    modules = dict(model.named_modules())
    quant = {n: m for n, m in modules.items()
             if isinstance(m, (jnn.QuantizedLinear, jnn.QuantizedSwitchLinear))}
    state = model.state_dict()
    report = LoadReport()
    pending: dict[str, dict] = {}

    from safetensors import safe_open

    for shard in shard_paths(path):
        with safe_open(str(shard), framework="pt") as f:
            for key in f.keys():
                mod, attr = _split(key)
                if mod in quant and attr in _QUANT_ATTRS:
                    pending.setdefault(mod, {})[attr] = f.get_tensor(key)
                elif key in state:
                    t = f.get_tensor(key)
                    dst = state[key]
                    if tuple(t.shape) != tuple(dst.shape):
                        raise ValueError(f"{key}: bundle shape {tuple(t.shape)} != "
                                         f"module shape {tuple(dst.shape)}")
                    with torch.no_grad():
                        dst.copy_(t.to(dst.dtype))
                    report.loaded += 1
                else:
                    report.unexpected.append(key)

    for mod, tensors in pending.items():
        m = quant[mod]
        mx = "scales" in tensors and tensors["scales"].dtype == torch.uint8
        lacking = [a for a in _QUANT_ATTRS if a not in tensors and not (mx and a == "biases")]
        if lacking:
            report.missing += [f"{mod}.{a}" for a in lacking]
            continue
        if mx:
            _load_mx(mod, m, tensors["weight"], tensors["scales"], device, report)
            continue
        w, s, b = tensors["weight"], tensors["scales"], tensors["biases"]
        if w.dtype not in (torch.uint32, torch.int32):
            raise ValueError(f"{mod}.weight: packed codes must be uint32 words, got {w.dtype}")
        if s.dtype not in (torch.bfloat16, torch.float16, torch.float32) or b.dtype != s.dtype:
            raise ValueError(f"{mod}: scales/biases must share a float dtype "
                             f"({s.dtype}, {b.dtype})")
        w = w.view(torch.int32).to(device)
        if mod in one_bit:
            if device.type != "cuda":
                raise ValueError(f"{mod}: 1-bit storage is expanded on the GPU; load onto a "
                                 "cuda device")
            w = ops.expand_packed_1bit_to_2bit(w).view(torch.int32)
            report.expanded.append(mod)
        bits, gs = _fix_bits(mod, m, w.shape[-1], s.shape[-1])
        if (bits, gs) != (m.bits, m.group_size):
            report.fixed[mod] = (bits, gs)
        lead = tuple(m.weight.shape[:-1])
        if tuple(w.shape[:-1]) != lead or tuple(s.shape[:-1]) != lead:
            raise ValueError(f"{mod}: bundle rows {tuple(w.shape[:-1])} do not match the "
                             f"module's {lead}")
        in_dim = s.shape[-1] * gs
        logical_in = getattr(m, "in_features", None) or getattr(m, "input_dims", None)
        if in_dim != logical_in or w.shape[-1] * 32 != bits * in_dim:
            raise ValueError(f"{mod}: shapes {tuple(w.shape)} / {tuple(s.shape)} fit no "
                             f"(bits, group_size) for {logical_in} input features")
        m.weight = w
        m.scales = s.to(device)
        m.biases = b.to(device)
        m.bits, m.group_size, m.mode = bits, gs, "affine"
        report.loaded += 3

    for mod in quant:
        if mod not in pending:
            report.missing += [f"{mod}.{a}" for a in _QUANT_ATTRS]
    if strict and (report.unexpected or report.missing):
        raise KeyError(f"bundle/module mismatch: unexpected {report.unexpected[:8]}, "
                       f"missing {report.missing[:8]}")
    return report
