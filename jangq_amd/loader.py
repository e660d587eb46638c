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
A module whose scales are uint8 (E8M0), dense or an expert stack, switches to the MX mode its
shapes give, mxfp4 or mxfp8 at group size 32, and drops the affine biases
(loader.py:1877-1912). Float expert stacks (SwitchLinear) that the bundle holds quantized are
upgraded to QuantizedSwitchLinear first (loader.py:1826-1848); a quantized gate loaded into a
float router (DenseRouter) is dequantized to fp32 on the GPU (loader.py:452-482); and the
reference's dtype policy (bfloat16 for 512+ experts at hidden 4096+, and for MLA models,
loader.py:536-557) is applied to the floating tensors at the end.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path

import torch

from . import nn as jnn
from . import ops
from . import shards
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
    upgraded: list = field(default_factory=list)
    dtype: str | None = None
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
    == 4 * word columns (loader.py:1877-1912); no biases. Dense modules and expert stacks."""
    w_cols, s_cols = w.shape[-1], s.shape[-1]
    if s_cols * 32 == w_cols * 8:
        mode, bits = "mxfp4", 4
    elif s_cols * 32 == w_cols * 4:
        mode, bits = "mxfp8", 8
    else:
        raise ValueError(f"{mod}: uint8 scales {tuple(s.shape)} fit no MX mode for weight "
                         f"{tuple(w.shape)}")
    in_f = getattr(m, "in_features", None) or getattr(m, "input_dims", None)
    if s_cols * 32 != in_f or tuple(w.shape[:-1]) != tuple(m.weight.shape[:-1]):
        raise ValueError(f"{mod}: {mode} shapes {tuple(w.shape)} / {tuple(s.shape)} do not fit "
                         f"the module (rows {tuple(m.weight.shape[:-1])}, {in_f} inputs)")
    m.weight = w.view(torch.int32).to(device)
    m.scales = s.to(device)
    m.biases = None
    m.bits, m.group_size, m.mode = bits, 32, mode
    report.fixed[mod] = (mode, bits, 32)
    report.loaded += 2


def dtype_policy(config: dict):
    """The float dtype the reference loader forces on a model (loader.py:536-557): bfloat16 for
    models with 512 or more experts and hidden size 4096 or more (float16 overflows at the
    shared expert's down projection) and for MLA models (mistral4, kv_lora_rank > 0, whose
    gate is dequantized to a float weight); None otherwise (stored dtypes kept)."""
    text = config.get("text_config", config) or {}
    n_exp = (text.get("num_experts") or text.get("num_local_experts")
             or text.get("n_routed_experts") or 0)
    if n_exp >= 512 and text.get("hidden_size", 0) >= 4096:
        return torch.bfloat16
    if text.get("model_type") == "mistral4" or (text.get("kv_lora_rank") or 0) > 0:
        return torch.bfloat16
    return None


def _apply_dtype(model: torch.nn.Module, dtype) -> int:
    """Cast every floating parameter and buffer of the model to dtype, the float32 router gate
    included (MLX set_dtype's default predicate); codes and uint8 MX scales keep theirs.
    Returns the number of tensors cast."""
    n = 0
    with torch.no_grad():
        for mod in model.modules():
            for name, t in list(mod._parameters.items()) + list(mod._buffers.items()):
                if t is None or not t.is_floating_point() or t.dtype == dtype:
                    continue
                new = t.to(dtype)
                if name in mod._parameters:
                    mod._parameters[name] = torch.nn.Parameter(new, requires_grad=False)
                else:
                    mod._buffers[name] = new
                n += 1
    return n


def _dequant_router(mod: str, m, t: dict, device, report: LoadReport):
    """A quantized gate for a float router: dequantized on the GPU to fp32 with the first of
    8, 6, 4, 3, 2 bits whose group size divides the row (loader.py:452-482). The reference
    takes the first bits whose group size merely divides (so a 4-bit gs-64 gate also reads as
    8-bit gs-32 at half its width); here the candidate must also give the router's input
    width, which picks the one reading whose shape the model can use."""
    w, s = t["weight"], t["scales"]
    b = t.get("biases")
    cols, scols = w.shape[-1], s.shape[-1]
    if w.shape[0] != m.out_features:
        raise ValueError(f"{mod}: gate rows {w.shape[0]} != {m.out_features} experts")
    for bits in (8, 6, 4, 3, 2):
        real = cols * 32 // bits
        gs = real // scols if scols else 0
        if gs in (32, 64, 128) and gs * scols == real and real == m.in_features:
            break
    else:
        raise ValueError(f"{mod}: quantized gate {tuple(w.shape)} / {tuple(s.shape)} fits no "
                         f"bits / group size for {m.in_features} inputs")
    s = s.to(device)
    b = torch.zeros_like(s) if b is None else b.to(device)
    dq = ops.dequantize(w.view(torch.int32).to(device), s, b, gs, bits, dtype=torch.float32)
    with torch.no_grad():
        m.weight = torch.nn.Parameter(dq, requires_grad=False)
    report.fixed[mod] = ("dequantized", bits, gs)
    report.loaded += 3


class _Views:
    """get_tensor over the zero-copy views of an aligned shard (context-manager form of
    safe_open)."""

    def __init__(self, shard):
        self.v = shards.open_views(shard)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False

    def keys(self):
        return self.v.keys()

    def get_tensor(self, key):
        return self.v[key]


def _open_shard(shard, device):
    """A GPU load of a dtype-aligned shard reads the tensors as views of the mapped file, so
    each upload copies straight from the page cache; other shards (and CPU loads, whose
    tensors must not alias a read-only mapping) go through safetensors' own reader."""
    from safetensors import safe_open
    if device.type == "cuda" and shards.verify_alignment(shard)[1] == 0:
        return _Views(shard)
    return safe_open(str(shard), framework="pt")


def load_bundle_into(model: torch.nn.Module, path, *, device=None,
                     strict: bool = False) -> LoadReport:
    """Assign a v2 bundle's tensors to ``model``'s quantized modules (QuantizedLinear,
    QuantizedSwitchLinear) and other parameters / buffers, by name, onto ``device`` (default:
    the device of the model's first tensor). Codes stay uint32 words (held as int32), scales
    and biases keep their stored dtype. With ``strict`` a key that matches nothing, or a
    module tensor the bundle lacks, raises KeyError."""
    cfg, jang = read_configs(path)
    one_bit = affine1_modules(jang)
    if device is None:
        first = next(iter(model.state_dict().values()), None)
        device = first.device if first is not None else torch.device("cpu")
    device = torch.device(device)
    report = LoadReport()

    from safetensors import safe_open

    keys = {}
    for shard in shard_paths(path):
        with safe_open(str(shard), framework="pt") as f:
            for key in f.keys():
                keys[key] = shard
    # Float expert stacks the bundle holds quantized become QuantizedSwitchLinear
    # (loader.py:1826-1848); their bits and group size are fixed below from the shapes.
    q = cfg.get("quantization") or {}
    upgrade = {n for n, m in model.named_modules()
               if isinstance(m, jnn.SwitchLinear) and f"{n}.scales" in keys}
    if upgrade:
        report.upgraded = jnn.upgrade_switch_to_quantized(
            model, int(q.get("bits", 4)), int(q.get("group_size", 64)), names=upgrade)
    modules = dict(model.named_modules())
    quant = {n: m for n, m in modules.items()
             if isinstance(m, (jnn.QuantizedLinear, jnn.QuantizedSwitchLinear))}
    routers = {n: m for n, m in modules.items() if isinstance(m, jnn.DenseRouter)}
    state = model.state_dict()
    pending: dict[str, dict] = {}
    gates: dict[str, dict] = {}

    for shard in shard_paths(path):
        with _open_shard(shard, device) as f:
            for key in f.keys():
                mod, attr = _split(key)
                if mod in routers and attr in _QUANT_ATTRS and f"{mod}.scales" in keys:
                    gates.setdefault(mod, {})[attr] = f.get_tensor(key)
                elif mod in quant and attr in _QUANT_ATTRS:
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

    for mod, t in gates.items():
        _dequant_router(mod, routers[mod], t, device, report)

    for mod in quant:
        if mod not in pending:
            report.missing += [f"{mod}.{a}" for a in _QUANT_ATTRS]
    dt = dtype_policy(cfg)
    if dt is not None:
        report.dtype = str(dt).replace("torch.", "")
        _apply_dtype(model, dt)
    if strict and (report.unexpected or report.missing):
        raise KeyError(f"bundle/module mismatch: unexpected {report.unexpected[:8]}, "
                       f"missing {report.missing[:8]}")
    return report
