"""Module layer mirroring the reference's quantized modules on torch.

  QuantizedLinear / JANGLinear   jang-tools/jang_tools/jangrt/linear.py:22-45 (mlx nn.QuantizedLinear)
  QuantizedSwitchLinear          mlx_lm switch_layers, as upgraded by loader.py:1826-1848;
                                 the DSV4.1 SwitchProj (dsv41/model.py:847-857) has the same call
  SwitchGLU                      mlx_lm SwitchGLU (restated at dots3/ops.py:195-223)
  SwitchLinear                   mlx_lm SwitchLinear (float experts), upgraded to
                                 QuantizedSwitchLinear by loader.py:1826-1848
  DenseRouter                    the float MoEGate of mistral4_mlx.py:343-352
  SparseMoeBlock                 qwen4_exp/modeling.py:577-599 routing + experts + shared expert
Parameters are plain tensors (weight uint32, scales/biases bf16 by default) that a loader
fills; every forward runs the gfx950 kernels through :mod:`jangq_amd.ops`.
"""
from __future__ import annotations

import math

import torch

from . import ops


class QuantizedLinear(torch.nn.Module):
    """y = x @ dequantize(weight)^T (+ bias)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 group_size: int = 64, bits: int = 4, *, dtype=torch.bfloat16, device=None):
        super().__init__()
        if (in_features * bits) % 32 or in_features % group_size:
            raise ValueError("in_features must fill whole uint32 words and whole groups")
        self.in_features, self.out_features = in_features, out_features
        self.bits, self.group_size, self.mode = bits, group_size, "affine"
        g = in_features // group_size
        self.register_buffer("weight", torch.zeros(
            (out_features, in_features * bits // 32), dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros((out_features, g), dtype=dtype, device=device))
        self.register_buffer("biases", torch.zeros((out_features, g), dtype=dtype, device=device))
        self.bias = (torch.nn.Parameter(torch.zeros(out_features, dtype=dtype, device=device),
                                        requires_grad=False) if bias else None)

    @classmethod
    def from_float(cls, w: torch.Tensor, group_size: int = 64, bits: int = 4,
                   scales_dtype=None) -> "QuantizedLinear":
        """Quantize a float [out, in] weight on the GPU (mx.quantize rule)."""
        out_f, in_f = w.shape
        m = cls(in_f, out_f, group_size=group_size, bits=bits,
                dtype=scales_dtype or w.dtype, device=w.device)
        wq, s, b = ops.quantize(w, group_size, bits, scales_dtype=scales_dtype)
        m.weight = wq.view(torch.int32)
        m.scales, m.biases = s, b
        return m

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                 self.group_size, self.bits, self.mode)
        return y if self.bias is None else y + self.bias


JANGLinear = QuantizedLinear


class QuantizedSwitchLinear(torch.nn.Module):
    """Stacked expert projection: x @ dequantize(weight[indices])^T via gather_qmm."""

    def __init__(self, input_dims: int, output_dims: int, num_experts: int, bias: bool = False,
                 group_size: int = 64, bits: int = 4, *, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.input_dims, self.output_dims, self.num_experts = input_dims, output_dims, num_experts
        self.bits, self.group_size, self.mode = bits, group_size, "affine"
        g = input_dims // group_size
        self.register_buffer("weight", torch.zeros(
            (num_experts, output_dims, input_dims * bits // 32), dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros((num_experts, output_dims, g), dtype=dtype,
                                                   device=device))
        self.register_buffer("biases", torch.zeros_like(self.scales))
        self.bias = (torch.nn.Parameter(torch.zeros((num_experts, output_dims), dtype=dtype,
                                                    device=device), requires_grad=False)
                     if bias else None)

    def forward(self, x: torch.Tensor, indices: torch.Tensor,
                sorted_indices: bool = False) -> torch.Tensor:
        y = ops.gather_qmm(x, self.weight, self.scales, self.biases, rhs_indices=indices,
                           transpose=True, group_size=self.group_size, bits=self.bits,
                           mode=self.mode, sorted_indices=sorted_indices)
        if self.bias is not None:
            y = y + self.bias[indices.long()].unsqueeze(-2)
        return y

    def as_tuple(self):
        return (self.weight, self.scales, self.biases, self.bits)


class SwitchGLU(torch.nn.Module):
    """down(silu(gate(x)) * up(x)) per selected expert; returns [..., k, hidden]."""

    def __init__(self, input_dims: int, hidden_dims: int, num_experts: int,
                 group_size: int = 64, bits: int = 4, down_bits: int | None = None, *,
                 dtype=torch.bfloat16, device=None):
        super().__init__()
        kw = dict(group_size=group_size, dtype=dtype, device=device)
        self.gate_proj = QuantizedSwitchLinear(input_dims, hidden_dims, num_experts, bits=bits, **kw)
        self.up_proj = QuantizedSwitchLinear(input_dims, hidden_dims, num_experts, bits=bits, **kw)
        self.down_proj = QuantizedSwitchLinear(hidden_dims, input_dims, num_experts,
                                               bits=down_bits or bits, **kw)

    def group_size(self) -> int:
        """The one group size the three projections share (the SwitchGLU launches take one)."""
        gs = {self.gate_proj.group_size, self.up_proj.group_size, self.down_proj.group_size}
        if len(gs) != 1:
            raise ValueError(f"SwitchGLU projections have different group sizes {sorted(gs)}")
        return self.gate_proj.group_size

    def is_affine(self) -> bool:
        return all(p.mode == "affine" for p in (self.gate_proj, self.up_proj, self.down_proj))

    def forward(self, x: torch.Tensor, indices: torch.Tensor,
                swiglu_limit: float = 0.0) -> torch.Tensor:
        if self.is_affine() and swiglu_limit == 0.0:
            return ops.switch_glu(x, indices, self.gate_proj.as_tuple(), self.up_proj.as_tuple(),
                                  self.down_proj.as_tuple(), self.group_size())
        # MX-mode stacks (or a clamp): the three gathers of mlx_lm SwitchGLU (restated at
        # dots3/ops.py:195-223) with the elementwise SwiGLU between them
        xe = x.reshape(*x.shape[:-1], 1, 1, x.shape[-1])
        g = self.gate_proj(xe, indices)
        u = self.up_proj(xe, indices)
        h = ops.swiglu(g, u, swiglu_limit)
        return self.down_proj(h, indices).squeeze(-2)


class SwitchLinear(torch.nn.Module):
    """Float stacked-expert projection (mlx_lm SwitchLinear): x @ weight[indices]^T. A bundle
    that holds quantized tensors for it upgrades it to QuantizedSwitchLinear
    (:func:`upgrade_switch_to_quantized`, loader.py:1826-1848)."""

    def __init__(self, input_dims: int, output_dims: int, num_experts: int, bias: bool = False,
                 *, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.input_dims, self.output_dims, self.num_experts = input_dims, output_dims, num_experts
        self.weight = torch.nn.Parameter(torch.zeros((num_experts, output_dims, input_dims),
                                                     dtype=dtype, device=device),
                                         requires_grad=False)
        self.bias = (torch.nn.Parameter(torch.zeros((num_experts, output_dims), dtype=dtype,
                                                    device=device), requires_grad=False)
                     if bias else None)

    def forward(self, x: torch.Tensor, indices: torch.Tensor,
                sorted_indices: bool = False) -> torch.Tensor:
        # x [..., M, K] broadcast against indices as gather_qmm does; fp32 products
        bshape = x.shape[:-2]
        lhs = torch.arange(math.prod(bshape), device=x.device).reshape(bshape)
        lhs_b, rhs_b = torch.broadcast_tensors(lhs, indices.long())
        xs = x.reshape(-1, *x.shape[-2:])[lhs_b.reshape(-1)].float()
        w = self.weight[rhs_b.reshape(-1)].float().transpose(-1, -2).contiguous()
        y = torch.matmul(xs, w)
        if self.bias is not None:
            y = y + self.bias[rhs_b.reshape(-1)].float().unsqueeze(-2)
        return y.to(x.dtype).reshape(*lhs_b.shape, *y.shape[-2:])


def upgrade_switch_to_quantized(model: torch.nn.Module, bits: int, group_size: int,
                                names=None) -> list:
    """Replace SwitchLinear modules (all, or those in ``names``) with QuantizedSwitchLinear of
    the same dimensions (jang-tools/jang_tools/loader.py:1826-1848). Returns the paths."""
    done = []
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, SwitchLinear) or (names is not None and name not in names):
            continue
        q = QuantizedSwitchLinear(mod.input_dims, mod.output_dims, mod.num_experts,
                                  bias=mod.bias is not None, group_size=group_size, bits=bits,
                                  device=mod.weight.device)
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, leaf, q)
        done.append(name)
    return done


class DenseRouter(torch.nn.Module):
    """A MoE router kept in floating point (mistral4_mlx.py:343-352 MoEGate: the gate stays
    float; the loader dequantizes a quantized gate into it, loader.py:452-482): logits =
    x @ weight^T accumulated in fp32 and returned in the promoted type of x and the weight
    (float32 for a float32 gate, bfloat16 once the loader's dtype policy casts both)."""

    def __init__(self, dims: int, num_experts: int, *, dtype=torch.float32, device=None):
        super().__init__()
        self.in_features, self.out_features = dims, num_experts
        self.weight = torch.nn.Parameter(torch.zeros((num_experts, dims), dtype=dtype,
                                                     device=device), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = torch.matmul(x.float(), self.weight.float().t().contiguous())
        return out.to(torch.promote_types(x.dtype, self.weight.dtype))


class SharedExpertMLP(torch.nn.Module):
    """Dense SwiGLU MLP of quantized linears (the shared expert); swiglu_limit > 0 clamps
    gate <= L and up to [-L, L] (dsv41/model.py:1237-1245)."""

    def __init__(self, dims: int, hidden: int, group_size: int = 64, bits: int = 8, *,
                 swiglu_limit: float = 0.0, dtype=torch.bfloat16, device=None):
        super().__init__()
        kw = dict(group_size=group_size, bits=bits, dtype=dtype, device=device)
        self.swiglu_limit = swiglu_limit
        self.gate_proj = QuantizedLinear(dims, hidden, **kw)
        self.up_proj = QuantizedLinear(dims, hidden, **kw)
        self.down_proj = QuantizedLinear(hidden, dims, **kw)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        g, u = self.gate_proj, self.up_proj
        h = ops.quantized_swiglu(x, (g.weight, g.scales, g.biases, g.bits),
                                 (u.weight, u.scales, u.biases, u.bits), g.group_size,
                                 swiglu_limit=self.swiglu_limit)
        return self.down_proj(h)

    def as_tuples(self):
        """(w, scales, biases, group_size, bits) of gate, up and down (ops.moe_block)."""
        return tuple((m.weight, m.scales, m.biases, m.group_size, m.bits)
                     for m in (self.gate_proj, self.up_proj, self.down_proj))


class SparseMoeBlock(torch.nn.Module):
    """Router (quantized gate) -> top-k -> SwitchGLU -> combine with the shared expert.

    Router forms (ops.moe_route): ``score_func`` "softmax" (qwen4_exp/modeling.py:586-593,
    mistral4_mlx.py:355-387), "sigmoid" (dots3/ops.py:149-162, laguna/model.py:50-62) or
    "sqrtsoftplus" (dsv41/model.py:1184-1190); ``e_score_bias`` adds a per-expert selection bias
    (buffer ``e_score_correction_bias``); ``n_group``/``topk_group`` limit the selection to the
    best groups; ``routed_scaling_factor`` scales the weights.
    ``shared_expert_gate``: the 1-row linear whose sigmoid scales the shared expert's output
    (qwen4_exp/modeling.py:583,599). ``combine`` "after" applies the routing weights to the
    experts' outputs (qwen4 / mlx_lm), "before" to h before the down projection (dsv41);
    ``swiglu_limit`` is the SwiGLU clamp of dsv41/model.py:1214-1218."""

    def __init__(self, dims: int, expert_hidden: int, num_experts: int, top_k: int, *,
                 norm_topk_prob: bool = True, shared_hidden: int | None = None,
                 group_size: int = 64, bits: int = 2, router_bits: int = 8,
                 shared_bits: int = 8, shared_group_size: int = 64, score_func: str = "softmax",
                 routed_scaling_factor: float = 1.0, renorm_eps: float | None = None,
                 e_score_bias: bool = False, n_group: int = 1, topk_group: int = 1,
                 shared_expert_gate: bool = False, swiglu_limit: float = 0.0,
                 combine: str = "after", dtype=torch.bfloat16, device=None):
        super().__init__()
        if shared_expert_gate and not shared_hidden:
            raise ValueError("shared_expert_gate needs a shared expert")
        self.top_k, self.norm_topk_prob = top_k, norm_topk_prob
        self.score_func, self.routed_scaling_factor = score_func, routed_scaling_factor
        self.renorm_eps, self.n_group, self.topk_group = renorm_eps, n_group, topk_group
        self.swiglu_limit, self.combine = swiglu_limit, combine
        self.gate = QuantizedLinear(dims, num_experts, group_size=64, bits=router_bits,
                                    dtype=dtype, device=device)
        self.switch_mlp = SwitchGLU(dims, expert_hidden, num_experts, group_size=group_size,
                                    bits=bits, dtype=dtype, device=device)
        self.shared_expert = (SharedExpertMLP(dims, shared_hidden, shared_group_size, shared_bits,
                                              swiglu_limit=swiglu_limit, dtype=dtype,
                                              device=device)
                              if shared_hidden else None)
        self.shared_expert_gate = (QuantizedLinear(dims, 1, group_size=64, bits=router_bits,
                                                   dtype=dtype, device=device)
                                   if shared_expert_gate else None)
        if e_score_bias:
            self.register_buffer("e_score_correction_bias",
                                 torch.zeros(num_experts, dtype=torch.float32, device=device))
        else:
            self.e_score_correction_bias = None

    def _route_kw(self):
        return dict(score=self.score_func, renorm=self.norm_topk_prob, renorm_eps=self.renorm_eps,
                    scaling=self.routed_scaling_factor, score_bias=self.e_score_correction_bias,
                    n_group=self.n_group, topk_group=self.topk_group)

    def route(self, x: torch.Tensor):
        """(expert ids, weights) of the router for x."""
        kw = self._route_kw()
        return ops.moe_route(self.gate(x), self.top_k, kw.pop("renorm"), **kw)

    def forward(self, x: torch.Tensor, logits: torch.Tensor | None = None) -> torch.Tensor:
        if logits is None:
            logits = self.gate(x)  # the router's bf16/f16 output is read as it is
        sgl = self.shared_expert_gate(x) if self.shared_expert_gate is not None else None
        m = self.switch_mlp
        if not m.is_affine():
            # MX-mode experts: routing, the three gathers and the combine as separate launches
            if self.combine != "after" or sgl is not None:
                raise NotImplementedError("MX-mode experts take the after-down combine without "
                                          "a shared-expert gate")
            kw = self._route_kw()
            idx, w = ops.moe_route(logits, self.top_k, kw.pop("renorm"), **kw)
            y = m(x, idx, self.swiglu_limit)
            shared = self.shared_expert(x) if self.shared_expert is not None else None
            return ops.moe_combine(y, w, shared)
        # routing, the routed experts, the shared expert and the combine in one call; at decode
        # sizes the routed experts take two launches (gate|up routing for itself, then down
        # with the combine inside).
        out, _, _ = ops.moe_block(
            x, logits, self.top_k, m.gate_proj.as_tuple(), m.up_proj.as_tuple(),
            m.down_proj.as_tuple(), m.group_size(),
            shared=self.shared_expert.as_tuples() if self.shared_expert is not None else None,
            shared_gate=sgl, combine=self.combine, swiglu_limit=self.swiglu_limit,
            **self._route_kw())
        return out
