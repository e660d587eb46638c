"""A JANG v2 bundle loaded onto the GPU modules and run: the 1-bit storage expansion of a
manifest-listed expert stack (bit-exact to the oracle's), the bits / group-size fix, and the
loaded MoE block's output against the oracle's composition."""
import numpy as np
import pytest
import torch

from jangq_amd import loader
from jangq_amd import nn as jnn
from oracle import jangq_oracle as O
from tests._util import assert_close, to_tensor, values_of
from tests.bundle_util import quantized, tensors_of, write_bundle

pytestmark = pytest.mark.gpu

H, I, E, K_TOP = 256, 128, 8, 2


def test_loaded_block_matches_oracle(tmp_path):
    q = {"gate": quantized(E, H, 8, 64, 1),
         "switch_mlp.gate_proj": quantized(I, H, 3, 128, 2, experts=E),
         "switch_mlp.up_proj": quantized(I, H, 3, 128, 3, experts=E),
         "shared_expert.gate_proj": quantized(256, H, 8, 64, 5),
         "shared_expert.up_proj": quantized(256, H, 8, 64, 6),
         "shared_expert.down_proj": quantized(H, 256, 8, 64, 7)}
    t = {}
    for name, (p, s, b) in q.items():
        t.update(tensors_of(name, p, s, b))
    # down stack stored as 1-bit codes (manifest), with 2-bit-range scales and biases
    rng = np.random.default_rng(11)
    one = rng.integers(0, 2**32, (E, H, I // 32), dtype=np.uint64).astype(np.uint32)
    _, ds, db = quantized(H, I, 2, 128, 4, experts=E)
    t.update(tensors_of("switch_mlp.down_proj", one, ds, db))
    write_bundle(tmp_path, t, manifest={"switch_mlp.down_proj": {"storage_bits": 1, "bits": 1}})

    blk = jnn.SparseMoeBlock(H, I, E, K_TOP, shared_hidden=256, group_size=64, bits=2,
                             router_bits=8, shared_bits=8, device="cuda")
    rep = loader.load_bundle_into(blk, tmp_path)
    assert rep.expanded == ["switch_mlp.down_proj"] and not rep.missing and not rep.unexpected
    two = O.expand_1bit_to_2bit(one)
    dn = blk.switch_mlp.down_proj
    assert (dn.bits, dn.group_size) == (2, 128)
    np.testing.assert_array_equal(dn.weight.cpu().numpy().view(np.uint32), two)

    x = O.round_bf16(np.random.default_rng(12).standard_normal((3, H), dtype=np.float32))
    y = blk(to_tensor(x, "bf16"))
    f = lambda name: (q[name][0], O.sidecar_f32(q[name][1], "bf16"),
                      O.sidecar_f32(q[name][2], "bf16"))
    gp, gs_, gb = f("gate")
    logits = O.round_bf16(O.quantized_matmul(x, gp, gs_, gb, 8, 64))
    idx, sc = O.route_topk(logits, K_TOP)
    # each pair in the stock order and roundings (g, u, h and the expert output in bf16)
    outs = []
    for t_ in range(x.shape[0]):
        rows = []
        for j in range(K_TOP):
            e = idx[t_, j]
            g = O.round_bf16(O.quantized_matmul(x[t_:t_ + 1], q["switch_mlp.gate_proj"][0][e],
                                                O.sidecar_f32(q["switch_mlp.gate_proj"][1][e], "bf16"),
                                                O.sidecar_f32(q["switch_mlp.gate_proj"][2][e], "bf16"), 3, 128))
            u = O.round_bf16(O.quantized_matmul(x[t_:t_ + 1], q["switch_mlp.up_proj"][0][e],
                                                O.sidecar_f32(q["switch_mlp.up_proj"][1][e], "bf16"),
                                                O.sidecar_f32(q["switch_mlp.up_proj"][2][e], "bf16"), 3, 128))
            h = O.round_bf16(O.silu(g) * u.astype(np.float64))
            rows.append(O.round_bf16(O.quantized_matmul(h, two[e], O.sidecar_f32(ds[e], "bf16"),
                                                        O.sidecar_f32(db[e], "bf16"), 2, 128))[0])
        outs.append(np.stack(rows))
    sw = np.stack(outs)
    routed = O.round_bf16((sw.astype(np.float64) * sc[..., None]).sum(1))
    sg, su, sd = f("shared_expert.gate_proj"), f("shared_expert.up_proj"), f("shared_expert.down_proj")
    g = O.round_bf16(O.quantized_matmul(x, *sg, 8, 64))
    u = O.round_bf16(O.quantized_matmul(x, *su, 8, 64))
    h = O.round_bf16(O.silu(g) * u)
    shared = O.round_bf16(O.quantized_matmul(h, *sd, 8, 64))
    assert_close(values_of(y), O.round_bf16(routed + shared), "loaded moe block")


class _RouterModel(torch.nn.Module):
    def __init__(self, experts, dims):
        super().__init__()
        self.gate = jnn.DenseRouter(dims, experts, device="cuda")


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32), (3, 128)])
def test_quantized_gate_into_float_router(tmp_path, bits, gs):
    """A quantized gate loaded into a float router is dequantized to fp32 (loader.py:452-482),
    bit-exact to the oracle's dequantization; the router's logits follow in fp32."""
    Ex, D = 16, 512
    p, s, b = quantized(Ex, D, bits, gs, 40 + bits)
    write_bundle(tmp_path, tensors_of("gate", p, s, b))
    m = _RouterModel(Ex, D)
    rep = loader.load_bundle_into(m, tmp_path)
    assert rep.fixed["gate"] == ("dequantized", bits, gs) and not rep.unexpected
    ref = O.dequantize_affine(p, O.sidecar_f32(s, "bf16"), O.sidecar_f32(b, "bf16"), bits, gs)
    assert m.gate.weight.dtype == torch.float32
    np.testing.assert_array_equal(m.gate.weight.cpu().numpy(), ref.astype(np.float32))
    x = O.round_bf16(np.random.default_rng(1).standard_normal((3, D), dtype=np.float32))
    y = m.gate(to_tensor(x, "bf16"))
    assert y.dtype == torch.float32
    exact = x.astype(np.float64) @ ref.astype(np.float64).T
    np.testing.assert_allclose(values_of(y), exact, rtol=1e-4, atol=1e-4)


def test_mx_expert_stack_loaded_and_run(tmp_path):
    """An mxfp4 expert stack in a bundle loads onto the block's SwitchGLU (mode, bits and group
    size from the shapes, no biases) and the loaded experts run the MX gathers."""
    rng = np.random.default_rng(21)
    t = {}
    t.update(tensors_of("gate", *quantized(E, H, 8, 64, 1)))
    host = {}
    for name, (n, kk) in {"gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}.items():
        packed = rng.integers(0, 2**32, (E, n, kk // 8), dtype=np.uint64).astype(np.uint32)
        sc = rng.integers(112, 122, (E, n, kk // 32)).astype(np.uint8)
        host[name] = (packed, sc)
        t[f"switch_mlp.{name}.weight"] = torch.from_numpy(packed.view(np.int32)).view(torch.uint32)
        t[f"switch_mlp.{name}.scales"] = torch.from_numpy(sc)
    write_bundle(tmp_path, t)
    blk = jnn.SparseMoeBlock(H, I, E, K_TOP, group_size=64, bits=2, router_bits=8, device="cuda")
    rep = loader.load_bundle_into(blk, tmp_path)
    assert all(rep.fixed[f"switch_mlp.{n}"] == ("mxfp4", 4, 32)
               for n in ("gate_proj", "up_proj", "down_proj"))
    x = O.round_bf16(rng.standard_normal((2, H), dtype=np.float32))
    idx = np.array([[1, 5], [7, 0]], dtype=np.int32)
    y = blk.switch_mlp(to_tensor(x, "bf16"), torch.from_numpy(idx).cuda())
    exact = np.zeros((2, K_TOP, H))
    for t_ in range(2):
        for j in range(K_TOP):
            e = idx[t_, j]
            mm = lambda v, nm: O.mx_quantized_matmul(v, host[nm][0][e], host[nm][1][e], "mxfp4")
            g = O.round_bf16(mm(x[t_:t_ + 1], "gate_proj"))
            u = O.round_bf16(mm(x[t_:t_ + 1], "up_proj"))
            exact[t_, j] = mm(O.round_bf16(O.glu(g, u)), "down_proj")[0]
    assert_close(values_of(y), O.round_bf16(exact), "loaded mx experts", exact=exact,
                 out_dtype="bf16", ulps=1)


def test_aligned_bundle_loads_the_same(tmp_path):
    """The same bundle repacked into dtype-aligned shards (read as views of the mapped files)
    loads tensors identical to the original's (read through safetensors)."""
    from jangq_amd import shards
    t = {}
    t.update(tensors_of("gate", *quantized(E, H, 8, 64, 1)))
    t.update(tensors_of("switch_mlp.gate_proj", *quantized(I, H, 3, 128, 2, experts=E)))
    t.update(tensors_of("switch_mlp.up_proj", *quantized(I, H, 3, 128, 3, experts=E)))
    t.update(tensors_of("switch_mlp.down_proj", *quantized(H, I, 4, 64, 4, experts=E)))
    t["norm.odd"] = torch.ones(3, dtype=torch.bfloat16)  # 6 bytes: misaligns what follows
    write_bundle(tmp_path / "src", t)
    shards.repack_bundle(tmp_path / "src", tmp_path / "al")
    for p in (tmp_path / "al").glob("*.safetensors"):
        assert shards.verify_alignment(p)[1] == 0
    mk = lambda: jnn.SparseMoeBlock(H, I, E, K_TOP, group_size=64, bits=2, router_bits=8,
                                    device="cuda")
    a, b = mk(), mk()
    ra = loader.load_bundle_into(a, tmp_path / "src")
    rb = loader.load_bundle_into(b, tmp_path / "al")
    assert ra.fixed == rb.fixed and ra.loaded == rb.loaded and ra.unexpected == rb.unexpected
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert sa[k].device.type == "cuda" and torch.equal(sa[k], sb[k]), k
