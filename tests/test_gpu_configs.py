"""GPU parity at the BASELINE configs' full sizes, through the operators the bench times.

The weights are seeded random codes built on the GPU (tests._util.RandQ): a 512-expert
stack is too large for the CPU quantizer, and any codes, scales and biases are a valid
affine weight. The oracle dequantizes only what a checked output needs (the selected
experts of sampled tokens, a column slice of a prefill output) and accumulates in fp64.
Tolerances: rel-L2 <= 1e-3 and max-abs <= 2e-2 beyond the output rounding (north star); the
MoE block outputs, whose stages round to bf16 in turn, are allowed one output ulp for that
rounding (tests._util.assert_close, ulps=1).

Config 5 routing follows its recipe: logits ~N(0,1) with +2 on round(0.1 * 512) = 51
experts chosen by a seeded permutation, softmax -> top-10 -> renormalise, plus the
unweighted shared expert (jang-tools/jang_tools/qwen4_exp/modeling.py:587-597)."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from jangq_amd import nn as jnn
from oracle import jangq_oracle as O
from tests._util import RandQ, assert_close, to_tensor, values_of

pytestmark = pytest.mark.gpu


def _deq(q: RandQ, e=None, rows=None):
    w, s, b = q.host(e, rows)
    return O.dequantize_affine(w, s, b, q.bits, q.gs).astype(np.float64)


def _rb(v, dt="bf16"):
    return O.round_to(v, dt).astype(np.float64)


def _moe_token_oracle(x, ids, w, g, u, d, shared=None):
    """One token of the MoE block: per slot round(down(round(silu(round(g)) * round(u)))),
    the fp64 slot-order weighted sum rounded, + the shared expert's output rounded again.
    Returns (output, value before the last rounding)."""
    cache = {}

    def W(q, e):
        key = (id(q), int(e))
        if key not in cache:
            cache[key] = _deq(q, e)
        return cache[key]

    acc = np.zeros(x.shape[-1], np.float64)
    for j, e in enumerate(ids):
        gv = _rb(x @ W(g, e).T)
        uv = _rb(x @ W(u, e).T)
        h = _rb(O.silu(gv) * uv)
        acc += w[j] * _rb(h @ W(d, e).T)
    if shared is None:
        return O.round_bf16(acc), acc
    r = _rb(acc) + shared
    return O.round_bf16(r), r


def _shared_oracle(x, sg, su, sd, pre=False):
    gv = _rb(x @ _deq(sg).T)
    uv = _rb(x @ _deq(su).T)
    h = _rb(O.silu(gv) * uv)
    y = h @ _deq(sd).T
    return (_rb(y), y) if pre else _rb(y)


def _skewed_logits(T, E, seed, skew):
    rng = np.random.default_rng(seed)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    if skew:
        lg[:, rng.permutation(E)[: round(0.1 * E)]] += 2.0
    return lg


def _block(E, H, I, bits, gs, k, shared_I, seed):
    blk = jnn.SparseMoeBlock(H, I, E, k, shared_hidden=shared_I, group_size=gs, bits=bits,
                             device="cuda")
    qs = {}
    for name, proj, rows, cols in (("g", blk.switch_mlp.gate_proj, I, H),
                                   ("u", blk.switch_mlp.up_proj, I, H),
                                   ("d", blk.switch_mlp.down_proj, H, I)):
        q = RandQ(rows, cols, bits, gs, seed=seed + len(qs), experts=E)
        proj.weight, proj.scales, proj.biases = q.dw, q.ds, q.db
        qs[name] = q
    if shared_I:
        for name, lin, rows, cols in (("sg", blk.shared_expert.gate_proj, shared_I, H),
                                      ("su", blk.shared_expert.up_proj, shared_I, H),
                                      ("sd", blk.shared_expert.down_proj, H, shared_I)):
            q = RandQ(rows, cols, 8, 64, seed=seed + 10 + len(qs))
            lin.weight, lin.scales, lin.biases = q.dw, q.ds, q.db
            qs[name] = q
    return blk, qs


def _check_block(blk, qs, T, E, H, k, seed, skew, sample):
    rng = np.random.default_rng(seed)
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    logits = _skewed_logits(T, E, seed + 1, skew)
    tx, tl = to_tensor(x, "bf16"), torch.from_numpy(logits).cuda()
    y = values_of(blk(tx, logits=tl))
    # ids of every token against the oracle's top-k
    ids, w = O.route_topk(logits, k, renorm=True)
    m = blk.switch_mlp
    out, gid, gw = jq.moe_experts(tx, tl, k, m.gate_proj.as_tuple(), m.up_proj.as_tuple(),
                                  m.down_proj.as_tuple(), m.group_size(), None, True)
    np.testing.assert_array_equal(gid.cpu().numpy(), ids)
    np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=2e-6, atol=1e-7)
    # the one-call form against the routing launch + SwitchGLU-with-combine (bit equality)
    rid, rw = jq.moe_route(tl, k, True)
    two = jq.switch_glu_combine(tx, rid, rw, m.gate_proj.as_tuple(), m.up_proj.as_tuple(),
                                m.down_proj.as_tuple(), m.group_size(), None)
    if not torch.equal(out.view(torch.int16), two.view(torch.int16)):
        bad = (out.view(torch.int16) != two.view(torch.int16)).nonzero().tolist()
        d = (out.float() - two.float()).abs().max().item()
        raise AssertionError(f"moe_experts != route + combine at {len(bad)} outputs (first "
                             f"{bad[:4]}), max |diff| {d}; ids equal "
                             f"{torch.equal(gid, rid)}, weights bit-equal "
                             f"{torch.equal(gw.view(torch.int32), rw.view(torch.int32))}")
    for t in sample:
        sh = None
        if "sg" in qs:
            sh = _shared_oracle(x[t].astype(np.float64), qs["sg"], qs["su"], qs["sd"])
        ref, pre = _moe_token_oracle(x[t].astype(np.float64), ids[t], w[t], qs["g"], qs["u"],
                                     qs["d"], sh)
        assert_close(y[t], ref, f"block token {t}", exact=pre, out_dtype="bf16", ulps=1)
        if sh is None:
            assert_close(values_of(out)[t], ref, f"moe_experts token {t}", exact=pre,
                         out_dtype="bf16", ulps=1)


@pytest.fixture(scope="module")
def c5_block():
    """Config 5: 512 experts, H 4096, I 1024, 2-bit g128; shared expert I 4096 at 8-bit g64."""
    blk, qs = _block(512, 4096, 1024, 2, 128, 10, 4096, seed=501)
    yield blk, qs
    del blk, qs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,sample", [(1, (0,)), (32, (0, 13, 31))])
def test_c5_moe_layer_full_size(c5_block, T, sample):
    blk, qs = c5_block
    print(f"config 5 T={T}", flush=True)
    _check_block(blk, qs, T, 512, 4096, 10, seed=505 + T, skew=True, sample=sample)


def test_c5_router_and_shared_full_size(c5_block):
    """The 8-bit router GEMV (512 x 4096) and the shared expert alone at T = 1 and 32."""
    blk, qs = c5_block
    rq = RandQ(512, 4096, 8, 64, seed=503)
    for T in (1, 32):
        rng = np.random.default_rng(T)
        x = O.round_bf16(rng.standard_normal((T, 4096), dtype=np.float32))
        tx = to_tensor(x, "bf16")
        lg = values_of(jq.quantized_matmul(tx, rq.dw, rq.ds, rq.db, True, 64, 8))
        ref = x.astype(np.float64) @ _deq(rq).T
        assert_close(lg, O.round_bf16(ref), f"router T{T}", exact=ref, out_dtype="bf16")
        sh = values_of(blk.shared_expert(tx))
        for t in (0, T - 1):
            r, pre = _shared_oracle(x[t].astype(np.float64), qs["sg"], qs["su"], qs["sd"], True)
            assert_close(sh[t], r, f"shared T{T} t{t}", exact=pre, out_dtype="bf16", ulps=1)


@pytest.fixture(scope="module")
def c3_block():
    """Config 3: 128 experts, H 4096, I 2048, 2-bit g64, top-4, no shared expert."""
    blk, qs = _block(128, 4096, 2048, 2, 64, 4, None, seed=301)
    yield blk, qs
    del blk, qs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,sample", [(1, (0,)), (16, (0, 7, 15)), (64, (0, 33, 63))])
def test_c3_moe_layer_full_size(c3_block, T, sample):
    blk, qs = c3_block
    print(f"config 3 T={T}", flush=True)
    _check_block(blk, qs, T, 128, 4096, 4, seed=303 + T, skew=False, sample=sample)


# Config 2 block projections: (N, K, bits) of q, k, v, o, gate, up, down.
C2 = {"q": (4096, 4096, 6), "k": (1024, 4096, 6), "v": (1024, 4096, 6), "o": (4096, 4096, 6),
      "g": (14336, 4096, 3), "u": (14336, 4096, 3), "d": (4096, 14336, 2)}


@pytest.fixture(scope="module")
def c2_layer():
    layer = {n: RandQ(N, K, b, 64, seed=200 + i) for i, (n, (N, K, b)) in enumerate(C2.items())}
    yield layer
    del layer
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M", [1, 8, 32])
def test_c2_block_full_size(c2_layer, M):
    """Every launch of the config-2 block step at batch M, as the bench runs it: q|k|v and
    gate|up grouped, o and down alone; rows checked on a slice of each output."""
    L = c2_layer
    print(f"config 2 M={M}", flush=True)
    rng = np.random.default_rng(290 + M)
    acts = {K: O.round_bf16(rng.standard_normal((M, K), dtype=np.float32)) for K in (4096, 14336)}
    tx = {K: to_tensor(a, "bf16") for K, a in acts.items()}
    tup = lambda n: (L[n].dw, L[n].ds, L[n].db, 64, L[n].bits)  # noqa: E731
    outs = dict(zip("qkv", jq.quantized_matmul_multi(tx[4096], [tup("q"), tup("k"), tup("v")])))
    outs.update(zip("gu", jq.quantized_matmul_multi(tx[4096], [tup("g"), tup("u")])))
    for n in "od":
        K = C2[n][1]
        outs[n] = jq.quantized_matmul(tx[K], L[n].dw, L[n].ds, L[n].db, True, 64, L[n].bits)
    for n, (N, K, bits) in C2.items():
        rows = slice(0, 256) if N <= 4096 else slice(N - 300, N)
        ref = acts[K].astype(np.float64) @ _deq(L[n], rows=rows).T
        got = values_of(outs[n])[:, rows]
        assert tuple(outs[n].shape) == (M, N)
        assert_close(got, O.round_bf16(ref), f"c2 {n} M{M}", exact=ref, out_dtype="bf16")


@pytest.mark.parametrize("bits", [4, 3])
def test_c4_prefill_full_size(bits):
    """Config 4: M = 2048, K = 4096, N = 14336 at 4- and 3-bit g64, the full launch, checked
    on two column slices (the first and the last, ragged against the 256-column tile)."""
    M, K, N = 2048, 4096, 14336
    q = RandQ(N, K, bits, 64, seed=400 + bits)
    rng = np.random.default_rng(402)
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    print(f"config 4 bits={bits}", flush=True)
    y = jq.quantized_matmul(to_tensor(x, "bf16"), q.dw, q.ds, q.db, True, 64, bits)
    assert tuple(y.shape) == (M, N)
    yv = values_of(y)
    for cols in (slice(0, 384), slice(N - 200, N)):
        ref = x.astype(np.float64) @ _deq(q, rows=cols).T
        assert_close(yv[:, cols], O.round_bf16(ref), f"c4 b{bits} cols {cols}", exact=ref,
                     out_dtype="bf16")
    del q, y
    torch.cuda.empty_cache()


@pytest.mark.parametrize("E,k,I,gs", [(8, 4, 2048, 64), (16, 10, 1024, 128)])
def test_routed_gateup_at_h4096(E, k, I, gs):
    """The gate|up launch that routes for itself at H = 4096 (64 lane chunks per 2-bit row:
    the one-row-group instantiation) against the routing launch + SwitchGLU-with-combine,
    bit for bit, and against the oracle."""
    H = 4096
    g = RandQ(I, H, 2, gs, seed=61, experts=E)
    u = RandQ(I, H, 2, gs, seed=62, experts=E)
    d = RandQ(H, I, 2, gs, seed=63, experts=E)
    rng = np.random.default_rng(E * k)
    x = O.round_bf16(rng.standard_normal((1, H), dtype=np.float32))
    logits = rng.standard_normal((1, E)).astype(np.float32)
    tx, tl = to_tensor(x, "bf16"), torch.from_numpy(logits).cuda()
    out, ids, w = jq.moe_experts(tx, tl, k, g.tup(), u.tup(), d.tup(), gs, None, True)
    ids2, w2 = jq.moe_route(tl, k, True)
    two = jq.switch_glu_combine(tx, ids2, w2, g.tup(), u.tup(), d.tup(), gs, None)
    assert torch.equal(ids, ids2) and torch.equal(w, w2)
    assert torch.equal(out.view(torch.int16), two.view(torch.int16))
    rid, rw = O.route_topk(logits, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rid)
    ref, pre = _moe_token_oracle(x[0].astype(np.float64), rid[0], rw[0], g, u, d)
    assert_close(values_of(out)[0], ref, f"routed gate|up E{E} k{k}", exact=pre, out_dtype="bf16",
                 ulps=1)
