"""GPU parity of the MoE path: router top-k, gather_qmm (device grouping by expert) and the
fused SwitchGLU launches, against the oracle's per-pair loops."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from jangq_amd import nn as jnn
from oracle import jangq_oracle as O
from tests._util import QWeight, RandQ, assert_close, to_tensor, values_of

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,E,k", [(1, 128, 4), (16, 128, 4), (64, 128, 4), (32, 512, 10),
                                   (5, 64, 1)])
def test_route_topk(T, E, k):
    rng = np.random.default_rng(T * 7 + E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if E == 512:  # config 5: +2 on 10% of experts
        logits[:, rng.permutation(E)[: round(0.1 * E)]] += 2.0
    idx, w = jq.moe_route(torch.from_numpy(logits).cuda(), k, renorm=True)
    ridx, rw = O.route_topk(logits, k, renorm=True)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    _, w2 = jq.moe_route(torch.from_numpy(logits).cuda(), k, renorm=False)
    np.testing.assert_allclose(w2.cpu().numpy(), O.route_topk(logits, k, renorm=False)[1],
                               rtol=2e-6, atol=1e-8)


def _stack(E, N, K, bits, gs, seed):
    return QWeight(N, K, bits, gs, seed=seed, experts=E)


@pytest.mark.parametrize("bits,gs", [(2, 64), (4, 32), (3, 128), (8, 64)])
@pytest.mark.parametrize("M", [1, 3])
def test_gather_qmm_pairs(bits, gs, M):
    E, N, K = 8, 128, 256
    qw = _stack(E, N, K, bits, gs, seed=bits + gs)
    rng = np.random.default_rng(5)
    B = 6
    x = O.round_bf16(rng.standard_normal((B, M, K), dtype=np.float32))
    lhs = np.array([0, 5, 5, 2, 3, 1, 0, 4, 2, 2], np.int32)
    rhs = np.array([7, 0, 3, 3, 3, 1, 7, 6, 0, 3], np.int32)
    y = jq.gather_qmm(to_tensor(x, "bf16"), qw.dw, qw.ds, qw.db,
                      torch.from_numpy(lhs).cuda(), torch.from_numpy(rhs).cuda(),
                      group_size=gs, bits=bits)
    ref = O.gather_qmm(x, qw.packed, qw.s, qw.b, lhs, rhs, bits, gs)
    assert tuple(y.shape) == (len(lhs), M, N)
    assert_close(values_of(y), O.round_bf16(ref), f"gather b{bits} g{gs} M{M}")


@pytest.mark.parametrize("bits,gs", [(2, 64), (4, 128)])
def test_gather_qmm_many_rows_per_expert(bits, gs):
    """Prefill-like grouping (hundreds of rows over 4 experts) takes the 16-row-tile GEMM."""
    E, N, K, n = 4, 96, 256, 300
    qw = _stack(E, N, K, bits, gs, seed=21)
    rng = np.random.default_rng(21)
    x = O.round_bf16(rng.standard_normal((n, 1, K), dtype=np.float32))
    rhs = rng.integers(0, E, size=n).astype(np.int32)
    rhs[:7] = 3  # skew
    y = jq.gather_qmm(to_tensor(x, "bf16"), qw.dw, qw.ds, qw.db,
                      rhs_indices=torch.from_numpy(rhs).cuda(), group_size=gs, bits=bits)
    ref = O.gather_qmm(x, qw.packed, qw.s, qw.b, np.arange(n), rhs, bits, gs)
    assert_close(values_of(y), O.round_bf16(ref), "many rows per expert")


def test_gather_qmm_mlx_broadcasting_and_sorted_flag():
    """SwitchGLU call shape: x [T,1,1,K], rhs [T,k] -> out [T,k,1,N]; the sorted path
    (_gather_sort: rows permuted by expert, sorted_indices=True) gives the same rows."""
    E, N, K, T, k = 16, 64, 128, 20, 4
    qw = _stack(E, N, K, 4, 64, seed=9)
    rng = np.random.default_rng(9)
    x = O.round_bf16(rng.standard_normal((T, K), dtype=np.float32))
    inds = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    tx = to_tensor(x, "bf16")
    y = jq.gather_qmm(tx.reshape(T, 1, 1, K), qw.dw, qw.ds, qw.db,
                      rhs_indices=torch.from_numpy(inds).cuda(), group_size=64, bits=4)
    assert tuple(y.shape) == (T, k, 1, N)
    ref = O.gather_qmm(x[:, None, :], qw.packed, qw.s, qw.b, np.repeat(np.arange(T), k),
                       inds.reshape(-1), 4, 64)
    assert_close(values_of(y).reshape(T * k, N), O.round_bf16(ref[:, 0]), "broadcast gather")
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    ys = jq.gather_qmm(tx[torch.from_numpy(order // k).cuda()].reshape(T * k, 1, K), qw.dw, qw.ds,
                       qw.db, rhs_indices=torch.from_numpy(flat[order]).cuda(), group_size=64,
                       bits=4, sorted_indices=True)
    inv = np.argsort(order)
    assert torch.equal(ys[torch.from_numpy(inv).cuda()].reshape(T, k, 1, N), y)


@pytest.mark.parametrize("bits,gs,M,xdt", [(2, 64, 1, "bf16"), (3, 128, 1, "bf16"),
                                           (4, 128, 2, "bf16"), (6, 64, 1, "f16"),
                                           (8, 128, 1, "bf16"), (5, 64, 1, "bf16")])
def test_gather_qmm_matrix_core_tiles(bits, gs, M, xdt):
    """Hundreds of plan rows over 16 experts (about 12 per expert, one skewed): the
    matrix-core tiles with LDS-streamed weights; ragged N, gathered x rows, M rows per pair."""
    E, N, K, n, B = 16, 100, 512, 200, 40
    qw = QWeight(N, K, bits, gs, seed=bits * 3 + gs, experts=E, sidecar=xdt)
    rng = np.random.default_rng(bits + gs + M)
    x = O.round_to(rng.standard_normal((B, M, K), dtype=np.float32), xdt)
    lhs = rng.integers(0, B, size=n).astype(np.int32)
    rhs = rng.integers(0, E, size=n).astype(np.int32)
    rhs[:9] = 5
    y = jq.gather_qmm(to_tensor(x, xdt), qw.dw, qw.ds, qw.db, torch.from_numpy(lhs).cuda(),
                      torch.from_numpy(rhs).cuda(), group_size=gs, bits=bits)
    ref = O.gather_qmm(x, qw.packed, qw.s, qw.b, lhs, rhs, bits, gs)
    assert tuple(y.shape) == (n, M, N)
    assert_close(values_of(y), O.round_to(ref, xdt), f"gather tiles b{bits} g{gs} M{M} {xdt}",
                 exact=ref, out_dtype=xdt)


@pytest.mark.parametrize("T,k,E,H,I,bits_gu,bits_d,gs,xdt",
                         [(64, 4, 32, 512, 256, 2, 2, 64, "bf16"),
                          (64, 4, 32, 512, 256, 3, 4, 64, "bf16"),
                          (64, 4, 32, 512, 256, 2, 3, 128, "bf16"),
                          (64, 4, 32, 512, 384, 4, 2, 64, "f16"),
                          (32, 4, 16, 4096, 512, 2, 2, 64, "bf16")])
def test_switch_glu_matrix_core_tiles(T, k, E, H, I, bits_gu, bits_d, gs, xdt):
    """SwitchGLU with several tokens per selected expert: gate|up (+ SiLU) and down on the
    matrix-core tiles (K = 4096 spreads a row over eight waves)."""
    g = QWeight(I, H, bits_gu, gs, seed=31, experts=E, sidecar=xdt)
    u = QWeight(I, H, bits_gu, gs, seed=32, experts=E, sidecar=xdt)
    d = QWeight(H, I, bits_d, gs, seed=33, experts=E, sidecar=xdt)
    rng = np.random.default_rng(T + H)
    x = O.round_to(rng.standard_normal((T, H), dtype=np.float32), xdt)
    inds = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    out = jq.switch_glu(to_tensor(x, xdt), torch.from_numpy(inds).cuda(),
                        (g.dw, g.ds, g.db, bits_gu), (u.dw, u.ds, u.db, bits_gu),
                        (d.dw, d.ds, d.db, bits_d), gs)
    ref, _ = O.switch_glu(x, inds, (g.packed, g.s, g.b, bits_gu), (u.packed, u.s, u.b, bits_gu),
                          (d.packed, d.s, d.b, bits_d), gs, xdt)
    assert tuple(out.shape) == (T, k, H)
    assert_close(values_of(out), ref, f"switch_glu tiles T{T} H{H} I{I} {xdt}")


@pytest.mark.parametrize("T,k,E,bits_gu,bits_d", [(1, 4, 32, 2, 2), (16, 4, 32, 2, 2),
                                                  (64, 4, 32, 3, 4), (7, 2, 8, 8, 6),
                                                  (160, 2, 4, 2, 3)])
def test_switch_glu(T, k, E, bits_gu, bits_d):
    H, I, gs = 256, 128, 64
    g = _stack(E, I, H, bits_gu, gs, seed=1)
    u = _stack(E, I, H, bits_gu, gs, seed=2)
    d = _stack(E, H, I, bits_d, gs, seed=3)
    rng = np.random.default_rng(T)
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    inds = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    out = jq.switch_glu(to_tensor(x, "bf16"), torch.from_numpy(inds).cuda(),
                        (g.dw, g.ds, g.db, bits_gu), (u.dw, u.ds, u.db, bits_gu),
                        (d.dw, d.ds, d.db, bits_d), gs)
    ref, _ = O.switch_glu(x, inds, (g.packed, g.s, g.b, bits_gu), (u.packed, u.s, u.b, bits_gu),
                          (d.packed, d.s, d.b, bits_d), gs, "bf16")
    assert tuple(out.shape) == (T, k, H)
    assert_close(values_of(out), ref, f"switch_glu T{T} k{k}")


@pytest.mark.parametrize("T", [1, 5])
def test_moe_block_module(T):
    """Router (8-bit gate) -> top-k -> SwitchGLU -> weighted sum + shared expert (decode-size
    fused SwiGLU at T = 1, grouped dense launch at T = 5)."""
    H, I, E, k = 256, 128, 16, 4
    blk = jnn.SparseMoeBlock(H, I, E, k, shared_hidden=256, bits=2, device="cuda")
    rng = np.random.default_rng(0)
    ws = {}

    def fill(lin, rows, K, bits, seed, experts=None):
        q = QWeight(rows, K, bits, 64, seed=seed, experts=experts)
        lin.weight, lin.scales, lin.biases = q.dw, q.ds, q.db
        ws[id(lin)] = q
        return q

    gq = fill(blk.gate, E, H, 8, 10)
    sg = [fill(blk.switch_mlp.gate_proj, I, H, 2, 11, E), fill(blk.switch_mlp.up_proj, I, H, 2, 12, E),
          fill(blk.switch_mlp.down_proj, H, I, 2, 13, E)]
    sh = [fill(blk.shared_expert.gate_proj, 256, H, 8, 14), fill(blk.shared_expert.up_proj, 256, H, 8, 15),
          fill(blk.shared_expert.down_proj, H, 256, 8, 16)]
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    y = blk(to_tensor(x, "bf16"))
    logits = O.round_bf16(O.quantized_matmul(x, gq.packed, gq.s, gq.b, 8, 64))
    idx, sc = O.route_topk(logits, k)
    sw, _ = O.switch_glu(x, idx, *[(q.packed, q.s, q.b, 2) for q in sg], 64, "bf16")
    routed = O.round_bf16((sw.astype(np.float64) * sc[..., None]).sum(1))
    g = O.round_bf16(O.quantized_matmul(x, sh[0].packed, sh[0].s, sh[0].b, 8, 64))
    u = O.round_bf16(O.quantized_matmul(x, sh[1].packed, sh[1].s, sh[1].b, 8, 64))
    h = O.round_bf16(O.silu(g) * u)
    shared = O.round_bf16(O.quantized_matmul(h, sh[2].packed, sh[2].s, sh[2].b, 8, 64))
    assert_close(values_of(y), O.round_bf16(routed + shared), "moe block")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("T,k,H", [(1, 4, 4096), (32, 10, 4096), (3, 2, 100)])
def test_moe_combine(dt, T, k, H):
    """One-launch combine against the caller composition (oracle), with and without the
    shared expert's output; H = 100 takes the unvectorised kernel."""
    rng = np.random.default_rng(T * 3 + k)
    y = O.round_to(rng.standard_normal((T, k, H), dtype=np.float32), dt)
    w = rng.random((T, k)).astype(np.float32)
    sh = O.round_to(rng.standard_normal((T, H), dtype=np.float32), dt)
    ty, tw, tsh = to_tensor(y, dt), torch.from_numpy(w).cuda(), to_tensor(sh, dt)
    for shared in (None, tsh):
        got = values_of(jq.moe_combine(ty, tw, shared))
        ref = O.moe_combine(y, w, None if shared is None else sh, dt)
        if dt == "f32":
            np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
        else:
            assert_close(got, ref, f"combine {dt} T{T} k{k}")


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 9])
def test_quantized_swiglu(bits, M):
    """Dense SwiGLU pair: one gathered launch at decode sizes (M <= 4; 2-bit M <= 2), the
    matrix-core gate|up launch with the SiLU * up epilogue above."""
    N, K, gs = 200, 512, 64
    g = QWeight(N, K, bits, gs, seed=bits * 3)
    u = QWeight(N, K, bits, gs, seed=bits * 3 + 1)
    rng = np.random.default_rng(M + bits)
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    h = jq.quantized_swiglu(to_tensor(x, "bf16"), (g.dw, g.ds, g.db, bits), (u.dw, u.ds, u.db, bits), gs)
    ref = O.swiglu_pair(x, (g.packed, g.s, g.b, bits), (u.packed, u.s, u.b, bits), gs)
    assert tuple(h.shape) == (M, N)
    assert_close(values_of(h), ref, f"swiglu b{bits} M{M}")


@pytest.mark.parametrize("bits,gs,K,xdt", [(2, 128, 4096, "bf16"), (3, 64, 4096, "bf16"),
                                           (4, 64, 2048, "f16"), (5, 128, 1024, "bf16"),
                                           (6, 64, 4096, "bf16"), (8, 64, 4096, "bf16"),
                                           (8, 128, 1024, "f16"), (4, 128, 512, "bf16")])
@pytest.mark.parametrize("M", [5, 9, 16, 32, 64])
def test_quantized_swiglu_matrix_core_pairs(bits, gs, K, xdt, M):
    """Decode batches of 5..64 rows at 8 bits, or of one activation block (8 rows at gs 64,
    16 at gs 128) at other widths: gate and up row blocks alternate in one matrix-core
    launch whose up item applies silu(round(g)) * round(u). Bit-equal to the grouped dense
    launch followed by the elementwise kernel (the same partial sums in the same order), with
    and without the clamp; N leaves a partial 16-row block and M a partial pass. One case is
    also checked against the oracle on a few rows."""
    N = 1000 + bits
    limit = 0.0 if M % 2 == 0 else 1.0
    print(f"swiglu matrix-core pairs b{bits} g{gs} K{K} {xdt} M{M}", flush=True)
    g = RandQ(N, K, bits, gs, seed=900 + bits + M, sidecar=xdt)
    u = RandQ(N, K, bits, gs, seed=901 + bits + M, sidecar=xdt)
    rng = np.random.default_rng(902 + M)
    x = O.round_to(rng.standard_normal((M, K), dtype=np.float32), xdt)
    tx = to_tensor(x, xdt)
    h = jq.quantized_swiglu(tx, (g.dw, g.ds, g.db, bits), (u.dw, u.ds, u.db, bits), gs,
                            swiglu_limit=limit)
    gy, uy = jq.quantized_matmul_multi(tx, [(g.dw, g.ds, g.db, gs, bits), (u.dw, u.ds, u.db, gs, bits)])
    ref = jq.swiglu(gy, uy, limit)
    assert tuple(h.shape) == (M, N)
    diff = (h.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert torch.equal(h, ref), (f"b{bits} g{gs} K{K} M{M}: fused differs from gate|up + swiglu "
                                 f"in {int((diff > 0).sum())} of {diff.numel()} values, "
                                 f"at most {int(diff.max())} ulp")
    if bits == 3 and M == 9:
        rows = slice(N - 40, N)
        gw = O.dequantize_affine(*g.host(None, rows), bits, gs).astype(np.float64)
        uw = O.dequantize_affine(*u.host(None, rows), bits, gs).astype(np.float64)
        gv = O.round_to(x.astype(np.float64) @ gw.T, xdt).astype(np.float64)
        uv = O.round_to(x.astype(np.float64) @ uw.T, xdt).astype(np.float64)
        if limit > 0:
            gv, uv = np.minimum(gv, limit), np.clip(uv, -limit, limit)
        exact = O.silu(gv) * uv
        assert_close(values_of(h)[:, rows], O.round_to(exact, xdt), f"swiglu pairs b{bits} M{M}",
                     exact=exact, out_dtype=xdt, ulps=1)


@pytest.mark.parametrize("T,k,E", [(1, 4, 128), (1, 10, 512), (2, 8, 64)])
def test_switch_glu_direct_pairs(T, k, E):
    """Decode routing (every pair its own expert tile, no plan kernel) at the configs' expert
    counts, with repeated experts across tokens."""
    H, I, gs = 512, 256, 128
    g = _stack(E, I, H, 2, gs, seed=31)
    u = _stack(E, I, H, 2, gs, seed=32)
    d = _stack(E, H, I, 2, gs, seed=33)
    rng = np.random.default_rng(E + k)
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    inds = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    if T > 1:
        inds[1, 0] = inds[0, 0]
    out = jq.switch_glu(to_tensor(x, "bf16"), torch.from_numpy(inds).cuda(),
                        (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2), (d.dw, d.ds, d.db, 2), gs)
    ref, _ = O.switch_glu(x, inds, (g.packed, g.s, g.b, 2), (u.packed, u.s, u.b, 2),
                          (d.packed, d.s, d.b, 2), gs, "bf16")
    assert_close(values_of(out), ref, f"switch_glu direct T{T} k{k} E{E}")
    # gather_qmm of the same pairs (one row each) also runs without a plan
    y = jq.gather_qmm(to_tensor(x, "bf16")[:, None, None, :], g.dw, g.ds, g.db,
                      rhs_indices=torch.from_numpy(inds).cuda(), group_size=gs, bits=2)
    lhs = np.repeat(np.arange(T), k)
    refg = O.gather_qmm(x[:, None, :], g.packed, g.s, g.b, lhs, inds.reshape(-1), 2, gs)
    assert_close(values_of(y).reshape(T * k, 1, I), O.round_bf16(refg), "gather direct")


@pytest.mark.parametrize("T,k,E,H,I,bits_d,gs,with_shared,xdt", [
    (1, 4, 128, 512, 256, 2, 64, True, "bf16"),    # config-3 shape class: combine inside the down launch
    (1, 10, 512, 512, 256, 2, 128, True, "bf16"),  # config-5 routing: top-10 of 512
    (2, 8, 64, 256, 384, 4, 64, False, "bf16"),
    (3, 2, 16, 384, 128, 3, 64, True, "bf16"),     # 32-lane rows (two rows per wave instruction)
    (1, 4, 4, 4096, 2048, 2, 64, True, "bf16"),    # config-3 sizes (down rows of 2048)
    (1, 6, 32, 256, 256, 8, 32, True, "f16"),      # f16, 8-bit down, group 32
    (2, 4, 16, 256, 512, 6, 64, False, "f16"),     # f16, 6-bit down
    (64, 4, 128, 512, 256, 2, 64, True, "bf16"),   # above decode sizes: the two-call form
])
def test_switch_glu_combine(T, k, E, H, I, bits_d, gs, with_shared, xdt):
    """Routed experts plus combine in one call: bit-identical to switch_glu followed by
    moe_combine on the GPU, and within tolerance of the oracle's composition."""
    g = QWeight(I, H, 2, gs, seed=41, experts=E, sidecar=xdt)
    u = QWeight(I, H, 2, gs, seed=42, experts=E, sidecar=xdt)
    d = QWeight(H, I, bits_d, gs, seed=43, experts=E, sidecar=xdt)
    rng = np.random.default_rng(T * 7 + k)
    x = O.round_to(rng.standard_normal((T, H), dtype=np.float32), xdt)
    inds = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    sh = O.round_to(rng.standard_normal((T, H), dtype=np.float32), xdt)
    tx, ti, tw = to_tensor(x, xdt), torch.from_numpy(inds).cuda(), torch.from_numpy(w).cuda()
    tsh = to_tensor(sh, xdt) if with_shared else None
    gt, ut, dt_ = (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2), (d.dw, d.ds, d.db, bits_d)
    got = jq.switch_glu_combine(tx, ti, tw, gt, ut, dt_, gs, tsh)
    two = jq.moe_combine(jq.switch_glu(tx, ti, gt, ut, dt_, gs), tw, tsh)
    assert tuple(got.shape) == (T, H)
    assert torch.equal(got.view(torch.int16), two.view(torch.int16)), "fused != two calls"
    sw, _ = O.switch_glu(x, inds, (g.packed, g.s, g.b, 2), (u.packed, u.s, u.b, 2),
                         (d.packed, d.s, d.b, bits_d), gs, xdt)
    ref = O.moe_combine(sw, w, sh if with_shared else None, xdt)
    # The value before the last rounding (slot sum rounded, + shared): the max-abs bound then
    # charges only what lies beyond the final rounding.
    pre = (sw.astype(np.float64) * w[..., None]).sum(1)
    if with_shared:
        pre = O.round_to(pre, xdt).astype(np.float64) + sh
    assert_close(values_of(got), ref, f"switch_glu_combine T{T} k{k} E{E} {xdt}", exact=pre,
                 out_dtype=xdt)


@pytest.mark.parametrize("T,k,E,H,I,with_shared,renorm", [
    (1, 4, 128, 512, 256, False, True),   # config-3 class: the gate|up launch routes for itself
    (1, 10, 512, 512, 256, True, True),   # config-5 class (top-10 of 512)
    (3, 2, 64, 384, 128, True, False),    # several tokens, no renormalisation
    (64, 4, 128, 256, 128, True, True),   # above decode sizes: routing launch, plan, tiles
    (1, 4, 640, 256, 128, False, True),   # more experts than the in-launch routing holds
])
def test_moe_experts(T, k, E, H, I, with_shared, renorm):
    """Routing + experts + combine in one call: ids, weights and output bit-identical to
    moe_route followed by switch_glu_combine; ids equal to the oracle's top-k."""
    gs = 64
    g = _stack(E, I, H, 2, gs, seed=51)
    u = _stack(E, I, H, 2, gs, seed=52)
    d = _stack(E, H, I, 2, gs, seed=53)
    rng = np.random.default_rng(T + E + k)
    x = to_tensor(O.round_bf16(rng.standard_normal((T, H), dtype=np.float32)), "bf16")
    logits = rng.standard_normal((T, E)).astype(np.float32)
    tl = torch.from_numpy(logits).cuda()
    sh = to_tensor(O.round_bf16(rng.standard_normal((T, H), dtype=np.float32)), "bf16") \
        if with_shared else None
    gt, ut, dt_ = (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2), (d.dw, d.ds, d.db, 2)
    out, ids, w = jq.moe_experts(x, tl, k, gt, ut, dt_, gs, sh, renorm)
    ids2, w2 = jq.moe_route(tl, k, renorm)
    out2 = jq.switch_glu_combine(x, ids2, w2, gt, ut, dt_, gs, sh)
    assert torch.equal(ids, ids2) and torch.equal(w, w2)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    np.testing.assert_array_equal(ids.cpu().numpy(), O.route_topk(logits, k, renorm)[0])


@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrtsoftplus"])
@pytest.mark.parametrize("T,E,k,groups,with_bias,ldt", [
    (3, 64, 4, (1, 1), False, "f32"),
    (2, 512, 10, (1, 1), True, "bf16"),   # config-5 width, bf16 router output read directly
    (4, 256, 8, (8, 4), True, "f32"),     # group-limited, DeepSeek-like
    (5, 640, 6, (4, 1), False, "f16"),    # more experts than the in-launch routing holds
])
def test_route_variants(score, T, E, k, groups, with_bias, ldt):
    """Every router form against the oracle: ids equal, weights within fp32 rounding."""
    rng = np.random.default_rng(E + k + T)
    logits = O.round_to(rng.standard_normal((T, E)).astype(np.float32) * 2, ldt)
    bias = rng.standard_normal(E).astype(np.float32) * 0.2 if with_bias else None
    ng, tg = groups
    tb = torch.from_numpy(bias).cuda() if with_bias else None
    idx, w = jq.moe_route(to_tensor(logits, ldt), k, True, score=score, score_bias=tb,
                          n_group=ng, topk_group=tg, scaling=1.5)
    ridx, rw = O.route_topk_ex(logits, k, score=score, bias=bias, n_group=ng, topk_group=tg,
                               renorm=True, scaling=1.5)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    _, w0 = jq.moe_route(to_tensor(logits, ldt), k, False, score=score, score_bias=tb,
                         n_group=ng, topk_group=tg)
    np.testing.assert_allclose(w0.cpu().numpy(), O.route_topk_ex(
        logits, k, score=score, bias=bias, n_group=ng, topk_group=tg, renorm=False)[1],
        rtol=1e-5, atol=1e-7)


def _moe_case(E, H, I, bits, gs, sI, seed):
    g = QWeight(I, H, bits, gs, seed=seed, experts=E)
    u = QWeight(I, H, bits, gs, seed=seed + 1, experts=E)
    d = QWeight(H, I, bits, gs, seed=seed + 2, experts=E)
    sh = None
    if sI:
        sh = [QWeight(sI, H, 8, 64, seed=seed + 3), QWeight(sI, H, 8, 64, seed=seed + 4),
              QWeight(H, sI, 8, 64, seed=seed + 5)]
    return g, u, d, sh


@pytest.mark.parametrize("T", [1, 5, 64])
@pytest.mark.parametrize("combine,limit,gated,score", [
    ("after", 0.0, False, "softmax"),
    ("after", 0.5, True, "softmax"),
    ("before", 0.0, False, "sqrtsoftplus"),
    ("before", 0.5, False, "sigmoid"),
])
def test_moe_block(T, combine, limit, gated, score):
    """jq_moe_block against the oracle's MoE token (both combine forms, the SwiGLU clamp, the
    sigmoid-gated shared term, sigmoid / sqrt-softplus routers with a selection bias and a
    scaling factor): T = 1 takes the two fused decode launches, T = 5 the routing launch and
    one-row tiles, T = 64 the plan and matrix-core tiles."""
    E, H, I, k, gs, sI = 32, 512, 256, 4, 64, 256
    g, u, d, sh = _moe_case(E, H, I, 2, gs, sI, seed=70)
    rng = np.random.default_rng(T * 11 + len(combine))
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    logits = O.round_bf16(rng.standard_normal((T, E)).astype(np.float32))
    bias = None if score == "softmax" else rng.standard_normal(E).astype(np.float32) * 0.1
    rsf = 1.0 if score == "softmax" else 2.0
    gl = O.round_bf16(rng.standard_normal(T).astype(np.float32)) if gated else None
    tsh = tuple((q.dw, q.ds, q.db, 64, 8) for q in sh)
    out, ids, w = jq.moe_block(
        to_tensor(x, "bf16"), to_tensor(logits, "bf16"), k, (g.dw, g.ds, g.db, 2),
        (u.dw, u.ds, u.db, 2), (d.dw, d.ds, d.db, 2), gs, shared=tsh,
        shared_gate=None if gl is None else to_tensor(gl, "bf16")[:, None], score=score,
        score_bias=None if bias is None else torch.from_numpy(bias).cuda(), scaling=rsf,
        combine=combine, swiglu_limit=limit)
    ridx, rw = O.route_topk_ex(logits, k, score=score, bias=bias, scaling=rsf)
    np.testing.assert_array_equal(ids.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    cache = {}

    def deq(c, e):
        key = (c, int(e))
        if key not in cache:
            q = {"g": g, "u": u, "d": d}[c]
            cache[key] = O.dequantize_affine(q.packed[e], q.s[e], q.b[e], 2, gs).astype(np.float64)
        return cache[key]

    Ws = [q.dequant().astype(np.float64) for q in sh]
    yv = values_of(out)
    for t in sorted({0, T // 2, T - 1}):
        s_out = O.shared_expert(x[t], *Ws, limit=limit)
        ref, pre = O.moe_token(x[t], ridx[t], rw[t], deq, combine, limit, s_out,
                               None if gl is None else gl[t])
        assert_close(yv[t], ref, f"moe_block T{T} t{t} {combine} L{limit}", exact=pre,
                     out_dtype="bf16", ulps=1)


@pytest.mark.parametrize("T", [1, 3])
def test_moe_block_equals_experts_call(T):
    """The default block (softmax, after-down combine, no clamp) is bit-identical to the shared
    expert's two calls followed by jq_moe_experts with its output."""
    E, H, I, k, gs, sI = 64, 512, 256, 6, 128, 512
    g, u, d, sh = _moe_case(E, H, I, 2, gs, sI, seed=80)
    rng = np.random.default_rng(T)
    x = to_tensor(O.round_bf16(rng.standard_normal((T, H), dtype=np.float32)), "bf16")
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    tsh = tuple((q.dw, q.ds, q.db, 64, 8) for q in sh)
    out, ids, w = jq.moe_block(x, logits, k, (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2),
                               (d.dw, d.ds, d.db, 2), gs, shared=tsh)
    hs = jq.quantized_swiglu(x, (sh[0].dw, sh[0].ds, sh[0].db, 8), (sh[1].dw, sh[1].ds, sh[1].db, 8), 64)
    s_out = jq.quantized_matmul(hs, sh[2].dw, sh[2].ds, sh[2].db, True, 64, 8)
    out2, ids2, w2 = jq.moe_experts(x, logits, k, (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2),
                                    (d.dw, d.ds, d.db, 2), gs, s_out)
    assert torch.equal(ids, ids2) and torch.equal(w, w2)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def test_moe_block_argument_errors():
    E, H, I, gs = 8, 256, 128, 64
    g, u, d, sh = _moe_case(E, H, I, 2, gs, 128, seed=90)
    x = torch.zeros((1, H), dtype=torch.bfloat16, device="cuda")
    lg = torch.zeros((1, E), device="cuda")
    gt, ut, dt_ = (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2), (d.dw, d.ds, d.db, 2)
    tsh = tuple((q.dw, q.ds, q.db, 64, 8) for q in sh)
    with pytest.raises(ValueError):  # gated shared term without a shared expert
        jq.moe_block(x, lg, 2, gt, ut, dt_, gs, shared_gate=x[:, :1])
    with pytest.raises(ValueError):  # gated shared term in the before-down form
        jq.moe_block(x, lg, 2, gt, ut, dt_, gs, shared=tsh, shared_gate=x[:, :1], combine="before")
    with pytest.raises(ValueError):  # groups that do not divide E
        jq.moe_block(x, lg, 2, gt, ut, dt_, gs, n_group=3, topk_group=1)
    with pytest.raises(ValueError):
        jq.moe_block(x, lg, 2, gt, ut, dt_, gs, score="relu")
    with pytest.raises(ValueError):
        jq.moe_block(x, lg[:, :4], 2, gt, ut, dt_, gs)


@pytest.mark.parametrize("T", [1, 6])
def test_moe_block_module_shared_gate(T):
    """SparseMoeBlock with the qwen-style shared_expert_gate (a 1-row 8-bit linear whose
    sigmoid scales the shared expert's output, qwen4_exp/modeling.py:599), bf16 router logits
    read directly."""
    H, I, E, k, sI = 256, 128, 16, 4, 256
    blk = jnn.SparseMoeBlock(H, I, E, k, shared_hidden=sI, bits=2, shared_expert_gate=True,
                             device="cuda")
    qs = {}

    def fill(name, lin, rows, K, bits, seed, experts=None):
        q = QWeight(rows, K, bits, 64, seed=seed, experts=experts)
        lin.weight, lin.scales, lin.biases = q.dw, q.ds, q.db
        qs[name] = q

    fill("r", blk.gate, E, H, 8, 20)
    fill("sg_lin", blk.shared_expert_gate, 1, H, 8, 21)
    for n, lin, rows, K, seed in (("g", blk.switch_mlp.gate_proj, I, H, 22),
                                  ("u", blk.switch_mlp.up_proj, I, H, 23),
                                  ("d", blk.switch_mlp.down_proj, H, I, 24)):
        fill(n, lin, rows, K, 2, seed, E)
    for n, lin, rows, K, seed in (("sg", blk.shared_expert.gate_proj, sI, H, 25),
                                  ("su", blk.shared_expert.up_proj, sI, H, 26),
                                  ("sd", blk.shared_expert.down_proj, H, sI, 27)):
        fill(n, lin, rows, K, 8, seed)
    rng = np.random.default_rng(T)
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    y = values_of(blk(to_tensor(x, "bf16")))
    deqd = {n: q.dequant().astype(np.float64) for n, q in qs.items() if n in ("r", "sg_lin", "sg", "su", "sd")}
    logits = O.round_bf16(x.astype(np.float64) @ deqd["r"].T)
    gl = O.round_bf16(x.astype(np.float64) @ deqd["sg_lin"].T)[:, 0]
    ids, w = O.route_topk(logits, k)

    def deq(c, e):
        q = qs[c]
        return O.dequantize_affine(q.packed[e], q.s[e], q.b[e], 2, 64).astype(np.float64)

    for t in range(T):
        s_out = O.shared_expert(x[t], deqd["sg"], deqd["su"], deqd["sd"])
        ref, pre = O.moe_token(x[t], ids[t], w[t], deq, "after", 0.0, s_out, gl[t])
        assert_close(y[t], ref, f"gated block t{t}", exact=pre, out_dtype="bf16", ulps=1)


@pytest.mark.parametrize("combine,limit,gated", [("after", 0.0, False), ("after", 0.4, True),
                                                 ("before", 0.4, False)])
@pytest.mark.parametrize("H,I,sI,bits,sbits,gs,E,k", [
    (4096, 1024, 4096, 2, 8, 128, 64, 10),   # config-5 shapes: 2-bit g128 experts, 8-bit shared
    (2048, 512, 2048, 3, 4, 64, 16, 4),      # 3-bit experts, 4-bit shared, one-wave rows
])
def test_moe_block_fused_decode(combine, limit, gated, H, I, sI, bits, sbits, gs, E, k):
    """One token with a shared expert: the routed experts' gate|up (routing in the launch) and
    the shared expert's gate|up share one launch. Checked against the oracle, and bit for bit
    against the shared expert's own launches followed by jq_moe_experts (the same row and
    gather bodies, the same reduction orders)."""
    g = RandQ(I, H, bits, gs, seed=E + 1, experts=E)
    u = RandQ(I, H, bits, gs, seed=E + 2, experts=E)
    d = RandQ(H, I, bits, gs, seed=E + 3, experts=E)
    sh = [RandQ(sI, H, sbits, 64, seed=E + 4), RandQ(sI, H, sbits, 64, seed=E + 5),
          RandQ(H, sI, sbits, 64, seed=E + 6)]
    rng = np.random.default_rng(H + k)
    x = O.round_bf16(rng.standard_normal((1, H), dtype=np.float32))
    logits = rng.standard_normal((1, E)).astype(np.float32)
    gl = O.round_bf16(rng.standard_normal(1).astype(np.float32)) if gated else None
    tx, tl = to_tensor(x, "bf16"), torch.from_numpy(logits).cuda()
    tsh = tuple((q.dw, q.ds, q.db, 64, sbits) for q in sh)
    out, ids, w = jq.moe_block(tx, tl, k, g.tup(), u.tup(), d.tup(), gs, shared=tsh,
                               shared_gate=None if gl is None else to_tensor(gl, "bf16")[:, None],
                               combine=combine, swiglu_limit=limit)
    ridx, rw = O.route_topk(logits, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ridx)
    if combine == "after" and not gated and limit == 0.0:
        hs = jq.quantized_swiglu(tx, (sh[0].dw, sh[0].ds, sh[0].db, sbits),
                                 (sh[1].dw, sh[1].ds, sh[1].db, sbits), 64)
        s_gpu = jq.quantized_matmul(hs, sh[2].dw, sh[2].ds, sh[2].db, True, 64, sbits)
        out2, ids2, w2 = jq.moe_experts(tx, tl, k, g.tup(), u.tup(), d.tup(), gs, s_gpu)
        assert torch.equal(ids, ids2) and torch.equal(w, w2)
        assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "fused != two-step"
    cache = {}

    def deq(c, e):
        if (c, int(e)) not in cache:
            ww, s_, b_ = {"g": g, "u": u, "d": d}[c].host(e)
            cache[(c, int(e))] = O.dequantize_affine(ww, s_, b_, bits, gs).astype(np.float64)
        return cache[(c, int(e))]

    Ws = [O.dequantize_affine(*q.host(), sbits, 64).astype(np.float64) for q in sh]
    s_out = O.shared_expert(x[0], *Ws, limit=limit)
    ref, pre = O.moe_token(x[0], ridx[0], rw[0], deq, combine, limit, s_out,
                           None if gl is None else gl[0])
    assert_close(values_of(out)[0], ref, f"fused decode {combine} L{limit}", exact=pre,
                 out_dtype="bf16", ulps=1)
    # a second call gives the same bits
    out3, _, _ = jq.moe_block(tx, tl, k, g.tup(), u.tup(), d.tup(), gs, shared=tsh,
                              shared_gate=None if gl is None else to_tensor(gl, "bf16")[:, None],
                              combine=combine, swiglu_limit=limit)
    assert torch.equal(out3.view(torch.int16), out.view(torch.int16))
