"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline: one decode step of the JANG-profile mixed-precision
transformer block at batch 1 — q/k/v/o 6-bit, MLP gate/up 3-bit, down 2-bit, group 64,
hidden 4096, 32/8 heads x 128, intermediate 14336 — reported as achieved HBM GB/s of the
packed weights' algorithmic bytes. One step streams every projection once:
  launch 1  q|k|v   (one grouped launch, same x)      launch 3  gate|up (one grouped launch)
  launch 2  o                                          launch 4  down
Attention and the SwiGLU elementwise are outside the path: o and down read seeded
synthetic activations of their true shapes. Weights are rotated over enough copies that
every step touches > 256 MB (the MI355X last-level cache holds one block).

Also reported (the "extra" object): configs 1 (single 4096x4096 4-bit GEMV), 2 at batch
8 and 32, 3 (128-expert MoE decode layer, tokens/s), 4 (prefill GEMM TFLOP/s, 4- and
3-bit) and 5 (512-expert MoE layer with shared expert, tokens/s).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true")
    p.add_argument("--only", default="", help="comma list of extra workloads to run")
    p.add_argument("--profile", choices=("gateup", "gateup8", "gateup32", "copy", "down", "c1",
                                         "c3", "c5"),
                   default=None,
                   help="run one workload eagerly for rocprofv3 counter passes and print one "
                        "JSON line: the gate|up launch (gateup; at batch 8 / 32: gateup8, "
                        "gateup32), a plain 256 MiB copy (copy), "
                        "the 2-bit down projection (down), config 1 (c1), or the MoE layer of "
                        "config 3 / 5 at T = 1 (c3, c5)")
    return p.parse_args()


# ----------------------------------------------------------------------------- helpers


class QW:
    """A quantized weight on the GPU: codes int32 [.., N, K*bits/32], bf16 scales/biases."""

    def __init__(self, w, bits, gs):
        import jangq_amd as jq

        self.bits, self.gs = bits, gs
        self.N, self.K = w.shape[-2], w.shape[-1]
        import torch

        self.w, self.s, self.b = jq.quantize(w, gs, bits)
        self.w = self.w.view(torch.int32)

    def clone(self):
        import copy

        c = copy.copy(self)
        c.w, c.s, c.b = self.w.clone(), self.s.clone(), self.b.clone()
        return c

    def nbytes(self, rows=None):
        """Algorithmic bytes: codes + bf16 scale + bias (of `rows` rows, default all)."""
        rows = self.N if rows is None else rows
        return rows * self.K * self.bits // 8 + rows * (self.K // self.gs) * 4

    def tup(self):
        return (self.w, self.s, self.b, self.gs, self.bits)


def randn(shape, std, gen, dtype=None):
    import torch

    return (torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32) * std).to(
        dtype or torch.bfloat16)


def timed(fn, steps, warmup):
    """Mean ms per step of fn(0), ..., fn(steps - 1).

    The W warmup calls run eagerly; the K timed calls are captured into one HIP graph and
    replayed once, bracketed by HIP events on torch's current stream (the stream every
    jangq_amd launch and the replay use), so host launch overhead is not measured."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    del g
    return ms


def copies_for(nbytes):
    """Rotated copies so one pass over them exceeds twice the last-level cache."""
    return max(2, int((2 * MALL_BYTES) // max(nbytes, 1)) + 1)


# ----------------------------------------------------------------------------- config 2


def c2_block(gen, M):
    import torch

    H, NQ, NKV, HD, I = 4096, 32, 8, 128, 14336
    q = QW(randn((NQ * HD, H), 0.02, gen), 6, 64)
    k = QW(randn((NKV * HD, H), 0.02, gen), 6, 64)
    v = QW(randn((NKV * HD, H), 0.02, gen), 6, 64)
    o = QW(randn((H, NQ * HD), 0.02, gen), 6, 64)
    g = QW(randn((I, H), 0.02, gen), 3, 64)
    u = QW(randn((I, H), 0.02, gen), 3, 64)
    d = QW(randn((H, I), 0.02, gen), 2, 64)
    layer = dict(q=q, k=k, v=v, o=o, g=g, u=u, d=d)
    x = randn((M, H), 1.0, gen)
    xo = randn((M, NQ * HD), 1.0, gen)
    xd = randn((M, I), 1.0, gen)
    wbytes = sum(w.nbytes() for w in layer.values())
    act = 2 * M * (H + H + H + NQ * HD + H + H + I)  # x reads per launch (q|k|v, g|u share)
    out = 2 * M * (NQ * HD + 2 * NKV * HD + H + 2 * I + H)
    return layer, (x, xo, xd), wbytes + act + out, wbytes


def block_step(layer, acts, outs=None):
    import jangq_amd as jq

    x, xo, xd = acts
    qkv = jq.quantized_matmul_multi(x, [layer["q"].tup(), layer["k"].tup(), layer["v"].tup()])
    ob = layer["o"]
    y_o = jq.quantized_matmul(xo, ob.w, ob.s, ob.b, True, ob.gs, ob.bits)
    gu = jq.quantized_matmul_multi(x, [layer["g"].tup(), layer["u"].tup()])
    db = layer["d"]
    y_d = jq.quantized_matmul(xd, db.w, db.s, db.b, True, db.gs, db.bits)
    return qkv, y_o, gu, y_d


def bench_c2(gen, M, steps, warmup):
    layer, acts, step_bytes, wbytes = c2_block(gen, M)
    R = copies_for(wbytes)
    layers = [layer] + [{k: w.clone() for k, w in layer.items()} for _ in range(R - 1)]
    ms = timed(lambda i: block_step(layers[i % R], acts), steps, warmup)
    # dominant kernel: the grouped gate|up launch
    import jangq_amd as jq

    x = acts[0]
    gu_bytes = layer["g"].nbytes() + layer["u"].nbytes() + 2 * x.numel() + 2 * 2 * x.shape[0] * 14336
    ms_gu = timed(lambda i: jq.quantized_matmul_multi(x, [layers[i % R]["g"].tup(),
                                                          layers[i % R]["u"].tup()]), steps, warmup)
    return dict(ms=ms, bytes=step_bytes, gbs=step_bytes / ms / 1e6, copies=R,
                gu_ms=ms_gu, gu_bytes=gu_bytes, gu_gbs=gu_bytes / ms_gu / 1e6), layer, acts


# ----------------------------------------------------------------------------- config 1


def bench_c1(gen, steps, warmup):
    import jangq_amd as jq

    w = QW(randn((4096, 4096), 0.02, gen), 4, 64)
    x = randn((1, 4096), 1.0, gen)
    nb = w.nbytes() + 2 * 4096 + 2 * 4096
    R = copies_for(w.nbytes())
    ws = [w] + [w.clone() for _ in range(R - 1)]
    ms = timed(lambda i: jq.quantized_matmul(x, ws[i % R].w, ws[i % R].s, ws[i % R].b, True, 64, 4),
               steps, warmup)
    return dict(ms=ms, bytes=nb, gbs=nb / ms / 1e6, frac=nb / ms / 1e6 / HBM_PEAK_GBS, copies=R)


# ----------------------------------------------------------------------------- config 4


def bench_c4(gen, bits, steps, warmup):
    import jangq_amd as jq

    M, K, N = 2048, 4096, 14336
    w = QW(randn((N, K), 0.02, gen), bits, 64)
    x = randn((M, K), 1.0, gen)
    import torch

    y = torch.empty((M, N), dtype=x.dtype, device="cuda")
    ms = timed(lambda i: jq.quantized_matmul(x, w.w, w.s, w.b, True, 64, bits, out=y), steps, warmup)
    flops = 2.0 * M * N * K
    return dict(ms=ms, tflops=flops / ms / 1e9, frac=flops / ms / 1e9 / BF16_PEAK_TFLOPS)


# ----------------------------------------------------------------------------- MoE configs


def moe_layer(gen, E, H, I, bits, gs, k, shared_I=None):
    import torch

    from jangq_amd import nn as jnn

    blk = jnn.SparseMoeBlock(H, I, E, k, shared_hidden=shared_I, group_size=gs, bits=bits,
                             device="cuda")
    router = QW(randn((E, H), 0.02, gen), 8, 64)
    blk.gate.weight, blk.gate.scales, blk.gate.biases = router.w, router.s, router.b
    for proj, (rows, cols) in ((blk.switch_mlp.gate_proj, (I, H)), (blk.switch_mlp.up_proj, (I, H)),
                               (blk.switch_mlp.down_proj, (H, I))):
        q = QW(randn((E, rows, cols), 0.02, gen), bits, gs)
        proj.weight, proj.scales, proj.biases = q.w, q.s, q.b
    if shared_I:
        for lin, (rows, cols) in ((blk.shared_expert.gate_proj, (shared_I, H)),
                                  (blk.shared_expert.up_proj, (shared_I, H)),
                                  (blk.shared_expert.down_proj, (H, shared_I))):
            q = QW(randn((rows, cols), 0.02, gen), 8, 64)
            lin.weight, lin.scales, lin.biases = q.w, q.s, q.b
    return blk, router


def _clone_dense(blk):
    """A copy of the block whose router and shared expert are new tensors (the expert stacks
    are shared: the rotated routings already spread them over more than the cache holds)."""
    import copy

    c = copy.copy(blk)
    c._modules = dict(blk._modules)
    for name in ("gate", "shared_expert"):
        m = blk._modules.get(name)
        if m is not None:
            mc = copy.deepcopy(m)
            c._modules[name] = mc
    return c


def bench_moe(gen, name, E, H, I, bits, gs, k, T, steps, warmup, shared_I=None, skew=False):
    import torch

    import jangq_amd as jq

    blk, router = moe_layer(gen, E, H, I, bits, gs, k, shared_I)
    R = 16  # distinct routings so the selected experts change every step
    xs = [randn((T, H), 1.0, gen) for _ in range(R)]
    logit_sets = []
    for r in range(R):
        lg = torch.randn((T, E), generator=gen, device="cuda", dtype=torch.float32)
        if skew:
            perm = torch.randperm(E, generator=gen, device="cuda")[: round(0.1 * E)]
            lg[:, perm] += 2.0
        logit_sets.append(lg)
    # Rotated copies of the router and the shared expert: every step reads a copy the previous
    # steps evicted (their bytes over the copies exceed twice the last-level cache).
    dense = router.nbytes() + (3 * (shared_I * H + shared_I * (H // 64) * 4) if shared_I else 0)
    C = copies_for(dense)
    blocks = [blk] + [_clone_dense(blk) for _ in range(C - 1)]

    def step(i):
        # The router GEMV runs (its bytes are counted below); routing uses the config's
        # synthetic N(0,1) logits so that the expert load is the one the config states.
        b = blocks[i % C]
        b.gate(xs[i % R])
        return b(xs[i % R], logits=logit_sets[i % R])

    ms = timed(step, steps, warmup)
    # Algorithmic bytes of one layer: router + distinct selected experts (+ shared).
    per_expert = 3 * (I * H * bits // 8 + I * (H // gs) * 4)  # gate + up + down
    distinct = []
    for lg in logit_sets:
        idx, _ = jq.moe_route(lg, k)
        distinct.append(len(torch.unique(idx)))
    mean_distinct = sum(distinct) / len(distinct)
    nb = dense + mean_distinct * per_expert
    return dict(ms=ms, tokens_per_s=T / ms * 1e3, distinct_experts=mean_distinct,
                bytes=nb, gbs=nb / ms / 1e6, frac=nb / ms / 1e6 / HBM_PEAK_GBS,
                dense_copies=C)


def bench_attn8(gen, T, steps, warmup):
    """Config 5's attention projections at 8-bit g64 (geometry of config 2: q/o 4096 x 4096,
    k/v 1024 x 4096): q|k|v grouped, then o, rotated copies."""
    import jangq_amd as jq

    H = 4096
    q, kk, v, o = (QW(randn((n, H), 0.02, gen), 8, 64) for n in (4096, 1024, 1024, 4096))
    x = randn((T, H), 1.0, gen)
    wb = sum(w.nbytes() for w in (q, kk, v, o))
    R = copies_for(wb)
    sets = [(q, kk, v, o)] + [tuple(w.clone() for w in (q, kk, v, o)) for _ in range(R - 1)]

    def step(i):
        a, b, c, d = sets[i % R]
        jq.quantized_matmul_multi(x, [a.tup(), b.tup(), c.tup()])
        return jq.quantized_matmul(x, d.w, d.s, d.b, True, 64, 8)

    ms = timed(step, steps, warmup)
    nb = wb + 2 * T * H * 2 + 2 * T * (4096 + 2048 + 4096)
    return dict(ms=ms, bytes=nb, gbs=nb / ms / 1e6, frac=nb / ms / 1e6 / HBM_PEAK_GBS, copies=R)


# ----------------------------------------------------------------------------- CPU baseline


def cpu_baseline_c2(min_seconds=10.0, max_seconds=30.0):
    """The reference CPU path restated (oracle/): numpy dequant (affine.py:445-463) then
    BLAS fp32 x @ W^T, for the config-2 block at batch 1, on this host's cores. The block's
    seven projections are quantized once and then run in passes until at least min_seconds of
    timed CPU work (bounded by max_seconds)."""
    import numpy as np

    cores = len(os.sched_getaffinity(0))
    from oracle import jangq_oracle as O

    rng = np.random.default_rng(200)
    H, I = 4096, 14336
    shapes = [((4096, H), 6), ((1024, H), 6), ((1024, H), 6), ((H, 4096), 6), ((I, H), 3),
              ((I, H), 3), ((H, I), 2)]
    mats = []
    for (N, K), bits in shapes:
        w = O.round_bf16(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        packed, s, b, _ = O.quantize_affine(w, bits, 64)
        x = O.round_bf16(rng.standard_normal((1, K), dtype=np.float32))
        mats.append((packed, O.sidecar_f32(s, "bf16"), O.sidecar_f32(b, "bf16"), bits, x, N, K))
    t_deq = t_mm = 0.0
    nbytes = 0
    done = 0
    while t_deq + t_mm < min_seconds:
        for packed, sf, bf, bits, x, N, K in mats:
            t0 = time.perf_counter()
            W = O.dequantize_affine(packed, sf, bf, bits, 64)
            t1 = time.perf_counter()
            y = x @ W.T
            t2 = time.perf_counter()
            t_deq += t1 - t0
            t_mm += t2 - t1
            nbytes += N * K * bits // 8 + N * (K // 64) * 4 + 2 * K + 2 * N
            done += 1
            if t_deq + t_mm > max_seconds:
                break
        if t_deq + t_mm > max_seconds:
            break
    secs = t_deq + t_mm
    return {"value": round(nbytes / secs / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{done} projections ({done / 7:.1f} passes over the config-2 block at batch "
                      f"1): numpy dequant ({t_deq:.2f} s) + BLAS fp32 matmul ({t_mm:.2f} s), "
                      f"vectorised unpack",
            "dequant_s": round(t_deq, 3), "matmul_s": round(t_mm, 3)}


def _rand_qweight(rng, rows, K, bits, gs):
    """Random packed codes with bf16-valued scales / biases (any codes are a valid weight)."""
    import numpy as np

    from oracle import jangq_oracle as O

    words = rng.integers(0, 1 << 32, size=(rows, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    qmax = (1 << bits) - 1
    s = O.round_bf16((rng.random((rows, K // gs), dtype=np.float32) * 0.5 + 0.75) * (0.07 / qmax))
    b = O.round_bf16(-s * (qmax / 2))
    return words, s, b


def cpu_baseline_moe(min_seconds=8.0, max_seconds=20.0):
    """Config-3 MoE decode on the host, the reference's per-active-expert loop
    (dots3/ops_selftest.py:18-28): per token, softmax top-4 of 128 logits, then for each
    selected expert numpy dequant (affine.py:445-463) of gate/up/down and fp32 BLAS matvecs,
    silu(g) * u, the weighted sum. Tokens until min_seconds of work."""
    import numpy as np

    from oracle import jangq_oracle as O

    rng = np.random.default_rng(301)
    E, H, I, k, gs = 128, 4096, 2048, 4, 64
    pool = 16  # distinct expert weights generated (a token's experts are drawn from them)
    experts = [[_rand_qweight(rng, r, c, 2, gs) for r, c in ((I, H), (I, H), (H, I))]
               for _ in range(pool)]
    t_deq = t_mm = 0.0
    tokens = 0
    while t_deq + t_mm < min_seconds and t_deq + t_mm < max_seconds:
        x = O.round_bf16(rng.standard_normal(H, dtype=np.float32))
        logits = rng.standard_normal((1, E)).astype(np.float32)
        idx, w = O.route_topk(logits, k)
        out = np.zeros(H, np.float32)
        for j, e in enumerate(idx[0]):
            mats = experts[int(e) % pool]
            t0 = time.perf_counter()
            Wg, Wu, Wd = (O.dequantize_affine(p, sc, bi, 2, gs) for p, sc, bi in mats)
            t1 = time.perf_counter()
            g, u = x @ Wg.T, x @ Wu.T
            out += np.float32(w[0, j]) * ((g / (1 + np.exp(-g)) * u) @ Wd.T)
            t2 = time.perf_counter()
            t_deq += t1 - t0
            t_mm += t2 - t1
        tokens += 1
    secs = t_deq + t_mm
    return {"value": round(tokens / secs, 3), "unit": "tokens/s",
            "sample": f"{tokens} config-3 tokens at T = 1 (4 experts each, 2-bit g64, H 4096, "
                      f"I 2048): numpy dequant {t_deq:.2f} s + BLAS matvecs {t_mm:.2f} s",
            "dequant_s": round(t_deq, 3), "matmul_s": round(t_mm, 3)}


def cpu_baseline_prefill(bits=4, min_seconds=5.0):
    """Config-4 prefill on the host: numpy dequant of the 14336 x 4096 weight then fp32 BLAS
    x @ W^T with x [2048, 4096]; passes until min_seconds."""
    import numpy as np

    from oracle import jangq_oracle as O

    rng = np.random.default_rng(401)
    M, K, N, gs = 2048, 4096, 14336, 64
    p, sc, bi = _rand_qweight(rng, N, K, bits, gs)
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    t_deq = t_mm = 0.0
    passes = 0
    while t_deq + t_mm < min_seconds:
        t0 = time.perf_counter()
        W = O.dequantize_affine(p, sc, bi, bits, gs)
        t1 = time.perf_counter()
        _ = x @ W.T
        t2 = time.perf_counter()
        t_deq += t1 - t0
        t_mm += t2 - t1
        passes += 1
    flops = 2.0 * M * N * K * passes
    return {"value": round(flops / (t_deq + t_mm) / 1e12, 4), "unit": "TFLOP/s",
            "sample": f"{passes} passes of config 4 ({bits}-bit): numpy dequant {t_deq:.2f} s + "
                      f"BLAS fp32 GEMM {t_mm:.2f} s",
            "dequant_s": round(t_deq, 3), "matmul_s": round(t_mm, 3)}


# ----------------------------------------------------------------------------- counters

TRAFFIC_FILE = ROOT / "profiles" / "gateup_c2_m1_traffic.txt"


def traffic_from_profile():
    """HBM bytes per gate|up launch from the committed counter summary (FETCH_SIZE and
    WRITE_SIZE passes, each scaled by the copy-kernel calibration), or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def profile_run(kind, steps):
    """Eager launches of one kernel for a counter pass (no graph: counters are per dispatch)."""
    import torch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(200)
    if kind == "copy":
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(generator=gen)
        dst = torch.empty_like(src)
        for _ in range(steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        return {"profile": "copy", "bytes_read": n, "bytes_written": n, "launches": steps}
    import jangq_amd as jq

    if kind in ("c3", "c5"):
        E, I, gs, k, sI = (128, 2048, 64, 4, None) if kind == "c3" else (512, 1024, 128, 10, 4096)
        blk, _ = moe_layer(gen, E, 4096, I, 2, gs, k, sI)
        xs = [randn((1, 4096), 1.0, gen) for _ in range(16)]
        lgs = []
        for _ in range(16):
            lg = torch.randn((1, E), generator=gen, device="cuda")
            if kind == "c5":
                lg[:, torch.randperm(E, generator=gen, device="cuda")[: round(0.1 * E)]] += 2.0
            lgs.append(lg)
        for i in range(steps):
            blk.gate(xs[i % 16])
            blk(xs[i % 16], logits=lgs[i % 16])
        torch.cuda.synchronize()
        return {"profile": kind, "launches": steps}
    if kind in ("down", "c1"):
        N, K, bits = (4096, 14336, 2) if kind == "down" else (4096, 4096, 4)
        w = QW(randn((N, K), 0.02, gen), bits, 64)
        R = copies_for(w.nbytes())
        ws = [w] + [w.clone() for _ in range(R - 1)]
        x = randn((1, K), 1.0, gen)
        for i in range(steps):
            q = ws[i % R]
            jq.quantized_matmul(x, q.w, q.s, q.b, True, 64, bits)
        torch.cuda.synchronize()
        return {"profile": kind, "algorithmic_bytes": w.nbytes() + 2 * K + 2 * N,
                "launches": steps, "copies": R}

    # gate|up of the config-2 block at batch 1 (gateup), 8 or 32 (gateup8 / gateup32)
    M = {"gateup": 1, "gateup8": 8, "gateup32": 32}[kind]
    layer, acts, _, _ = c2_block(gen, M)
    R = copies_for(layer["g"].nbytes() + layer["u"].nbytes())
    gs = [(layer["g"], layer["u"])] + [(layer["g"].clone(), layer["u"].clone())
                                      for _ in range(R - 1)]
    for i in range(steps):
        g, u = gs[i % R]
        jq.quantized_matmul_multi(acts[0], [g.tup(), u.tup()])
    torch.cuda.synchronize()
    x = acts[0]
    nb = layer["g"].nbytes() + layer["u"].nbytes() + 2 * x.numel() + 2 * 2 * M * 14336
    return {"profile": kind, "algorithmic_bytes": nb, "launches": steps, "copies": R}


# ----------------------------------------------------------------------------- main


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a run)"}))
        sys.exit(2)
    ncores = str(len(os.sched_getaffinity(0)))
    for var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
        os.environ.setdefault(var, ncores)
    import torch

    from jangq_amd import _lib

    if not _lib.LIB_PATH.exists():
        from jangq_amd import build as jb

        jb.build()
    torch.cuda.set_device(0)
    if args.profile:
        print(json.dumps(profile_run(args.profile, args.steps)))
        return
    gen = torch.Generator(device="cuda")
    gen.manual_seed(200)

    res, layer, acts = bench_c2(gen, 1, args.steps, args.warmup)
    extra = {}
    wanted = set(filter(None, args.only.split(",")))

    def want(name):
        return not args.no_extra and (not wanted or name in wanted)

    s2, w2 = max(20, args.steps // 4), max(5, args.warmup // 4)
    if want("c2"):
        for M in (8, 32):
            r, _, _ = bench_c2(gen, M, s2, w2)
            extra[f"c2_block_M{M}"] = {"gbs": round(r["gbs"], 1), "ms": round(r["ms"], 4),
                                       "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
    if want("c1"):
        r = bench_c1(gen, args.steps, args.warmup)
        extra["c1_gemv_4096x4096_4bit"] = {k: round(v, 5) if isinstance(v, float) else v
                                           for k, v in r.items()}
    if want("c4"):
        for bits in (4, 3):
            r = bench_c4(gen, bits, 10, 3)
            extra[f"c4_prefill_{bits}bit"] = {k: round(v, 4) for k, v in r.items()}
    if want("c3"):
        for T in (1, 16, 64):
            r = bench_moe(gen, "c3", 128, 4096, 2048, 2, 64, 4, T, s2, w2)
            extra[f"c3_moe_T{T}"] = {k: round(v, 4) for k, v in r.items()}
    if want("c5"):
        for T in (1, 32):
            r = bench_moe(gen, "c5", 512, 4096, 1024, 2, 128, 10, T, s2, w2, shared_I=4096,
                          skew=True)
            extra[f"c5_moe_T{T}"] = {k: round(v, 4) for k, v in r.items()}
            r = bench_attn8(gen, T, s2, w2)
            extra[f"c5_attention_8bit_T{T}"] = {k: round(v, 4) for k, v in r.items()}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_c2()
        cpu["other"] = {"c3_moe_T1": cpu_baseline_moe(),
                        "c4_prefill_4bit": cpu_baseline_prefill(4)}
        cpu["note"] = ("the oracle's restatement of the reference CPU path (kind port); its 3/6-bit "
                       "unpack is vectorised where the reference loops per element "
                       "(pack.py:132-149), so those figures flatter the reference; the MLX CPU "
                       "backend does not exist off Apple silicon and is not timed")

    line = {
        "metric": "decode quant-GEMV HBM GB/s (% of 8 TB/s peak); MoE layer tokens/sec",
        "value": round(res["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) bf16 weights quantized on the GPU, N(0,1) bf16 activations)",
        "config": {
            "workload": "config 2: mixed-precision block decode, batch 1 (q/k/v/o 6-bit, "
                        "gate/up 3-bit, down 2-bit, group 64, hidden 4096, 32/8 heads x 128, "
                        "intermediate 14336); 4 launches per step",
            "global_batch": 1,
            "frac_hbm_peak": round(res["gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_step": res["bytes"],
            "weight_copies_rotated": res["copies"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "gemv_row_kernel, gate|up grouped launch (3-bit g64, 2 x 14336 x 4096, batch 1)",
            "bound": "hbm",
            "achieved": round(res["gu_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(res["gu_gbs"] / HBM_PEAK_GBS, 4),
            "avg_launch_ms": round(res["gu_ms"], 5),
            "algorithmic_bytes": res["gu_bytes"],
            "traffic": traffic_from_profile(),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
