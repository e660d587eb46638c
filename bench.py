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
    p.add_argument("--profile", choices=("gateup", "copy"), default=None,
                   help="run only the dominant kernel (gateup) or a plain 256 MiB copy (copy), "
                        "eagerly, for rocprofv3 counter passes; prints one JSON line")
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
    def step(i):
        # The router GEMV runs (its bytes are counted below); routing uses the config's
        # synthetic N(0,1) logits so that the expert load is the one the config states.
        blk.gate(xs[i % R])
        return blk(xs[i % R], logits=logit_sets[i % R])

    ms = timed(step, steps, warmup)
    # Algorithmic bytes of one layer: router + distinct selected experts (+ shared).
    per_expert = 3 * (I * H * bits // 8 + I * (H // gs) * 4)  # gate + up + down
    distinct = []
    for lg in logit_sets:
        idx, _ = jq.moe_route(lg, k)
        distinct.append(len(torch.unique(idx)))
    mean_distinct = sum(distinct) / len(distinct)
    nb = router.nbytes() + mean_distinct * per_expert
    if shared_I:
        nb += 3 * (shared_I * H + shared_I * (H // 64) * 4)
    return dict(ms=ms, tokens_per_s=T / ms * 1e3, distinct_experts=mean_distinct,
                bytes=nb, gbs=nb / ms / 1e6, frac=nb / ms / 1e6 / HBM_PEAK_GBS)


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

    layer, acts, _, _ = c2_block(gen, 1)
    R = copies_for(layer["g"].nbytes() + layer["u"].nbytes())
    gs = [(layer["g"], layer["u"])] + [(layer["g"].clone(), layer["u"].clone())
                                      for _ in range(R - 1)]
    for i in range(steps):
        g, u = gs[i % R]
        jq.quantized_matmul_multi(acts[0], [g.tup(), u.tup()])
    torch.cuda.synchronize()
    x = acts[0]
    nb = layer["g"].nbytes() + layer["u"].nbytes() + 2 * x.numel() + 2 * 2 * 14336
    return {"profile": "gateup", "algorithmic_bytes": nb, "launches": steps, "copies": R}


# ----------------------------------------------------------------------------- main


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a run)"}))
        sys.exit(2)
    os.environ.setdefault("OMP_NUM_THREADS", str(len(os.sched_getaffinity(0))))
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

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_c2()

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
