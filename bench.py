"""Benchmark: attention double backward (Flash-HOG) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-ms T] [--no-cpu-baseline]

Workload: B=4, N=2048, H=16, D=64, bf16, causal, scale 1/sqrt(64); seeded
N(0, 1) inputs resident in HBM. One step = one fhog_attention_bwdbwd call
(D precompute, passes 1-3, pass 4) given (q, k, v, O, L, dO, ddQ, ddK, ddV),
O and L coming from this library's own forward.

value = algorithmic TFLOP/s of the whole double backward: 24 * d flops per
unmasked (query, key) pair (the 12 distinct N_Q x N_K x d products; the
recomputation the passes do is not counted), divided by the measured time.
The roofline block describes the dominant kernel, stage 1 (passes 1-3), whose
algorithmic share is the 9 products it is first to need (18 * d per pair),
timed per launch with HIP events on the stream it runs on.

Clock settling: from idle, the MI355X raises its shader clock over the first
~30 ms of sustained load (measured: the first 50 double backwards of a fresh
process average 405 us, the following ones 337 us, and the same ramp repeats
after a second of idle). Before the W warm-up steps the benchmark therefore
runs the workload untimed for --settle-ms (default 200 ms), so that the K
timed steps measure the sustained rate.

Prints one JSON line on stdout; progress goes to stderr.

    python bench.py --configs

times the double backward through the C ABI on each GPU configuration of the
reference's benchmark set (B4 N2048 H16 D64 bf16 causal; B2 N8192 H16 D128
bf16 causal; B8 N1000 H12 D64 fp16 non-causal; B1 N32768 H8 D64 bf16 causal)
and reports per configuration the time, algorithmic TFLOP/s, the two stages'
times and the peak extra HBM of one call beside the size of one fp32
N_Q x N_K tensor over all (batch, head) pairs, the least a materialising
(quadratic) implementation holds. One JSON line per configuration on stdout.

    python bench.py --hvp-table {b1,tokens}

times instead the end-to-end causal-attention Hessian-vector product through
the public front-end (forward + first backward + double backward), on the
shapes of the reference's HVP tables (flash_hog/csrc/tk_bwdbwd/BENCHMARKS.md:
12 heads, head_dim 64, causal, fp32 inputs cast to bf16 around the attention
call; "b1" = batch 1 at sequence 512 ... 131072, "tokens" = batch x sequence
= 262144). Prints one markdown row per shape on stderr and one JSON line per
shape on stdout. Up to sequence 4096 the HVP is also captured in a HIP graph
(torch.cuda.graph) and the mean replay time reported beside the eager time.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
for _p in (REPO, REPO / "flash-hog_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

MI355X_PEAK_BF16_TFLOPS = 2516.6  # dense bf16 MFMA
MI355X_PEAK_HBM_GBS = 8000.0

WORKLOAD = dict(batch=4, seq=2048, heads=16, head_dim=64, dtype="bf16", causal=True)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def unmasked_pairs(n_q, n_k, causal):
    if not causal:
        return n_q * n_k
    full = min(n_q, n_k)
    return full * (full + 1) // 2 + max(0, n_q - n_k) * n_k


def make_inputs(torch, B, N, H, D, dtype, device, seed=0):
    names = ("q", "k", "v", "do", "ddq", "ddk", "ddv")
    out = {}
    for i, n in enumerate(names):
        gen = torch.Generator().manual_seed(seed + i)
        out[n] = torch.randn((B, N, H, D), generator=gen).to(dtype).to(device)
    return out


# HBM bytes per launch of the stage-1 kernel, measured by two rocprofv3 PMC runs
# of this benchmark (FETCH_SIZE, then WRITE_SIZE) and calibrated with the same
# counters on a plain device copy of known size; written by the profiling step
# into profiles/ (see the file for the commands).
TRAFFIC_FILE = REPO / "profiles" / "bwdbwd_q32_kernel_b4_n2048_h16_d64_bf16_causal.traffic.json"


def stage1_traffic():
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    fetch = t["kernel_fetch_kib"] * t["copy_read_bytes"] / t["copy_fetch_kib"]
    write = t["kernel_write_kib"] * t["copy_write_bytes"] / t["copy_write_kib"]
    return {"bytes": int(fetch + write), "source": TRAFFIC_FILE.name}


def available_cores():
    """CPUs this process may use: its affinity mask, capped by the cgroup CPU
    quota (cpu.max, cgroup v2) when one is set, since a container can see more
    CPUs than its quota lets it run at once."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, math.ceil(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_baseline(args, B, N, H, D, scale, causal):
    """The reference's CPU path restated: torch-CPU fp32 autograd double VJP of
    materialised attention (oracle/autodiff.py), one (batch, head) slice at a
    time, over the whole workload or until about args.cpu_seconds elapse."""
    import torch

    from oracle import autodiff

    cores = args.cpu_threads or available_cores()
    torch.set_num_threads(cores)
    names = ("q", "k", "v", "do", "ddq", "ddk", "ddv")

    def slice_inputs(i):
        gen = torch.Generator().manual_seed(1000 + i)
        return [torch.randn((1, N, 1, D), generator=gen) for _ in names]

    autodiff.double_vjp(*slice_inputs(0), scale, causal)  # warm-up
    done, busy = 0, 0.0
    while done < B * H and busy < args.cpu_seconds:
        xs = slice_inputs(done)
        t0 = time.perf_counter()
        autodiff.double_vjp(*xs, scale, causal)
        busy += time.perf_counter() - t0
        done += 1
    flops = 24.0 * D * unmasked_pairs(N, N, causal) * done
    return {
        "value": flops / busy / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{done} of the {B * H} (batch, head) slices of B{B} N{N} H{H} D{D} causal, fp32 torch-CPU "
                   f"autograd double VJP of materialised attention (oracle/autodiff.py), {busy:.1f} s"),
        "ms_per_slice": busy / done * 1e3,
    }


def settle(torch, fn, ms, batch=8):
    """Runs fn untimed until `ms` of wall time have passed (GPU clock ramp)."""
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()
        n += batch
    log(f"settle: {n} untimed calls in {(time.perf_counter() - t0) * 1e3:.0f} ms")


GRAPH_MAX_SEQ = 4096  # graph replay is also timed up to this sequence length (host overhead matters there)

HVP_TABLES = {
    "b1": [(1, 512 << i) for i in range(9)],
    "tokens": [(262144 // (512 << i), 512 << i) for i in range(9)],
}


def hvp_table(args):
    """Mean HVP time per shape (the reference's protocol: warm-up, then 10
    iterations, 5 at sequence >= 16k, 3 at >= 64k) and faithfulness: cosine
    similarity and max relative error of the concatenated (q, k, v) HVP against
    a dense fp32 torch-autograd HVP of the same function where that fits
    (batch * sequence^2 <= 2048^2), else, on two (batch, head) slices (the
    first and the last), against the fp32 closed form of the attention double
    backward evaluated a block of query rows at a time
    (tests/gpu_reference.py, pinned to the fp64 oracle by the GPU tests)."""
    import torch

    sys.path.insert(0, str(REPO / "tests"))
    import gpu_reference

    import flash_hog

    dev = torch.device("cuda:0")
    H, D = 12, 64
    scale = D ** -0.5

    def attn_flash(dtype):
        def f(q, k, v):
            return flash_hog.dot_product_attention(q.to(dtype), k.to(dtype), v.to(dtype), is_causal=True,
                                                   scale=scale).float()
        return f

    def attn_standin(dtype):
        """The HVP's function with attention replaced by an element-wise
        product (same casts, same autograd graph depth, no kernel of this
        library): its eager HVP time is what everything but attention costs,
        host time at short sequences (where the GPU work is shorter than the
        host's) and the casts' and products' memory traffic at large batch."""
        def f(q, k, v):
            return (q.to(dtype) * k.to(dtype) * v.to(dtype)).float()
        return f

    def attn_dense(q, k, v):
        qh, kh, vh = (t.permute(0, 2, 1, 3).contiguous() for t in (q, k, v))
        s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) * scale
        n = s.shape[-1]
        s = s.masked_fill(torch.ones(n, n, device=s.device, dtype=torch.bool).triu(1), float("-inf"))
        return torch.matmul(torch.softmax(s, dim=-1), vh).permute(0, 2, 1, 3)

    def hvp(attn, x, cot, tan):
        """grad of <grad(loss), tan> with loss = <attn(x), cot>, as the reference's make_hvp."""
        x = [t.detach().requires_grad_(True) for t in x]
        loss = (attn(*x) * cot).sum()
        g = torch.autograd.grad(loss, x, create_graph=True)
        return torch.autograd.grad(g, x, tan)

    def hvp_vjp(attn, x, cot, tan):
        """The same HVP as two vector-Jacobian products (no reduction), for graph capture."""
        x = [t.detach().requires_grad_(True) for t in x]
        g = torch.autograd.grad(attn(*x), x, cot, create_graph=True)
        return torch.autograd.grad(g, x, tan)

    def eager_ms(f, x, cot, tan, iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(2):
            out = hvp(f, x, cot, tan)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            out = hvp(f, x, cot, tan)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters, out

    def graph_ms(f, x, cot, tan, iters):
        """Mean replay time of the HVP captured in a HIP graph (torch.cuda.graph)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                hvp_vjp(f, x, cot, tan)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = hvp_vjp(f, x, cot, tan)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        del graph, out
        return e0.elapsed_time(e1) / iters

    def hvp_slices(x, cot, tan, slices):
        """The HVP on (batch, head) slices: (q, k, v) cotangents of the double
        backward with residual (x, O, L, dO = cot) and cotangents tan, with O, L
        from the fp32 forward of x; attention heads are independent, so a slice
        of the full HVP is the HVP of that slice."""
        out = []
        for b, h in slices:
            sl = lambda t: t[b, :, h, :].contiguous()
            q, k, v = (sl(t) for t in x)
            rows = max(128, min(4096, (1 << 28) // q.shape[0]))
            o, lse = gpu_reference.fwd_head_chunked(q, k, v, scale, True, rows=rows)
            dq2, dk2, dv2, _ = gpu_reference.bwdbwd_head_chunked(
                q, k, v, o, sl(cot), *(sl(t) for t in tan), lse, scale, True, rows=rows)
            out += [dq2, dk2, dv2]
        return out

    def compare(a, r):
        a = torch.cat([t.double().flatten() for t in a])
        r = torch.cat([t.double().flatten() for t in r])
        cos = float(torch.dot(a, r) / (a.norm() * r.norm()))
        return cos, float((a - r).abs().max() / r.abs().max())

    rows = []
    settled = False
    log("| batch | seq | HVP (ms) | HVP, graph replay (ms) | stand-in HVP (ms) | faithfulness |")
    log("|--:|--:|--:|--:|--:|:--|")
    for B, N in HVP_TABLES[args.hvp_table]:
        gen = torch.Generator().manual_seed(B * 7919 + N)
        mk = lambda: torch.randn((B, N, H, D), generator=gen).to(dev)
        x, cot, tan = [mk(), mk(), mk()], mk(), [mk(), mk(), mk()]
        f = attn_flash(torch.bfloat16)
        iters = 3 if N >= 65536 else 5 if N >= 16384 else 10
        if not settled:
            settle(torch, lambda: hvp(f, x, cot, tan), args.settle_ms, batch=1)
            settled = True
        ms, out = eager_ms(f, x, cot, tan, iters)
        gms = graph_ms(f, x, cot, tan, iters) if N <= GRAPH_MAX_SEQ else None
        standin_ms = eager_ms(attn_standin(torch.bfloat16), x, cot, tan, iters)[0] if N <= GRAPH_MAX_SEQ else None
        if B * N * N <= 2048 * 2048:
            ref, against = hvp(attn_dense, x, cot, tan), "dense fp32"
        else:
            slices = [(0, 0), (B - 1, H - 1)]
            ref, against = hvp_slices(x, cot, tan, slices), "fp32 closed form, 2 heads"
            out = [t[b, :, h, :] for b, h in slices for t in out]
        faith = "not measured"
        row = {"table": args.hvp_table, "batch": B, "seq": N, "heads": H, "head_dim": D, "hvp_ms": round(ms, 4),
               "hvp_graph_ms": None if gms is None else round(gms, 4),
               "standin_hvp_ms": None if standin_ms is None else round(standin_ms, 4), "iterations": iters}
        if ref is not None:
            cos, rel = compare(out, ref)
            faith = f"cos {cos:.4f}, max rel err {rel:.1e} vs {against}"
            row.update(cos=round(cos, 6), max_rel_err=rel, against=against)
        torch.cuda.synchronize()
        gtxt = "-" if gms is None else f"{gms:.2f}"
        ftxt = "-" if standin_ms is None else f"{standin_ms:.2f}"
        log(f"| {B} | {N} | {ms:.2f} | {gtxt} | {ftxt} | {faith} |")
        print(json.dumps(row), flush=True)
        rows.append(row)
        del x, cot, tan, out, ref
        torch.cuda.empty_cache()
    return 0


CONFIGS = [
    dict(name="B4 N2048 H16 D64 bf16 causal", batch=4, seq=2048, heads=16, head_dim=64, dtype="bf16", causal=True),
    dict(name="B2 N8192 H16 D128 bf16 causal", batch=2, seq=8192, heads=16, head_dim=128, dtype="bf16", causal=True),
    dict(name="B8 N1000 H12 D64 fp16 non-causal", batch=8, seq=1000, heads=12, head_dim=64, dtype="fp16",
         causal=False, qkv_scale=0.5),
    dict(name="B1 N32768 H8 D64 bf16 causal", batch=1, seq=32768, heads=8, head_dim=64, dtype="bf16", causal=True),
]


def run_configs(args):
    """Times the double backward on every GPU configuration (see the module docstring)."""
    import torch

    from flash_hog import _hip

    dev = torch.device("cuda:0")
    lib = _hip.lib()
    dtypes = {"bf16": torch.bfloat16, "fp16": torch.float16}
    log("| config | ms | alg. TFLOP/s | % bf16 peak | stage 1 ms | stage 2 ms | peak extra HBM | one fp32 N x N tensor |")
    log("|---|--:|--:|--:|--:|--:|--:|--:|")
    for c in CONFIGS:
        if args.config and not any(sel in c["name"] for sel in args.config):
            continue
        B, N, H, D = c["batch"], c["seq"], c["heads"], c["head_dim"]
        dtype, causal = dtypes[c["dtype"]], c["causal"]
        scale = 1.0 / math.sqrt(D)
        x = make_inputs(torch, B, N, H, D, dtype, dev)
        if c.get("qkv_scale"):
            for k in ("q", "k", "v"):
                x[k] = (x[k].float() * c["qkv_scale"]).to(dtype)
        o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
        outs = [torch.empty_like(x[k]) for k in ("q", "k", "v", "do")]
        stats = torch.empty((3, B, H, N), device=dev, dtype=torch.float32)
        stream = torch.cuda.current_stream(dev)
        s_ptr = stream.cuda_stream
        common = (x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), o.data_ptr(), x["do"].data_ptr(),
                  x["ddq"].data_ptr(), x["ddk"].data_ptr(), x["ddv"].data_ptr(), lse.data_ptr(),
                  *[t.data_ptr() for t in outs], stats[0].data_ptr(), stats[1].data_ptr(), stats[2].data_ptr())
        dims = (B, N, N, H, H, D, _hip.DTYPE_CODES[dtype], int(causal), scale)
        step = lambda: _hip.check(lib.fhog_attention_bwdbwd(s_ptr, *common, *dims))
        stage = lambda k: _hip.check(lib.fhog_attention_bwdbwd_stage(s_ptr, k, *common, *dims))
        settle(torch, step, args.settle_ms, batch=1)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        steps = max(10, args.steps // max(1, (N * N * B * H) // (2048 * 2048 * 64)))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for e in ev:
            e[0].record(stream)
            stage(1)
            e[1].record(stream)
            stage(2)
            e[2].record(stream)
        torch.cuda.synchronize()
        s1 = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
        s2 = sum(e[1].elapsed_time(e[2]) for e in ev) / steps
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse, causal, scale)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(dev) - base
        pairs = unmasked_pairs(N, N, causal) * B * H
        tflops = 24.0 * D * pairs / (ms * 1e-3) / 1e12
        quad = 4.0 * B * H * N * N
        row = {"config": c["name"], "ms": round(ms, 4), "alg_tflops": round(tflops, 2),
               "pct_of_bf16_peak": round(100 * tflops / MI355X_PEAK_BF16_TFLOPS, 2), "stage1_ms": round(s1, 4),
               "stage2_ms": round(s2, 4), "peak_extra_hbm_bytes": int(peak), "fp32_nxn_bytes": int(quad),
               "steps": steps}
        log(f"| {c['name']} | {ms:.3f} | {tflops:.1f} | {100 * tflops / MI355X_PEAK_BF16_TFLOPS:.1f} | {s1:.3f} | "
            f"{s2:.3f} | {peak / 2**20:.1f} MiB | {quad / 2**30:.1f} GiB |")
        print(json.dumps(row), flush=True)
        del x, o, lse, outs, stats
        torch.cuda.empty_cache()
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description="Flash-HOG double-backward benchmark")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="run the workload untimed for this long before the warm-up steps (clock ramp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the CPU baseline (default: every core available to the process)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (PMC byte-counter calibration)")
    ap.add_argument("--configs", action="store_true",
                    help="time the double backward on every GPU configuration of the benchmark set instead")
    ap.add_argument("--config", action="append", default=[],
                    help="with --configs: only configurations whose name contains this text (repeatable)")
    ap.add_argument("--hvp-table", choices=sorted(HVP_TABLES),
                    help="time the end-to-end HVP on the shapes of one of the reference's HVP tables instead")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the double backward shards over "
              f"(batch, head) with no exchange, so whole-job throughput at N GPUs is N x the one-GPU value.",
              file=sys.stderr)
        return 2
    if args.hvp_table:
        return hvp_table(args)
    if args.configs:
        return run_configs(args)

    import torch

    from flash_hog import _hip

    dev = torch.device("cuda:0")
    B, N, H, D = WORKLOAD["batch"], WORKLOAD["seq"], WORKLOAD["heads"], WORKLOAD["head_dim"]
    causal = WORKLOAD["causal"]
    dtype = torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    lib = _hip.lib()

    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"calibration copy: {args.calibrate_copy_mib} MiB read + written")

    x = make_inputs(torch, B, N, H, D, dtype, dev)
    o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
    dq2, dk2, dv2, ddo = (torch.empty_like(x[n]) for n in ("q", "k", "v", "do"))
    stats = torch.empty((3, B, H, N), device=dev, dtype=torch.float32)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    s_ptr = stream.cuda_stream
    common = (x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), o.data_ptr(), x["do"].data_ptr(),
              x["ddq"].data_ptr(), x["ddk"].data_ptr(), x["ddv"].data_ptr(), lse.data_ptr(),
              dq2.data_ptr(), dk2.data_ptr(), dv2.data_ptr(), ddo.data_ptr(),
              stats[0].data_ptr(), stats[1].data_ptr(), stats[2].data_ptr())
    dims = (B, N, N, H, H, D, _hip.DTYPE_CODES[dtype], int(causal), scale)

    def step():
        _hip.check(lib.fhog_attention_bwdbwd(s_ptr, *common, *dims))

    def stage(k):
        _hip.check(lib.fhog_attention_bwdbwd_stage(s_ptr, k, *common, *dims))

    mem0 = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    settle(torch, step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly `steps` double backwards.
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / args.steps
    log(f"double backward: {ms_per_step:.4f} ms/step (events), wall {wall * 1e3 / args.steps:.4f} ms/step")

    # Per-kernel timing of both stages with events on the launch stream.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for e in evs:
        e[0].record(stream)
        stage(1)
        e[1].record(stream)
        stage(2)
        e[2].record(stream)
    torch.cuda.synchronize()
    s1_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    s2_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    log(f"stage 1 (passes 1-3): {s1_ms:.4f} ms, stage 2 (pass 4): {s2_ms:.4f} ms")

    pairs = unmasked_pairs(N, N, causal) * B * H
    alg_flops = 24.0 * D * pairs
    value = alg_flops / (ms_per_step * 1e-3) / 1e12
    s1_alg = 18.0 * D * pairs
    s1_tflops = s1_alg / (s1_ms * 1e-3) / 1e12
    # executed MFMA work per unmasked pair: stage 1 = 11 products (5 score and
    # 6 output products in one sweep, 22 d flops) and 1 d for a product with a
    # ones operand that sums x over the keys, stage 2 = 8 products (16 d)
    exec_tflops = (23.0 + 16.0) * D * pairs / (ms_per_step * 1e-3) / 1e12
    traffic = stage1_traffic()

    # Peak memory of one call with torch-owned outputs, against the inputs.
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse, causal, scale)
    torch.cuda.synchronize()
    peak_extra = torch.cuda.max_memory_allocated(dev) - base

    # End-to-end HVP (forward + first backward + double backward), as the reference benchmarks.
    torch.cuda.synchronize()
    for _ in range(3):
        o2, l2 = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
        _hip.attention_bwd(x["q"], x["k"], x["v"], o2, x["do"], l2, causal, scale)
        _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o2, x["do"], x["ddq"], x["ddk"], x["ddv"], l2, causal, scale)
    torch.cuda.synchronize()
    h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h0.record(stream)
    reps = 10
    for _ in range(reps):
        o2, l2 = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
        _hip.attention_bwd(x["q"], x["k"], x["v"], o2, x["do"], l2, causal, scale)
        _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o2, x["do"], x["ddq"], x["ddk"], x["ddv"], l2, causal, scale)
    h1.record(stream)
    torch.cuda.synchronize()
    hvp_ms = h0.elapsed_time(h1) / reps

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu = cpu_baseline(args, B, N, H, D, scale, causal)
        log(f"cpu baseline: {cpu['value']:.4f} TFLOP/s on {cpu['cores']} cores ({cpu['sample']})")

    result = {
        "metric": "double-bwd TFLOP/s + % bf16 MFMA peak, B4 H16 N2048 D64 causal",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "attention double backward (Flash-HOG), causal", "batch": B, "seq_len": N,
                   "heads": H, "head_dim": D, "scale": scale, "parallelism": "none (1 GPU)"},
        "pct_of_bf16_peak": round(100.0 * value / MI355X_PEAK_BF16_TFLOPS, 3),
        "roofline": {"bound": "mfma", "kernel": "bwdbwd_q32_kernel (stage 1, passes 1-3 in one sweep)",
                     "achieved": round(s1_tflops, 3), "peak": MI355X_PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(s1_tflops / MI355X_PEAK_BF16_TFLOPS, 5),
                     "traffic": None if traffic is None else traffic["bytes"],
                     "traffic_source": None if traffic is None else traffic["source"],
                     "alg_flops_per_launch": s1_alg, "ms_per_launch": round(s1_ms, 5)},
        "cpu_baseline": None if cpu is None else {k: (round(v, 6) if isinstance(v, float) else v)
                                                  for k, v in cpu.items()},
        # whole step: 24 d flops per unmasked pair over the whole double
        # backward's time (the roofline entry above credits stage 1 with the
        # score products stage 2 recomputes)
        "detail": {"whole_step_frac": round(value / MI355X_PEAK_BF16_TFLOPS, 5),
                   "stage2_ms": round(s2_ms, 5), "executed_mfma_tflops": round(exec_tflops, 3),
                   "alg_gflop_per_step": round(alg_flops / 1e9, 3), "peak_extra_hbm_bytes": int(peak_extra),
                   "hvp_ms": round(hvp_ms, 5), "wall_ms_per_step": round(wall * 1e3 / args.steps, 5)},
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
