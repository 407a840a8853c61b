"""Benchmark of the MI355X VSA hot path (one JSON line on stdout).

Workload (the metric's configuration): fused VSA
forward + backward, B=1, H=40, S=40,960, D=128, bf16, block (4,8,8) -> 256
tokens, 160 full blocks, topk=20, gate ~ U(0,1) of shape [B,H,S,D];
q, k, v, dO ~ N(0,1).  A step is one forward + backward of ``vsa_mi355x.mi355x_vsa``
over that synthetic batch, inputs resident in HBM.

value = effective TFLOP/s = 3.5 * 4*B*H*Qb*topk*be^2*D / step time (only the
selected block pairs count; recompute does not).  Beside it: per-kernel HIP
event timings (the roofline of the dominant kernel) and the CPU oracle timed
on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "simple-vsa_amd"))

MFMA_BF16_PEAK_TFLOPS = 2516.6   # MI355X dense bf16
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3      # MI355X published dense fp32

CFG = dict(B=1, H=40, S=40960, D=128, block=(4, 8, 8), topk=20)

# The BASELINE.json configurations that run on the GPU (configs[1..4]); c3 is
# the metric's workload and the default.
WORKLOADS = {
    "c2": dict(name="Small GPU (BASELINE configs[1])", B=1, H=12, S=16384, D=128,
               block=(1, 1, 256), topk=8, gate="token", last_valid=200),
    "c3": dict(name="Video-DiT mid shape (BASELINE configs[2])", B=1, H=40, S=40960, D=128,
               block=(4, 8, 8), topk=20, gate="full"),
    # c3 with a per-token gate [B, H, S, 1] (the config leaves the gate's shape open)
    "c3tok": dict(name="Video-DiT mid shape, gate [B,H,S,1]", B=1, H=40, S=40960, D=128,
                  block=(4, 8, 8), topk=20, gate="token"),
    "c4": dict(name="Long video shape (BASELINE configs[3])", B=1, H=40, S=92160, D=128,
               block=(1, 1, 256), topk=45, gate=None, every8th=192, amp=0.5),
    "c5": dict(name="Route-skew explicit routing (BASELINE configs[4])", B=1, H=24, S=40960,
               D=64, block=(1, 1, 64), topk=32, gate=None, zipf=1.2),
    # not a BASELINE row: the c3 sequence in FastVideo's native (4,4,4) tiles at the same
    # 87.5 % sparsity (64-token blocks, topk 80)
    "t444": dict(name="c3 sequence with FastVideo (4,4,4) tiles", B=1, H=40, S=40960, D=128,
                 block=(4, 4, 4), topk=80, gate="full"),
    # not a BASELINE row: head_dim 256 at the c3 sequence and sparsity, half the heads
    # (the same FLOPs as c3)
    "d256": dict(name="c3 sequence at head_dim 256", B=1, H=20, S=40960, D=256,
                 block=(4, 8, 8), topk=20, gate="full"),
    # not a BASELINE row: the c3 shape with fp32 inputs (fp32 vector-ALU kernels)
    "c3f32": dict(name="Video-DiT mid shape in fp32", B=1, H=40, S=40960, D=128,
                  block=(4, 8, 8), topk=20, gate="full", dtype="fp32"),
}


def flops_fwd(B, H, S, D, be, topk):
    return 4.0 * B * H * (S // be) * topk * be * be * D


def _events_time(fn, iters):
    import torch
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def _timed_steps(fn, steps):
    """Run ``fn`` ``steps`` times between two device synchronisations.
    Returns (mean ms per step from the host clock around the whole run, median
    ms per step from HIP events recorded between consecutive steps on the
    launch stream; recording them adds no synchronisation)."""
    import torch
    stream = torch.cuda.current_stream()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks[0].record(stream)
    for i in range(steps):
        fn()
        marks[i + 1].record(stream)
    torch.cuda.synchronize()
    mean = (time.perf_counter() - t0) * 1e3 / steps
    per = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(steps))
    mid = steps // 2
    median = per[mid] if steps % 2 else 0.5 * (per[mid - 1] + per[mid])
    return mean, median


def host_cpu():
    """The host CPU the baseline runs on: model, logical CPUs of the machine and
    of this process, and the physical cores among this process's CPUs."""
    info = {"model": None, "os_cpu_count": os.cpu_count()}
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except AttributeError:
        allowed = list(range(os.cpu_count() or 1))
    info["cpus_allowed"] = len(allowed)
    cores, proc = {}, {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f.read().split("\n") + [""]:
                if not ln.strip():
                    if "processor" in proc:
                        cores[int(proc["processor"])] = (proc.get("physical id", "0"),
                                                         proc.get("core id", proc["processor"]))
                        info["model"] = info["model"] or proc.get("model name")
                    proc = {}
                    continue
                key, _, val = ln.partition(":")
                proc[key.strip()] = val.strip()
    except OSError:
        pass
    phys = {cores[c] for c in allowed if c in cores}
    info["physical_cores_allowed"] = len(phys) if phys else len(allowed)
    return info


def cpu_baseline(heads: int = 8):
    """The CPU oracle (a restatement of torch_vsa) fwd+bwd on `heads` heads of
    the workload, one head at a time (heads are independent; one head's
    fp32 intermediates are a few GB), with one torch thread per physical core
    this process may use (at most OMP_NUM_THREADS when that is set).
    Returns (TFLOP/s, seconds, threads, host description)."""
    import torch
    sys.path.insert(0, ROOT)
    from oracle import vsa_oracle as O
    host = host_cpu()
    threads = host["physical_cores_allowed"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(max(1, threads))
    threads = torch.get_num_threads()
    B, S, D, topk = CFG["B"], CFG["S"], CFG["D"], CFG["topk"]
    be = math.prod(CFG["block"])
    g = torch.Generator().manual_seed(0)
    vbs = torch.full((S // be,), be)
    total = 0.0
    for _ in range(heads):
        shape = (B, 1, S, D)
        q, k, v = (torch.randn(shape, generator=g).to(torch.bfloat16).requires_grad_()
                   for _ in range(3))
        do = torch.randn(shape, generator=g).to(torch.bfloat16)
        gate = torch.rand(shape, generator=g).to(torch.bfloat16).requires_grad_()
        t0 = time.perf_counter()
        out = O.torch_vsa(q, k, v, vbs, vbs, topk, CFG["block"], gate)
        torch.autograd.grad(out, (q, k, v, gate), do)
        total += time.perf_counter() - t0
    f = 3.5 * flops_fwd(B, heads, S, D, be, topk)
    return f / total / 1e12, total, threads, host


def _zipf_routes(h, qb, kb, tk, s, seed=5):
    import numpy as np
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, kb + 1) ** s
    p /= p.sum()
    perm = rng.permutation(kb)
    sel = np.stack([np.stack([perm[rng.choice(kb, tk, replace=False, p=p)] for _ in range(qb)])
                    for _ in range(h)])
    return sel[None].astype(np.int32)


def run_workload(key, steps, warmup):
    """Time fwd and fwd+bwd of one BASELINE workload; report ms, effective
    TFLOP/s and the peak HBM the op allocates beyond its inputs."""
    import torch
    from vsa_mi355x import mi355x as M
    w = WORKLOADS[key]
    dev = torch.device("cuda", 0)
    B, H, S, D, topk = w["B"], w["H"], w["S"], w["D"], w["topk"]
    be = math.prod(w["block"])
    nb = S // be
    amp = w.get("amp", 1.0)
    dt = {"bf16": torch.bfloat16, "fp32": torch.float32}[w.get("dtype", "bf16")]
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(B, H, S, D, generator=g, device=dev, dtype=dt) * amp
               for _ in range(3))
    do = torch.randn(B, H, S, D, generator=g, device=dev, dtype=dt)
    gate = None
    if w["gate"] == "full":
        gate = torch.rand(B, H, S, D, generator=g, device=dev, dtype=dt)
    elif w["gate"] == "token":
        gate = torch.rand(B, H, S, 1, generator=g, device=dev, dtype=dt)
    vbs = torch.full((nb,), be, dtype=torch.int32)
    if "last_valid" in w:
        vbs[-1] = w["last_valid"]
    if "every8th" in w:
        vbs[7::8] = w["every8th"]
    vbs = vbs.to(dev)
    leaves = [t.requires_grad_() for t in (q, k, v)] + ([gate.requires_grad_()] if gate is not None else [])
    if "zipf" in w:
        sel = torch.from_numpy(_zipf_routes(H, nb, nb, topk, w["zipf"])).to(dev)
        fwd = lambda: M.mi355x_sparse_attention(q, k, v, sel, vbs, block_size=w["block"])
    else:
        fwd = lambda: M.mi355x_vsa(q, k, v, vbs, vbs, topk, w["block"], gate)

    def step():
        torch.autograd.grad(fwd(), leaves, do)

    def fwd_only():
        with torch.no_grad():
            fwd()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    ms, ms_median = _timed_steps(step, steps)
    fms = _events_time(fwd_only, max(5, steps // 2))
    F = flops_fwd(B, H, S, D, be, topk)   # padded volume, selected pairs only
    return {"workload": key, "name": w["name"], "dtype": w.get("dtype", "bf16"),
            "ms_fwd_bwd": round(ms, 3), "ms_fwd_bwd_median": round(ms_median, 3),
            "ms_fwd": round(fms, 3),
            "tflops_fwd_bwd": round(3.5 * F / (ms * 1e-3) / 1e12, 1),
            "tflops_fwd": round(F / (fms * 1e-3) / 1e12, 1),
            "pct_bf16_peak_fwd_bwd": round(100 * 3.5 * F / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 2),
            "peak_hbm_gib_beyond_inputs": round(peak / 2 ** 30, 3), "steps": steps,
            **({"pct_fp32_peak_fwd_bwd": round(100 * 3.5 * F / (ms * 1e-3) / 1e12
                                               / FP32_PEAK_TFLOPS, 2)}
               if dt == torch.float32 else {})}


def run_tiling(steps, warmup):
    """tile / untile of a c3-sized token tensor ([1, 40960, 40, 128] bf16 on a
    20 x 32 x 64 latent in (4, 8, 8) tiles) and of a latent with partial tiles;
    HBM-bound row moves, reported against the 8 TB/s roof (read + write bytes)."""
    import torch
    from vsa_mi355x import tiling
    out = {"workload": "tiling", "cases": []}
    for shape, ts, inner in (((20, 32, 64), (4, 8, 8), (40, 128)),
                             ((21, 30, 52), (4, 4, 4), (40, 128))):
        S = math.prod(shape)
        meta = tiling.build_vsa_metadata(shape, ts, device="cuda")
        nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
        x = torch.randn(1, S, *inner, device="cuda", dtype=torch.bfloat16)
        tpi, npi, rev = (meta[k] for k in ("tile_partition_indices", "non_pad_index",
                                           "reverse_tile_partition_indices"))
        t = tiling.tile(x, tpi, npi, nb, be)
        row = 2 * math.prod(inner)
        for _ in range(warmup):
            tiling.tile(x, tpi, npi, nb, be)
            tiling.untile(t, npi, rev)
        t_ms = _events_time(lambda: tiling.tile(x, tpi, npi, nb, be), steps)
        u_ms = _events_time(lambda: tiling.untile(t, npi, rev), steps)
        meta_ms = _events_time(lambda: tiling._metadata.__wrapped__(shape, ts, torch.device("cuda", 0)), steps)
        t_bytes = S * row + nb * be * row          # read the tokens, write the padded layout
        u_bytes = 2 * S * row                      # read the real rows, write raster order
        out["cases"].append({
            "latent": list(shape), "tile": list(ts), "row_bytes": row, "tokens": S,
            "padded_rows": nb * be,
            "tile_ms": round(t_ms, 4), "tile_gbps": round(t_bytes / (t_ms * 1e-3) / 1e9, 1),
            "tile_frac_hbm": round(t_bytes / (t_ms * 1e-3) / 8e12, 3),
            "untile_ms": round(u_ms, 4), "untile_gbps": round(u_bytes / (u_ms * 1e-3) / 1e9, 1),
            "untile_frac_hbm": round(u_bytes / (u_ms * 1e-3) / 8e12, 3),
            "metadata_ms": round(meta_ms, 4)})
    return out


def run_gate(steps, warmup):
    """c3 with the gate produced by CompressionGate(dim=5120, heads=40) from
    hidden states [1, 40960, 5120]: fwd+bwd of (gate GEMM + mi355x_vsa) with the
    gate consumed in the producer's token-major layout, against the same step
    with the gate made contiguous first (what a [B,H,S,D]-only op needs)."""
    import torch
    from vsa_mi355x import CompressionGate
    from vsa_mi355x import mi355x as M
    B, H, S, D, topk = CFG["B"], CFG["H"], CFG["S"], CFG["D"], CFG["topk"]
    be = math.prod(CFG["block"])
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16)
                   for _ in range(4))
    hidden = torch.randn(B, S, H * D, generator=g, device=dev, dtype=torch.bfloat16)
    layer = CompressionGate(H * D, H).to(dev, torch.bfloat16)
    vbs = torch.full((S // be,), be, device=dev, dtype=torch.int32)
    leaves = [t.requires_grad_() for t in (q, k, v)] + list(layer.parameters())
    res = {"workload": "gate", "gemm_tflop": 2 * B * S * (H * D) ** 2 / 1e12}
    for name, contiguous in (("token_major", False), ("contiguous_copy", True)):
        def step():
            gate = layer(hidden)
            if contiguous:
                gate = gate.contiguous()
            out = M.mi355x_vsa(q, k, v, vbs, vbs, topk, CFG["block"], gate)
            torch.autograd.grad(out, leaves, do)
        for _ in range(warmup):
            step()
        res[name + "_ms"] = round(_events_time(step, steps), 3)
    res["saved_ms"] = round(res["contiguous_copy_ms"] - res["token_major_ms"], 3)
    return res


def run_tiled(steps, warmup):
    """c3 as a video DiT holds it: raster-order tokens of a 20x32x64 latent in
    (4,8,8) tiles (40,960 tokens, 160 blocks of 256), gate of q's shape.
    fwd+bwd of mi355x_vsa_tiled (tile / untile fused into the op) against the
    unfused tile -> mi355x_vsa -> untile composition, with q, k, v, gate, dout
    head-major [B, H, S, D] and token-major [B, S, H, D]."""
    import torch
    from vsa_mi355x import tiled, tiling
    B, H, D, topk = CFG["B"], CFG["H"], CFG["D"], CFG["topk"]
    shape, ts = (20, 32, 64), CFG["block"]
    S = math.prod(shape)
    nb, be = math.prod([math.ceil(a / b) for a, b in zip(shape, ts)]), math.prod(ts)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16)
                   for _ in range(4))
    gate = torch.rand(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16)
    leaves = [t.requires_grad_() for t in (q, k, v, gate)]
    meta = tiling.build_vsa_metadata(shape, ts, device=dev)
    res = {"workload": "tiled", "latent": list(shape), "tile": list(ts)}
    # token-major [B, S, H, D] copies: the layout a DiT's projections produce
    qt, kt, vt, gt = (x.detach().transpose(1, 2).contiguous().requires_grad_()
                      for x in (q, k, v, gate))
    dot = do.transpose(1, 2).contiguous()
    runs = (("fused", lambda: tiled.mi355x_vsa_tiled(q, k, v, shape, topk, ts, gate), leaves, do),
            ("composition", lambda: tiled._composition(q, k, v, meta, nb, be, ts, topk, gate),
             leaves, do),
            ("token_major_fused", lambda: tiled.mi355x_vsa_tiled(qt, kt, vt, shape, topk, ts, gt,
                                                                 token_major=True),
             [qt, kt, vt, gt], dot),
            ("token_major_composition", lambda: tiled._composition(qt, kt, vt, meta, nb, be, ts,
                                                                   topk, gt, token_major=True),
             [qt, kt, vt, gt], dot))
    for name, fwd, lv, grad in runs:
        def step(fwd=fwd, lv=lv, grad=grad):
            torch.autograd.grad(fwd(), lv, grad)

        def fwd_only(fwd=fwd):
            with torch.no_grad():
                fwd()
        for _ in range(warmup):
            step()
        res[name + "_fwd_bwd_ms"] = round(_events_time(step, steps), 3)
        res[name + "_fwd_ms"] = round(_events_time(fwd_only, steps), 3)
    for pre in ("", "token_major_"):
        res[pre + "saved_fwd_bwd_ms"] = round(res[pre + "composition_fwd_bwd_ms"]
                                              - res[pre + "fused_fwd_bwd_ms"], 3)
        res[pre + "saved_fwd_ms"] = round(res[pre + "composition_fwd_ms"]
                                          - res[pre + "fused_fwd_ms"], 3)
    return res


def run_views(steps, warmup):
    """c3 as a DiT's projections hand it over: q, k, v and the gate are
    [B, H, S, D] views of token-major [B, S, H, D] tensors (the gate producer's
    view, common.py:326-328) and the output is consumed as [B, S, H*D].
    fwd+bwd of mi355x_vsa reading the views in place against the same op on
    contiguous copies (what a contiguous-only kernel needs: three copies in,
    one out, and the same again for the gradients)."""
    import torch
    from vsa_mi355x import mi355x as M
    B, H, S, D, topk = CFG["B"], CFG["H"], CFG["S"], CFG["D"], CFG["topk"]
    be = math.prod(CFG["block"])
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    base = [torch.randn(B, S, H, D, generator=g, device=dev, dtype=torch.bfloat16)
            for _ in range(3)]
    gbase = torch.rand(B, S, H, D, generator=g, device=dev, dtype=torch.bfloat16)
    do = torch.randn(B, S, H * D, generator=g, device=dev, dtype=torch.bfloat16)
    leaves = [t.requires_grad_() for t in (*base, gbase)]
    vbs = torch.full((S // be,), be, dtype=torch.int32, device=dev)
    res = {"workload": "views", "B": B, "H": H, "S": S, "D": D, "block": list(CFG["block"]),
           "topk": topk}

    def views():
        q, k, v, gate = (x.transpose(1, 2) for x in leaves)
        return M.mi355x_vsa(q, k, v, vbs, vbs, topk, CFG["block"], gate)

    def copies():
        q, k, v, gate = (x.transpose(1, 2) for x in leaves)
        return M.mi355x_vsa(q.contiguous(), k.contiguous(), v.contiguous(), vbs, vbs, topk,
                            CFG["block"], gate)

    for name, fwd in (("views", views), ("copies", copies)):
        def step(fwd=fwd):
            out = fwd().transpose(1, 2).reshape(B, S, H * D)
            torch.autograd.grad(out, leaves, do)

        def fwd_only(fwd=fwd):
            with torch.no_grad():
                fwd().transpose(1, 2).reshape(B, S, H * D)
        for _ in range(warmup):
            step()
        res[name + "_fwd_bwd_ms"] = round(_events_time(step, steps), 3)
        res[name + "_fwd_ms"] = round(_events_time(fwd_only, steps), 3)
    res["saved_fwd_bwd_ms"] = round(res["copies_fwd_bwd_ms"] - res["views_fwd_bwd_ms"], 3)
    res["saved_fwd_ms"] = round(res["copies_fwd_ms"] - res["views_fwd_ms"], 3)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)   # BASELINE: >= 10 warm-up iterations
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--kernels-only", action="store_true", help="skip the CPU baseline and summary")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy a 1 GiB buffer 3 times (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--workload-steps", type=int, default=10,
                    help="timed steps of each other BASELINE configuration (c2, c4, c5) "
                         "reported under 'workloads' of the c3 line; 0 skips them")
    ap.add_argument("--cpu-heads", type=int, default=16,
                    help="heads of the workload timed on the CPU oracle (one at a time)")
    ap.add_argument("--workload",
                    choices=sorted(WORKLOADS) + ["tiling", "gate", "tiled", "views"],
                    default="c3",
                    help="BASELINE configuration to run (c3 is the metric's workload)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); every MI355X box "
              "in this setup has a single GPU.  Per-GPU sharding is by heads; see DESIGN.md.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_probe:
        src = torch.ones(1 << 29, device="cuda", dtype=torch.bfloat16)   # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * src.element_size()}))
        return

    from vsa_mi355x import mi355x as M

    if args.workload == "gate":
        print(json.dumps(run_gate(args.steps, args.warmup)), flush=True)
        return
    if args.workload == "tiling":
        print(json.dumps(run_tiling(args.steps, args.warmup)), flush=True)
        return
    if args.workload == "tiled":
        print(json.dumps(run_tiled(args.steps, args.warmup)), flush=True)
        return
    if args.workload == "views":
        print(json.dumps(run_views(args.steps, args.warmup)), flush=True)
        return
    if args.workload != "c3":
        print(json.dumps(run_workload(args.workload, args.steps, args.warmup)), flush=True)
        return

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, H, S, D, topk = CFG["B"], CFG["H"], CFG["S"], CFG["D"], CFG["topk"]
    be = math.prod(CFG["block"])
    nb = S // be
    scale = 1.0 / math.sqrt(D)
    g = torch.Generator(device=dev).manual_seed(0)
    shape = (B, H, S, D)
    q, k, v, do = (torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
                   for _ in range(4))
    gate = torch.rand(shape, generator=g, device=dev, dtype=torch.bfloat16)
    vbs = torch.full((nb,), be, device=dev, dtype=torch.int32)
    for t in (q, k, v, gate):
        t.requires_grad_()

    def step():
        out = M.mi355x_vsa(q, k, v, vbs, vbs, topk, CFG["block"], gate)
        torch.autograd.grad(out, (q, k, v, gate), do)

    def fwd_only():
        with torch.no_grad():
            M.mi355x_vsa(q, k, v, vbs, vbs, topk, CFG["block"], gate)

    for _ in range(args.warmup):
        step()
    ms_step, ms_median = _timed_steps(step, args.steps)
    fwd_ms = _events_time(fwd_only, max(5, args.steps // 2))

    # ---- per-kernel timings (HIP events on the launch stream) -------------
    F_fwd = flops_fwd(B, H, S, D, be, topk)
    with torch.no_grad():
        qd, kd, vd, gd = (t.detach() for t in (q, k, v, gate))
        qc, kc, vc = M.block_mean_qkv(qd, kd, vd, vbs, vbs, be)
        _, probs, outc, sel = M.coarse_forward(qc, kc, vc, topk, scale)
        out, lse, fine = M.sparse_forward(qd, kd, vd, sel, vbs, be, scale, out_c=outc, gate=gd)
        delta, d_outc, _ = M.backward_prep(fine, do, be, out_c=outc, gate=gd)
        dqc, dkc, dvc = M.coarse_backward(qc, kc, vc, probs, d_outc, scale)
        inverse, offsets, counts = M.invert_routes(sel, nb)
        order = M.dkdv_tile_order(counts, B * H, S, D, be)
        from vsa_mi355x import _lib
        code, st = _lib.dtype_code(qd.dtype), _lib.stream_of(qd)
        dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)

        def k_dq():
            _lib.call("vsa_sparse_bwd_dq", _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), _lib.ptr(do),
                      _lib.ptr(lse), _lib.ptr(delta), _lib.ptr(sel), _lib.ptr(vbs), _lib.ptr(dq),
                      _lib.ptr(dqc), _lib.ptr(vbs), B * H, S, S, D, be, topk, scale, code, st)

        def k_dkdv():
            _lib.call("vsa_sparse_bwd_dkdv", _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd),
                      _lib.ptr(do), _lib.ptr(lse), _lib.ptr(delta), _lib.ptr(counts),
                      _lib.ptr(offsets), _lib.ptr(inverse), _lib.ptr(vbs), _lib.ptr(dk),
                      _lib.ptr(dv), _lib.ptr(dkc), _lib.ptr(dvc), B * H, S, S, D, be, topk,
                      scale, _lib.ptr(order), code, st)

        it = 10
        kt = {
            "pool_qkv": (_events_time(lambda: M.block_mean_qkv(qd, kd, vd, vbs, vbs, be), it),
                         None, None),
            "coarse_fwd_topk": (_events_time(lambda: M.coarse_forward(qc, kc, vc, topk, scale), it),
                                None, None),
            "sparse_fwd": (_events_time(lambda: M.sparse_forward(qd, kd, vd, sel, vbs, be, scale,
                                                                 out_c=outc, gate=gd), it),
                           F_fwd, F_fwd),
            "bwd_prep": (_events_time(lambda: M.backward_prep(fine, do, be, out_c=outc, gate=gd),
                                      it), None, None),
            "coarse_bwd": (_events_time(lambda: M.coarse_backward(qc, kc, vc, probs, d_outc,
                                                                  scale), it), None, None),
            "csr_build": (_events_time(lambda: M.invert_routes(sel, nb), it), None, None),
            # attributed (the 2.5 F_fwd backward split 1.5 / 1.0) and executed FLOPs:
            # dK/dV recomputes S and dP (2 of its 4 products)
            "sparse_bwd_dq": (_events_time(k_dq, it), 1.5 * F_fwd, 1.5 * F_fwd),
            "sparse_bwd_dkdv": (_events_time(k_dkdv, it), 1.0 * F_fwd, 2.0 * F_fwd),
        }
    kernels = {n: {"ms": round(t, 4)} for n, (t, _, _) in kt.items()}
    for n, (t, f, fx) in kt.items():
        if f:
            kernels[n]["tflops_algorithmic"] = round(f / (t * 1e-3) / 1e12, 1)
            kernels[n]["tflops_executed"] = round(fx / (t * 1e-3) / 1e12, 1)
            kernels[n]["frac_bf16_peak_executed"] = round(fx / (t * 1e-3) / 1e12
                                                          / MFMA_BF16_PEAK_TFLOPS, 4)
    # the bandwidth kernels against the HBM peak, on the bytes each must move
    # once: pooling reads q, k, v and writes the block means; bwd_prep (delta and
    # the combine backward) reads the fine output, dO and the gate and writes
    # d_gate and delta (the block-sized out_c / d_out_c are counted too)
    tok = qd.numel() * qd.element_size()
    pooled = B * H * nb * D * qd.element_size()
    gbytes = gd.numel() * gd.element_size() if gd is not None else 0
    bw_bytes = {"pool_qkv": 3 * tok + 3 * pooled,
                "bwd_prep": 2 * tok + 2 * gbytes + B * H * S * 4 + 2 * pooled}
    for n, nbytes in bw_bytes.items():
        gbs = nbytes / (kt[n][0] * 1e-3) / 1e9
        kernels[n]["gbs_algorithmic"] = round(gbs, 1)
        kernels[n]["frac_hbm_peak"] = round(gbs / HBM_PEAK_GBS, 3)
    dom = max((n for n in kt if kt[n][1]), key=lambda n: kt[n][0])
    dom_t, dom_f, _ = kt[dom]
    achieved = dom_f / (dom_t * 1e-3) / 1e12

    # HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy of known size)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"{dom}_c3_traffic.txt")
    if os.path.exists(tpath):
        with open(tpath) as f:
            for ln in f:
                if ln.startswith("hbm_bytes_per_launch:"):
                    traffic = int(ln.split(":", 1)[1].strip())

    F_total = 3.5 * F_fwd
    value = F_total / (ms_step * 1e-3) / 1e12
    # the other BASELINE configurations, a few steps each, after c3's tensors are freed
    workloads = None
    if not args.kernels_only and args.workload_steps > 0:
        del q, k, v, do, gate, qd, kd, vd, gd, out, lse, fine, delta, dq, dk, dv
        torch.cuda.empty_cache()
        workloads = {}
        for key in ("c2", "c3tok", "c4", "c5"):
            r = run_workload(key, args.workload_steps, 3)
            workloads[key] = {n: r[n] for n in ("ms_fwd_bwd", "ms_fwd_bwd_median", "ms_fwd",
                                                "tflops_fwd_bwd",
                                                "tflops_fwd", "pct_bf16_peak_fwd_bwd",
                                                "peak_hbm_gib_beyond_inputs", "steps")}
            torch.cuda.empty_cache()
    cpu = None
    if not (args.no_cpu or args.kernels_only):
        cv, cs, cth, host = cpu_baseline(heads=args.cpu_heads)
        cpu = {"value": round(cv, 4), "unit": "TFLOP/s", "cores": cth, "kind": "port",
               "sample": f"oracle torch_vsa fwd+bwd, {args.cpu_heads} of {H} heads of the "
                         "workload, one head at a time "
                         f"(B=1,H=1,S={S},D={D},be={be},topk={topk}, bf16 inputs), "
                         f"{cs:.1f} s wall, throughput in effective TFLOP/s",
               "host": {"cpu_model": host["model"], "os_cpu_count": host["os_cpu_count"],
                        "cpus_allowed": host["cpus_allowed"],
                        "physical_cores_allowed": host["physical_cores_allowed"],
                        "torch_threads": cth}}
    line = {
        "metric": "VSA fwd+bwd ms & effective TFLOP/s (% bf16 MFMA peak) at 40k tokens, block 256",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(ms_median, 4),
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(ms_step - fwd_ms, 4),
        "pct_bf16_peak": round(100 * value / MFMA_BF16_PEAK_TFLOPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q,k,v,dO ~ N(0,1), gate ~ U(0,1), seed 0)",
        "config": {"workload": "Video-DiT mid shape (BASELINE configs[2])", "B": B, "H": H,
                   "seq_len": S, "head_dim": D, "block_size": list(CFG["block"]),
                   "block_elements": be, "topk": topk, "gate": "[B,H,S,D]",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic},
        "kernels": kernels,
        "workloads": workloads,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
