"""Benchmark: the ZeRO optimizer step over one GPU's flat partition.

Workload (the headline): a Llama-3-8B ZeRO-2
one-rank shard of 1,003,782,656 contiguous elements. bf16 grads
N(0, 5e-4^2), fp32 master N(0, 0.02^2), fp32 exp_avg = exp_avg_sq = 0, bf16
params; AdamW lr 3e-4, betas (0.9, 0.95), eps 1e-8, weight_decay 0.1, gradient
clipping at 1.0 (active: the grad norm is about 15.8); bf16 => no loss scaling.
Synthetic data, generated on the GPU with a seeded generator.

One step = K1 (unscale + inf/NaN + norm partials) -> K0 (finalize) -> K2
(AdamW + cast), three launches on torch's current stream, no host sync.
Algorithmic bytes: K1 2 B/elt, K2 28 B/elt, step 30 B/elt.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--numel N]

After the headline's timed steps the same run measures configs[0] and
configs[1] (the flat drop-in step), configs[3] (the ragged K1/K0/K3 step) and
configs[4] (state in pinned host memory) as secondary keys, and
times the reference's CPU route (torch.optim.AdamW on CPU fp32, on the same
inputs) as cpu_baseline.

Prints one JSON line (rank 0). --gpus above 1 is refused: this build runs and
measures one GPU; the multi-GPU layout is described in the design notes.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

HEADLINE_NUMEL = 1_003_782_656
HBM_PEAK_GBS = 8000.0
K1_BYTES, K2_BYTES = 2, 28


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--numel", type=int, default=HEADLINE_NUMEL)
    ap.add_argument("--cpu-sample", type=int, default=-1,
                    help="elements in the CPU-baseline sample (-1: the whole shard; 0 disables it)")
    ap.add_argument("--cpu-steps", type=int, default=5,
                    help="timed CPU-baseline steps after one warm-up (median reported)")
    ap.add_argument("--secondary", type=int, default=1,
                    help="after the headline, also measure configs[0] and configs[1] (the flat drop-in step), "
                         "configs[3] (the ragged K1/K0/K3 step) and configs[4] (state offloaded to pinned host "
                         "memory) in the same run (0 disables)")
    ap.add_argument("--traffic", default=os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                                      "k2_adamw_flat_llama8b_shard_traffic.json"))
    ap.add_argument("--torch-gpu", type=int, default=1,
                    help="also time the reference's update as torch ops on this GPU (context line; 0 disables)")
    ap.add_argument("--tuning", default="",
                    help="k1_bpc,k2_bpc,k2_unroll,nt[,k2_cu_eighths,k2_drain] (library launch-shape override; "
                         "the default is 2,0,0,1,0,-1: 0 and -1 pick by size)")
    ap.add_argument("--k2-chunk", type=int, default=None,
                    help="K2 part size in elements (dsx_set_tuning_k2_chunk; 0: one launch; default: the library's 2^26)")
    ap.add_argument("--fold", type=int, default=None,
                    help="largest partition whose one-call step runs as two launches, K0 folded into K2 "
                         "(dsx_set_tuning_fold; 0: always three launches; default: the library's 3*2^23)")
    ap.add_argument("--tuning-multi", default="",
                    help="k3_bpc,k3_unroll,nt,drain (K3 launch-shape override; k3_bpc 0 picks by chunk count)")
    ap.add_argument("--workload", default="llama8b-shard",
                    choices=["llama8b-shard", "llama8b-dropin", "llama-ragged", "llama70b-offload", "gpt2-small",
                             "mlp", "mlp-train", "ffn-train"],
                    help="llama8b-shard: the headline flat step (K1/K0/K2); llama8b-dropin: the same shard "
                         "through the drop-in optimizer classes in a fresh process; llama-ragged: configs[3]'s 289-tensor "
                         "list through K3; llama70b-offload: configs[4] with state in pinned host memory; "
                         "gpt2-small / mlp: configs[1] / configs[0] through the drop-in optimizer classes, eager, "
                         "graph-replayed and ragged; mlp-train: a whole training iteration of configs[0]'s "
                         "model, eager and captured in one graph; ffn-train: a 0.94e9-parameter training "
                         "iteration with the two ways grads reach the flat buffer (secondary lines, not the headline)")
    ap.add_argument("--pinned-budget-gib", type=float, default=32.0,
                    help="llama70b-offload: pinned host memory for the fp32 state (the shard shrinks to fit)")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="for rocprofv3 --pmc runs: launch K1, K0, K2 and the traffic probe three times each "
                         "(with --workload llama-ragged / gpt2-small: three steps of that list's ragged form) "
                         "and one 1 GiB fp32 copy (the byte-counter calibration), then exit without timing")
    return ap.parse_args()


def k2_parts(n: int, chunk) -> int:
    """Consecutive dispatches one dsx_adamw_flat call issues over n elements
    (the library splits K2 into parts of about 2^26 elements by default)."""
    chunk = (1 << 26) if chunk is None else chunk
    return -(-n // chunk) if chunk > 0 and n > chunk else 1


def _calibration_copy(dev) -> None:
    """A plain copy kernel of known size (2^28 fp32 = 1 GiB read and 1 GiB
    written), three times, so that FETCH_SIZE / WRITE_SIZE per dispatch can
    be scaled by what the counters report for it."""
    import torch
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def profile_ragged(workload: str, dev) -> int:
    """For rocprofv3 runs over the ragged form: three steps of configs[3]'s
    list (K1 over the chunk table, K0, K3), or of configs[1]'s GPT-2-small
    list through the drop-in MultiTensorAdamWOptimizer (K1 over the chunk
    table, K0, K2 for wte and K3 over the other 147 tensors), then the copy
    calibration."""
    import math

    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    if workload == "llama-ragged":
        ts, table = ragged_list(dev, [math.prod(s) for s in llama_ragged_shapes()])
        hyper = AdamWHyper(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=1.0)
        scfg = ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=2, min_scale=1.0)
        bc = BiasCorrectionTable(dev, hyper.beta1, hyper.beta2)
        st = ops.new_state(dev, scfg.init_scale, scfg.hysteresis)
        nparts = ops.suggest_partials(table.numel)
        parts = torch.zeros(nparts, dtype=torch.float64, device=dev)
        out = ops.new_scalars(dev)
        for _ in range(3):
            ops.unscale_norm_multi(table, st, parts, nparts)
            ops.finalize(parts, nparts, st, scfg.to_c(), hyper.to_c(), bc.table, bc.length, out)
            ops.adamw_multi(table, out)
        torch.cuda.synchronize()
        del ts, table
    else:
        from distributedspeed_amd.optimizers import MultiTensorAdamWOptimizer
        gen = torch.Generator(device=dev)
        gen.manual_seed(1)
        ps = [torch.nn.Parameter(torch.empty(s, device=dev).normal_(0.0, 0.02, generator=gen))
              for s in gpt2_small_shapes()]
        sc = ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=1, min_scale=1.0)
        opt = MultiTensorAdamWOptimizer(ps, lr=6e-4, weight_decay=0.01, max_grad_norm=1.0,
                                        param_dtype=torch.float16, loss_scaler=sc, device=dev)
        for p in opt.dsx_params:
            p.grad = (torch.empty(p.shape, device=dev).normal_(0.0, 1e-3, generator=gen) * 2.0 ** 16).half()
        for _ in range(3):
            opt.step()
        torch.cuda.synchronize()
        st = opt.store
        big = sum(st.master[i].numel() for i in st.k2_tensors)
        _progress(f"gpt2-small ragged: K2 over {len(st.k2_tensors)} tensors / {big} elements, K3 over the other "
                  f"{len(st.params) - len(st.k2_tensors)} / {st.numel - big} elements "
                  f"({(st.small_table or st._table).nchunks} chunks)")
        del opt, ps
    torch.cuda.empty_cache()
    _calibration_copy(dev)
    _progress("profile-kernels done")
    return 0


def profile_kernels(n: int, dev) -> int:
    """Three dispatches of each kernel of the step and of the traffic probe,
    plus the copy calibration (_calibration_copy)."""
    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, FlatStep, ScalerConfig
    hyper = AdamWHyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    master, exp_avg, exp_avg_sq, p16, grad = make_inputs(n, 2, dev)
    fs = FlatStep(n, dev, hyper, ScalerConfig(mode="none"))
    hc, sc = hyper.to_c(), fs.scaler.to_c()
    for _ in range(3):
        fs.steps_issued += 1
        fs.bc.ensure(fs.steps_issued)
        ops.unscale_norm(grad, fs.state, fs.partials, fs.nparts)
        ops.finalize(fs.partials, fs.nparts, fs.state, sc, hc, fs.bc.table, fs.bc.length, fs.scalars)
        ops.adamw_flat(master, exp_avg, exp_avg_sq, p16, grad, fs.scalars)
    for _ in range(3):
        ops.traffic_probe_flat(master, exp_avg, exp_avg_sq, p16, grad)
    torch.cuda.synchronize()
    del master, exp_avg, exp_avg_sq, p16, grad
    _calibration_copy(dev)
    _progress("profile-kernels done")
    return 0


def _progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def master_and_grad(n: int, seed: int, device):
    """configs[2]'s values: fp32 master N(0, 0.02^2) and bf16 grads
    N(0, 5e-4^2), drawn chunk by chunk from one seeded generator on the GPU."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    master = torch.empty(n, dtype=torch.float32, device=device)
    grad = torch.empty(n, dtype=torch.bfloat16, device=device)
    chunk = 1 << 27
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        master[s:e].normal_(0.0, 0.02, generator=gen)
        grad[s:e].copy_(torch.empty(e - s, dtype=torch.float32, device=device).normal_(0.0, 5e-4, generator=gen))
    return master, grad


def make_inputs(n: int, seed: int, device):
    import torch
    master, grad = master_and_grad(n, seed, device)
    exp_avg = torch.zeros(n, dtype=torch.float32, device=device)
    exp_avg_sq = torch.zeros(n, dtype=torch.float32, device=device)
    p16 = master.to(torch.bfloat16)
    return master, exp_avg, exp_avg_sq, p16, grad


def llama_ragged_shapes():
    """32 x (4096^2 x4, 4096x14336 x2, 14336x4096, 4096 x2) +
    128256x4096 -- 289 tensors, 8,310,226,944 elements."""
    shapes = []
    for _ in range(32):
        shapes += [(4096, 4096)] * 4 + [(4096, 14336)] * 2 + [(14336, 4096)] + [(4096,)] * 2
    shapes.append((128256, 4096))
    return shapes


def gpt2_small_shapes():
    """wte, wpe, 12 x {ln_1 w,b; c_attn w,b; attn c_proj w,b;
    ln_2 w,b; c_fc w,b; mlp c_proj w,b}, ln_f w,b -- 148 tensors,
    124,439,808 elements."""
    d, ff, vocab, ctx = 768, 3072, 50257, 1024
    shapes = [(vocab, d), (ctx, d)]
    for _ in range(12):
        shapes += [(d,), (d,), (d, 3 * d), (3 * d,), (d, d), (d,), (d,), (d,), (d, ff), (ff,), (ff, d), (d,)]
    return shapes + [(d,), (d,)]


def mlp_shapes():
    """784x1024, 1024, 1024x1024, 1024, 1024x10, 10 -- 1,863,690 elements."""
    return [(1024, 784), (1024,), (1024, 1024), (1024,), (10, 1024), (10,)]


def measure_dropin(dev, gpt2: bool, steps: int, warmup: int,
                   modes=("flat_eager", "flat_graph", "ragged_eager")) -> dict:
    """configs[0] (mlp) or configs[1] (gpt2-small) through the drop-in
    optimizer classes, Python host code included: the flat form eager (one C
    call per step), the flat form replayed as a HIP graph, and the ragged
    form (K3). These partitions are small enough that launch and host
    overhead matter, which is what the modes show. fp16 params and grads;
    gpt2-small: grads N(0, 1e-3^2) x 2^16, dynamic scaler (init 2^16, window
    1000), clip 1.0; mlp: grads N(0, 0.01^2) x 2^16, static scale 2^16, no
    clip. Events around `steps` calls of opt.step() after `warmup`."""
    import math

    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    shapes = gpt2_small_shapes() if gpt2 else mlp_shapes()
    n = sum(math.prod(s) for s in shapes)
    if gpt2:
        sc = ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=1, min_scale=1.0)
        sigma, clip, kw = 1e-3, 1.0, dict(lr=6e-4, weight_decay=0.01)
    else:
        sc = ScalerConfig(mode="static", init_scale=2.0 ** 16)
        sigma, clip, kw = 0.01, 0.0, dict(lr=1e-4, weight_decay=0.01)
    every = {"flat_eager": (AdamWOptimizer, {}), "flat_graph": (AdamWOptimizer, {"graph": True}),
             "ragged_eager": (MultiTensorAdamWOptimizer, {})}
    out = {}
    for name in modes:
        cls, extra = every[name]
        gen = torch.Generator(device=dev)
        gen.manual_seed(1)
        ps = [torch.nn.Parameter(torch.empty(s, device=dev).normal_(0.0, 0.02, generator=gen)) for s in shapes]
        opt = cls(ps, max_grad_norm=clip, param_dtype=torch.float16, loss_scaler=sc, device=dev, **kw, **extra)
        for p in opt.dsx_params:
            g = torch.empty(p.shape, device=dev).normal_(0.0, sigma, generator=gen).mul_(2.0 ** 16)
            if p.grad is None:
                p.grad = g.to(torch.float16)
            else:
                p.grad.copy_(g)
        for _ in range(warmup):
            opt.step()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        s0.record()
        for _ in range(steps):
            opt.step()
        t_issue = time.perf_counter() - t0
        s1.record()
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / steps
        st = opt.read_state()
        out[name] = {"ms_per_step": round(ms, 4), "gparam_per_s": round(n / ms / 1e6, 3),
                     "host_issue_us_per_step": round(t_issue / steps * 1e6, 1),
                     "achieved_tbps": round(30 * n / ms / 1e9, 4), "state_error": st.error,
                     "last_skip": st.last_skip}
        _progress(f"{'configs[1]' if gpt2 else 'configs[0]'} {name}: {out[name]}")
        del opt, ps
        torch.cuda.empty_cache()
    return {"workload": "gpt2-small fp16 (BASELINE configs[1])" if gpt2 else "mlp fp16 (BASELINE configs[0])",
            "storage": "f32 state / fp16 grads+params", "tensors": len(shapes), "numel": n, "steps": steps,
            "warmup": warmup, "modes": out}


def measure_dropin_headline(dev, n: int, steps: int, warmup: int, headline_ms: float | None,
                            fold_restore: int = 3 << 23) -> dict:
    """configs[2] through the drop-in classes: the same shard (one parameter
    of n elements, the headline's seed and values, bf16 params and grads,
    no loss scale, lr 3e-4, betas (0.9, 0.95), eps 1e-8, wd 0.1, clip 1.0)
    stepped by AdamWOptimizer.step() -- what the reference's stages call,
    Src/zero/stage2.py:609-612 -- and then by ZeROOptimizer.step(), the
    engine's step (Src/zero/optimizer.py:212-274), on the same optimizer.
    Both issue one dsx_zero_step_plan call per step: K1, then K0's finalize
    folded into the first of K2's parts, then the other parts (the headline
    times the three bare entry points instead). Between them, on the same
    buffers, AdamWOptimizer.step() with the fold switched off
    (dsx_set_tuning_fold(0): K1, K0 and the 15 K2 parts as three entry
    points, the headline's form), so that the path's cost is told apart
    from where this run's allocations landed; the fold bound is then set
    back to fold_restore. Last, the headline's own three entry points
    (unscale_norm, finalize, adamw_flat, with their own state and records)
    over the optimizer's flat buffers: the headline's calls on this run's
    allocations. Events around `steps` steps after `warmup` on the stream
    the kernels run on. headline_ms (None when no headline ran in this
    process) gives each form's over_headline_ms."""
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    from distributedspeed_amd.zero import ZeROOptimizer
    master, grad = master_and_grad(n, 2, dev)
    p = torch.nn.Parameter(master)
    del master
    opt = AdamWOptimizer([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0,
                         param_dtype=torch.bfloat16, loss_scaler=ScalerConfig(mode="none"), device=dev)
    p.grad.copy_(grad)  # the parameter's view of the flat grad buffer
    del grad
    zo = ZeROOptimizer(opt, config={"stage": 2, "gradient_accumulation_steps": 1})
    torch.cuda.synchronize()
    out = {}

    def fold(v):
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(v))

    f = opt.flat
    hyper = AdamWHyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    hc, scc = hyper.to_c(), ScalerConfig(mode="none").to_c()
    bc = BiasCorrectionTable(dev, hyper.beta1, hyper.beta2)
    bc.ensure(2 * (warmup + steps))
    st3, rec3 = ops.new_state(dev, 1.0, 1), ops.new_scalars(dev)
    np3 = ops.suggest_partials(n)
    parts3 = torch.zeros(np3, dtype=torch.float64, device=dev)
    g3 = f.grad[:n]
    bufs3 = (f.master[:n], f.exp_avg[:n], f.exp_avg_sq[:n], f.param16[:n])

    def entry_points():
        ops.unscale_norm(g3, st3, parts3, np3)
        ops.finalize(parts3, np3, st3, scc, hc, bc.table, bc.length, rec3)
        ops.adamw_flat(*bufs3, g3, rec3)

    for name, fn, fold_to in (("AdamWOptimizer.step", opt.step, fold_restore),
                              ("AdamWOptimizer.step, fold off (three launches)", opt.step, 0),
                              ("ZeROOptimizer.step", zo.step, fold_restore),
                              ("the headline's three entry points on these buffers", entry_points, fold_restore)):
        fold(fold_to)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        s0.record()
        for _ in range(steps):
            fn()
        t_issue = time.perf_counter() - t0
        s1.record()
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / steps
        st = opt.read_state() if fn is not entry_points else ops.read_state(st3)
        out[name] = {"ms_per_step": round(ms, 4), "gparam_per_s": round(n / ms / 1e6, 3),
                     "pct_of_8tbps_end_to_end": round(100 * 30 * n / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                     "over_headline_ms": round(ms / headline_ms, 4) if headline_ms else None,
                     "host_issue_us_per_step": round(t_issue / steps * 1e6, 1),
                     "state_error": st.error, "last_skip": st.last_skip}
        _progress(f"configs[2] drop-in {name}: {out[name]}")
    fold(fold_restore)
    out["ZeROOptimizer.step"]["current_step"] = zo.current_step
    del zo, opt, p, f, g3, bufs3, parts3
    torch.cuda.empty_cache()
    return {"workload": "llama3-8b zero2 one-rank shard (BASELINE configs[2]) through the drop-in classes",
            "storage": "f32 state / bf16 grads+params", "numel": n, "steps": steps, "warmup": warmup,
            "path": "dsx_zero_step_plan: " + ("K1, then K2 with K0's finalize folded into every block"
                                               if n <= 3 << 23 else
                                               f"K1, then K2 in {k2_parts(n, None)} parts with K0's finalize "
                                               "folded into the first"),
            "headline_ms_per_step": round(headline_ms, 4) if headline_ms else None, "modes": out}


def bench_dropin_headline(a, dev) -> int:
    """configs[2] through the drop-in classes as its own line, in a fresh
    process (measure_dropin_headline with no headline run before it, so its
    buffers are the process's first large allocations)."""
    n = int(a.numel)
    r = measure_dropin_headline(dev, n, a.steps, a.warmup, None, 3 << 23 if a.fold is None else a.fold)
    modes = r["modes"]
    bad = [k for k, v in modes.items() if v["state_error"] or v["last_skip"]]
    if bad:
        print(json.dumps({"error": f"{bad}: state error or skipped step"}))
        return 1
    m = modes["AdamWOptimizer.step"]
    print(json.dumps({
        "metric": "drop-in optimizer step Gparam/s (configs[2], fresh process)", "value": m["gparam_per_s"],
        "unit": "Gparam/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": m["ms_per_step"],
        "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": r["workload"], "storage": r["storage"], "numel": n, "path": r["path"]},
        "modes": modes}), flush=True)
    return 0


def bench_dropin(a, dev) -> int:
    """configs[0] or configs[1] as its own line (measure_dropin, every mode)."""
    r = measure_dropin(dev, a.workload == "gpt2-small", a.steps, a.warmup)
    modes = r["modes"]
    bad = [k for k, v in modes.items() if v["state_error"] or v["last_skip"]]
    if bad:
        print(json.dumps({"error": f"{bad}: state error or skipped step"}))
        return 1
    best = max(modes, key=lambda k: modes[k]["gparam_per_s"])
    print(json.dumps({
        "metric": f"drop-in optimizer step Gparam/s ({'configs[1]' if 'gpt2' in r['workload'] else 'configs[0]'})",
        "value": modes[best]["gparam_per_s"], "unit": "Gparam/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": modes[best]["ms_per_step"], "higher_is_better": True,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": r["workload"], "storage": r["storage"], "tensors": r["tensors"], "numel": r["numel"],
                   "best_mode": best},
        "modes": modes}), flush=True)
    return 0


def bench_mlp_train(a, dev) -> int:
    """configs[0]'s MLP (784-1024-1024-10, fp16 params, static scale 2^16,
    AdamW lr 1e-4 wd 0.01) trained on synthetic batches of 32: one whole
    iteration -- zero_grad, forward, cross-entropy * loss scale, backward,
    fused step -- run eagerly, and captured once into a HIP graph
    (AdamWOptimizer(capturable=True)) and replayed with prepare_step()."""
    import torch
    import torch.nn.functional as F
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer

    def make():
        torch.manual_seed(0)
        model = torch.nn.Sequential(torch.nn.Linear(784, 1024), torch.nn.ReLU(), torch.nn.Linear(1024, 1024),
                                    torch.nn.ReLU(), torch.nn.Linear(1024, 10)).to(dev)
        opt = AdamWOptimizer(model.parameters(), lr=1e-4, weight_decay=0.01, param_dtype=torch.float16,
                             loss_scaler=ScalerConfig(mode="static", init_scale=2.0 ** 16), device=dev, capturable=True)
        return model, opt

    def iteration(model, opt, x, y):
        opt.zero_grad()
        loss = F.cross_entropy(model(x).float(), y)
        (loss * opt.loss_scale_tensor()).backward()
        opt.step()

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    x = torch.randn(32, 784, device=dev, generator=gen).half()
    y = torch.randint(0, 10, (32,), device=dev, generator=gen)
    res = {}
    model, opt = make()
    for _ in range(a.warmup):
        iteration(model, opt, x, y)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(a.steps):
        iteration(model, opt, x, y)
    e1.record()
    torch.cuda.synchronize()
    res["eager_us_per_iter"] = round(e0.elapsed_time(e1) / a.steps * 1e3, 2)
    model, opt = make()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(max(3, a.warmup)):
            iteration(model, opt, x, y)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        iteration(model, opt, x, y)
    for _ in range(a.warmup):
        opt.prepare_step()
        graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(a.steps):
        opt.prepare_step()
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    res["graph_us_per_iter"] = round(e0.elapsed_time(e1) / a.steps * 1e3, 2)
    st = opt.read_state()
    if st.error or st.last_skip:
        print(json.dumps({"error": f"state error={st.error} skip={st.last_skip}"}))
        return 1
    print(json.dumps({
        "metric": "training iteration (fwd + bwd + fused step) us, configs[0] MLP, batch 32",
        "value": res["graph_us_per_iter"], "unit": "us/iter", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "higher_is_better": False, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "mlp training iteration (BASELINE configs[0] model)", "batch": 32,
                   "storage": "fp16 params/grads, f32 state"},
        "modes": res, "speedup_graph_over_eager": round(res["eager_us_per_iter"] / res["graph_us_per_iter"], 3)}),
        flush=True)
    return 0


def bench_ffn_train(a, dev) -> int:
    """The grad-producer side of the step: a 0.94e9-parameter stack of bf16
    feed-forward blocks (8 x [4096 -> 14336, ReLU, 14336 -> 4096], no bias)
    trained on 16 synthetic tokens, so weight traffic sets the pace. One
    iteration = zero_grad, forward, loss, backward, fused step (clip 1.0).
    Both storage forms, each with both ways of handling the grads, alternated
    in blocks of a.steps iterations: zero_grad(set_to_none=True) -- the flat
    form copies autograd's grads into its buffer in a post-accumulate hook,
    taking the norm's partials on the way so the step skips K1 (4 B/elt
    instead of 10), the ragged form reads them where autograd put them
    (0 B/elt instead of 8) -- and zero_grad(set_to_none=False) -- grads
    zeroed in place, then autograd accumulates into them."""
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    d, ff, blocks, tokens = 4096, 14336, 8, 16

    def make(cls):
        torch.manual_seed(0)
        layers = []
        for _ in range(blocks):
            layers += [torch.nn.Linear(d, ff, bias=False), torch.nn.ReLU(), torch.nn.Linear(ff, d, bias=False)]
        model = torch.nn.Sequential(*layers).to(dev, torch.bfloat16)
        for mod in model:
            if isinstance(mod, torch.nn.Linear):
                torch.nn.init.normal_(mod.weight, 0.0, 0.02)
        opt = cls(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, max_grad_norm=1.0,
                  param_dtype=torch.bfloat16, device=dev)
        return model, opt

    forms = {"flat": make(AdamWOptimizer), "ragged": make(MultiTensorAdamWOptimizer)}
    n_params = sum(p.numel() for p in forms["flat"][0].parameters())
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    x = torch.randn(tokens, d, device=dev, generator=gen).to(torch.bfloat16)

    def iteration(form, set_to_none):
        model, opt = forms[form]
        opt.zero_grad(set_to_none=set_to_none)
        model(x).float().pow(2).mean().backward()
        opt.step()

    modes = [(f, m) for f in ("flat", "ragged") for m in (True, False)]
    for mode in modes:
        for _ in range(max(1, a.warmup)):
            iteration(*mode)
    torch.cuda.synchronize()
    times = {mode: [] for mode in modes}
    for _ in range(3):
        for mode in modes:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(a.steps):
                iteration(*mode)
            e1.record()
            torch.cuda.synchronize()
            times[mode].append(e0.elapsed_time(e1) / a.steps)
    for _, opt in forms.values():
        st = opt.read_state()
        if st.error or st.last_skip:
            print(json.dumps({"error": f"state error={st.error} skip={st.last_skip}"}))
            return 1
    med = {mode: sorted(v)[1] for mode, v in times.items()}
    name = {True: "set_to_none", False: "in_place"}
    print(json.dumps({
        "metric": "training iteration ms, 0.94e9-parameter bf16 feed-forward stack, 16 tokens",
        "value": round(med[("flat", True)], 4), "unit": "ms/iter", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "higher_is_better": False, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "ffn stack training iteration (grad-producer side of the step)", "params": n_params,
                   "blocks": blocks, "d_model": d, "d_ff": ff, "tokens": tokens,
                   "storage": "bf16 params/grads, f32 state"},
        "ms_per_iter": {f"{f}_{name[m]}": round(t, 4) for (f, m), t in med.items()},
        "runs_ms": {f"{f}_{name[m]}": [round(t, 4) for t in v] for (f, m), v in times.items()},
        "saving_ms": {f: round(med[(f, False)] - med[(f, True)], 4) for f in ("flat", "ragged")},
        "saving_ms_at_8tbs": {"flat (6 B/param: copy instead of zero + add, no K1 pass)":
                              round(6 * n_params / 8e12 * 1e3, 4),
                              "ragged (8 B/param)": round(8 * n_params / 8e12 * 1e3, 4)},
    }), flush=True)
    return 0


def ragged_list(dev, sizes):
    """configs[3]'s tensors (seed 4): fp32 master N(0, 0.02^2), m = v = 0,
    fp16 params, fp16 grads N(0, 1e-3^2) x 2^16; and their chunk table."""
    import torch
    from distributedspeed_amd import ops
    _progress(f"configs[3]: allocating {len(sizes)} tensors / {sum(sizes)} elements")
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    ts = []
    for k in sizes:
        p = torch.empty(k, device=dev).normal_(0.0, 0.02, generator=gen)
        g = torch.empty(k, device=dev).normal_(0.0, 1e-3, generator=gen).mul_(2.0 ** 16).to(torch.float16)
        ts.append((p, torch.zeros(k, device=dev), torch.zeros(k, device=dev), p.to(torch.float16), g))
    return ts, ops.ChunkTable(*[[t[j] for t in ts] for j in range(5)])


def measure_ragged(dev, steps: int, warmup: int) -> dict:
    """configs[3] through K3: fp16 grads N(0, 1e-3^2) x 2^16, dynamic scaler
    (init 2^16, window 1000, hysteresis 2, min 1), AdamW defaults, clip 1.0.
    One step = K1 over the chunk table, K0, K3 (three launches). Returns the
    figures (ms/step, Gparam/s, TB/s at 30 B/elt, K1 and K3 times)."""
    import math

    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    sizes = [math.prod(s) for s in llama_ragged_shapes()]
    n = sum(sizes)
    ts, table = ragged_list(dev, sizes)
    hyper = AdamWHyper(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=1.0)
    scfg = ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=2, min_scale=1.0)
    bc = BiasCorrectionTable(dev, hyper.beta1, hyper.beta2, capacity=warmup + 3 * steps + 8)
    st = ops.new_state(dev, scfg.init_scale, scfg.hysteresis)
    nparts = ops.suggest_partials(n)
    parts = torch.zeros(nparts, dtype=torch.float64, device=dev)
    out = ops.new_scalars(dev)
    hc, sc = hyper.to_c(), scfg.to_c()

    def step(ev=None):
        if ev:
            ev[0].record()
        ops.unscale_norm_multi(table, st, parts, nparts)
        if ev:
            ev[1].record()
        ops.finalize(parts, nparts, st, sc, hc, bc.table, bc.length, out)
        if ev:
            ev[2].record()
        ops.adamw_multi(table, out)
        if ev:
            ev[3].record()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(steps):
        step()
    s1.record()
    torch.cuda.synchronize()
    ms = s0.elapsed_time(s1) / steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    k1 = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    k3 = sum(e[2].elapsed_time(e[3]) for e in evs) / steps
    s = ops.read_state(st)
    res = {"workload": "llama ragged list (BASELINE configs[3]), K1 / K0 / K3 over the chunk table",
           "storage": "f32 state / fp16 grads+params", "tensors": len(sizes), "numel": n, "chunks": table.nchunks,
           "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4), "gparam_per_s": round(n / ms / 1e6, 3),
           "achieved_tbps_end_to_end": round(30 * n / ms / 1e9, 4),
           "pct_of_8tbps_end_to_end": round(100 * 30 * n / ms / 1e6 / HBM_PEAK_GBS, 2),
           "kernels_ms": {"k1_unscale_norm_multi": round(k1, 4), "k2_adamw_multi": round(k3, 4)},
           "k3_gbs": round(28 * n / k3 / 1e6, 1), "k3_frac_of_8tbs": round(28 * n / k3 / 1e6 / HBM_PEAK_GBS, 4),
           "state_error": s.error, "last_skip": s.last_skip}
    del ts, table
    torch.cuda.empty_cache()
    return res


def bench_ragged(a, dev) -> int:
    """configs[3] as its own line (measure_ragged)."""
    r = measure_ragged(dev, a.steps, a.warmup)
    if r["state_error"] or r["last_skip"]:
        print(json.dumps({"error": f"state error={r['state_error']} skip={r['last_skip']}"}))
        return 1
    print(json.dumps({
        "metric": "ragged multi-tensor ZeRO step Gparam/s (configs[3], K3)", "value": r["gparam_per_s"],
        "unit": "Gparam/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": r["ms_per_step"],
        "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {k: r[k] for k in ("workload", "storage", "tensors", "numel", "chunks")},
        "achieved_tbps_end_to_end": r["achieved_tbps_end_to_end"], "kernels_ms": r["kernels_ms"],
        "k3_gbs": r["k3_gbs"], "k3_frac_of_8tbs": r["k3_frac_of_8tbs"],
    }), flush=True)
    return 0


def link_ceiling(dev) -> dict:
    """Plain pinned-host <-> HBM copy bandwidth (offload.measure_link),
    measured in a fresh child process (the only child bench.py starts;
    subprocess.run waits for it to exit). Either process may see the two
    directions run one at a time (the both-ways figure then halves): on
    these boxes that has happened both in a process that had freed large
    device buffers and in the fresh child. So measure_offload also measures
    the link on the step's own streams (offload.measure_streamer_link) and
    takes the larger both-ways figure as the ceiling. Falls back to this
    process."""
    import subprocess
    root = os.path.dirname(os.path.abspath(__file__))
    code = ("import json, sys, torch; sys.path.insert(0, %r); from distributedspeed_amd.offload import measure_link; "
            "print(json.dumps(measure_link(torch.device('cuda', %d))))" % (root, dev.index or 0))
    try:
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
        if r.returncode == 0:
            out = json.loads(r.stdout.strip().splitlines()[-1])
            out["measured_in"] = "a fresh process"
            return out
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    from distributedspeed_amd.offload import measure_link
    out = measure_link(dev)
    out["measured_in"] = "this process"
    return out


def measure_offload(dev, full: int, budget_gib: float, steps: int) -> dict:
    """Llama-3-70B ZeRO-3 one-rank shard, 8,819,213,312 elements,
    fp32 master/m/v in pinned host memory (105.8 GB) streamed through HBM in
    64 Mi-element chunks, bf16 grads N(0, 3e-4^2) and params in HBM; AdamW lr
    1.5e-4, betas (0.9, 0.95), wd 0.1. Bound by the host link (12 B/elt each
    way), so the figure of merit is link GB/s against the measured link
    ceiling, not HBM TB/s."""
    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    from distributedspeed_amd.offload import HostStateStreamer, pinned_zeros
    chunk = 64 << 20
    _progress("measuring the host link")
    link = link_ceiling(dev)
    # The machine caps GPU-visible pinned host memory (one hipHostMalloc above
    # 32 GiB fails, ~64 GiB in total, and the runtime needs part of it), so the
    # shard is sized to a pinned budget: 12 B of state per element.
    budget = int(budget_gib * 2**30)
    n = min(full, budget // 12 // chunk * chunk)
    _progress(f"link {link}; allocating {n} of {full} elements of pinned state ({12 * n / 2**30:.1f} GiB)")
    grad = torch.empty(n, dtype=torch.bfloat16, device=dev)
    p16 = torch.empty(n, dtype=torch.bfloat16, device=dev)
    master, m, v = pinned_zeros(n), pinned_zeros(n), pinned_zeros(n)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    tmp = torch.empty(chunk, device=dev)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        tmp[:e - s].normal_(0.0, 0.02, generator=gen)
        master[s:e].copy_(tmp[:e - s])
        p16[s:e].copy_(tmp[:e - s])
        grad[s:e].copy_(tmp[:e - s].normal_(0.0, 3e-4, generator=gen))
        if (s // chunk) % 16 == 0:
            _progress(f"filled {e}/{n}")
    del tmp
    torch.cuda.synchronize()
    hyper = AdamWHyper(lr=1.5e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    scfg = ScalerConfig(mode="none")
    bc = BiasCorrectionTable(dev, hyper.beta1, hyper.beta2)
    st = ops.new_state(dev, 1.0, 1)
    nparts = ops.suggest_partials(n)
    parts = torch.zeros(nparts, dtype=torch.float64, device=dev)
    out = ops.new_scalars(dev)
    streamer = HostStateStreamer(dev, chunk)

    def step():
        ops.unscale_norm(grad, st, parts, nparts)
        ops.finalize(parts, nparts, st, scfg.to_c(), hyper.to_c(), bc.table, bc.length, out)
        streamer.run((master, m, v), p16, grad, [(0, n, out)])

    _progress("warmup step")
    step()
    torch.cuda.synchronize()
    times = []
    for i in range(steps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        _progress(f"step {i + 1}: {times[-1]:.3f} s")
    s = ops.read_state(st)
    # The link measured right after the timed steps, in this process, on the
    # step's own copy streams and pinned buffers; the ceiling is the larger
    # of this and the fresh process's figure.
    _progress("measuring the host link on the step's own streams")
    from distributedspeed_amd.offload import measure_streamer_link
    # the copy-only schedule is also started as a step starts it, behind K1
    # (which reads the grads and writes the partials, and changes no state)
    link_here = measure_streamer_link(streamer, (master, m, v), pipeline_passes=3,
                                      lead=lambda: ops.unscale_norm(grad, st, parts, nparts))
    link_here["measured_in"] = "this process, the step's copy streams and pinned buffers, after the timed steps"
    ceiling = max(link["both_each_way"], link_here["both_each_way"])
    sec = sorted(times)[len(times) // 2]
    each_way = 12 * n / sec / 1e9
    del grad, p16, master, m, v, streamer
    torch.cuda.empty_cache()
    return {"workload": "llama3-70b zero3 one-rank shard, state offloaded (BASELINE configs[4])",
            "storage": "f32 state (pinned host) / bf16 grads+params", "numel": n, "chunk_elems": chunk,
            "steps": steps, "warmup": 1, "ms_per_step": round(sec * 1e3, 1),
            "gparam_per_s": round(n / sec / 1e9, 4), "link_gbs_each_way": round(each_way, 2),
            "link_ceiling_gbs": {k: (round(x, 2) if isinstance(x, float) else x) for k, x in link.items()},
            "link_ceiling_in_process_gbs": {k: (round(x, 2) if isinstance(x, float) else x)
                                            for k, x in link_here.items()},
            "bidirectional_ceiling_gbs": round(ceiling, 2),
            "frac_of_measured_bidirectional_link": round(each_way / ceiling, 4),
            "frac_of_one_direction_link": round(each_way / max(min(link["h2d"], link["d2h"]),
                                                               min(link_here["h2d"], link_here["d2h"])), 4),
            "reduced_from_numel": full if n != full else None,
            "reduction_reason": (f"pinned budget {budget_gib} GiB: this machine caps GPU-visible pinned host "
                                 "memory (no single hipHostMalloc above 32 GiB, ~64 GiB in total); the full shard "
                                 "needs 105.8 GB; the step is host-link-bound, so Gparam/s does not depend on the size")
            if n != full else None,
            "state_t": s.t, "skipped": s.last_skip, "state_error": s.error}


def bench_offload(a, dev) -> int:
    """configs[4] as its own line (measure_offload)."""
    full = int(a.numel) if a.numel != HEADLINE_NUMEL else 8_819_213_312
    r = measure_offload(dev, full, a.pinned_budget_gib, max(1, min(a.steps, 3)))
    print(json.dumps({
        "metric": "offloaded ZeRO step (configs[4]): Gparam/s and host-link GB/s each way",
        "value": r["gparam_per_s"], "unit": "Gparam/s", "n_gpus": 1, "steps": r["steps"], "warmup": 1,
        "ms_per_step": r["ms_per_step"], "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {k: r[k] for k in ("workload", "storage", "numel", "chunk_elems")},
        **{k: r[k] for k in ("link_gbs_each_way", "link_ceiling_gbs", "link_ceiling_in_process_gbs",
                             "bidirectional_ceiling_gbs", "frac_of_measured_bidirectional_link",
                             "frac_of_one_direction_link", "reduced_from_numel", "reduction_reason", "state_t")},
        "skipped": r["skipped"],
    }), flush=True)
    return 0


def torch_gpu_reference(master, grad16, hyper, ours_ms: float, steps: int = 5) -> dict:
    """The reference's update at world size 1 as torch runs it on this GPU,
    over the same shard: fp32 grads from the 16-bit ones, the norm with a
    host read (Src/zero/utils.py:150), g *= max/(norm + 1e-6) when above the
    threshold (utils.py:211-214), torch.optim.AdamW.step
    (Src/zero/stage2.py:609-612; default dispatch = multi-tensor, and fused),
    then the bf16 cast of the updated fp32 params. Timed with events around
    `steps` steps after two warm-up steps; context only (not the headline)."""
    import torch
    _progress("torch reference path on the GPU")
    p = torch.nn.Parameter(master.detach().clone())
    p16 = torch.empty_like(p, dtype=torch.bfloat16)
    res = {"what": "fp32 grad copy + norm (.item()) + clip + torch.optim.AdamW.step + bf16 cast, same shard"}
    for name, kw in (("foreach", {}), ("fused", {"fused": True})):
        opt = torch.optim.AdamW([p], lr=hyper.lr, betas=(hyper.beta1, hyper.beta2), eps=hyper.eps,
                                weight_decay=hyper.weight_decay, **kw)

        def step():
            g = grad16.float()
            norm = float(torch.linalg.vector_norm(g).item())
            if norm > hyper.max_grad_norm:
                g.mul_(hyper.max_grad_norm / (norm + 1e-6))
            p.grad = g
            opt.step()
            p.grad = None
            p16.copy_(p)

        for _ in range(2):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        res[f"{name}_ms_per_step"] = round(ms, 3)
        res[f"speedup_of_fused_step_over_{name}"] = round(ms / ours_ms, 2)
        del opt
    del p, p16
    torch.cuda.empty_cache()
    return res


def host_info() -> dict:
    """The host the CPU baseline runs on: core counts and the CPU model
    (lscpu's "Model name", else /proc/cpuinfo's)."""
    import subprocess
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model}


def cpu_threads() -> tuple[int, str]:
    """Threads for the CPU baseline and why: the job's CPU share. A GPU box
    of this pool grants one GPU's job 16 host threads and says so in
    OMP_NUM_THREADS; elsewhere the CPUs this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env), "OMP_NUM_THREADS (the host threads granted to this job)"
    return len(os.sched_getaffinity(0)), "the CPUs in this process's affinity set"


def cpu_baseline(master_h, grad_h, hyper, steps: int = 5, shard: int | None = None,
                 gpu_norm: float | None = None) -> dict | None:
    """The reference's CPU route timed on this host's cores, on the same
    inputs as the GPU run (copied to host memory). The reference has no CPU
    Adam kernel: its cpu_offload route parks the state on the host and steps
    it with torch.optim.AdamW (Src/zero/stage1.py:376-398, 482-498;
    Src/zero/stage2.py:432-454, 563-582), whose default CPU dispatch is the
    single-tensor loop. One step, as the reference's ZeRO step orders it:
    fp32 grads from the bf16 ones (no loss scale for bf16, so no unscale),
    the norm as compute_norm takes it (t.norm(dtype=float32).item() ** 2
    summed, then ** 0.5: Src/zero/utils.py:146-154), g *= max / (norm + 1e-6)
    when above the threshold (utils.py:211-214), AdamW.step() on one flat fp32
    master, then the bf16 cast of the result. 1 warm-up step, then the median
    of `steps`. Beside it: torch's fused CPU AdamW (the fastest CPU route
    torch has) and this repository's C oracle (a port of the whole step on
    OpenMP threads).

    The norms: torch's CPU fp32 reductions (the reference's compute_norm
    and torch.linalg.vector_norm alike) lose accuracy as the sample grows
    (about 19% low over 1.0e9 bf16 values), so the record holds each norm
    beside an fp64 one (the oracle's compensated block sums) with its
    relative error, and the GPU step's norm (gpu_norm: the step's
    DsxStepScalars.norm over the same values) with its error too."""
    if master_h is None:
        return None
    import numpy as np
    import torch
    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    from oracle import oracle as O

    ns = master_h.numel()
    threads, why = cpu_threads()
    torch.set_num_threads(threads)
    mx = hyper.max_grad_norm

    def torch_route(nsteps, **kw):
        param = torch.nn.Parameter(master_h.clone())
        opt = torch.optim.AdamW([param], lr=hyper.lr, betas=(hyper.beta1, hyper.beta2), eps=hyper.eps,
                                weight_decay=hyper.weight_decay, **kw)
        p16 = torch.empty(ns, dtype=torch.bfloat16)
        times, norm = [], None
        for _ in range(1 + nsteps):
            t0 = time.perf_counter()
            g = grad_h.float()
            norm = (g.norm(dtype=torch.float32).item() ** 2) ** 0.5
            if norm > mx:
                g.mul_(mx / (norm + 1e-6))
            param.grad = g
            opt.step()
            param.grad = None
            p16.copy_(param.detach())
            times.append(time.perf_counter() - t0)
        del opt, param, p16
        return sorted(times[1:])[len(times[1:]) // 2], norm, len(times) - 1

    g16 = grad_h.view(torch.int16).numpy().view(np.uint16)
    _progress("cpu baseline: the fp64 norm")
    norm64 = O.sumsq_parallel(g16, O.BF16, 1.0, 1024) ** 0.5

    _progress(f"cpu baseline: torch.optim.AdamW(foreach=False) on {ns} elements, {threads} threads")
    t_ref, norm_ref, n_ref = torch_route(steps, foreach=False)
    norm_vec = float(torch.linalg.vector_norm(grad_h.float()).item())

    def rel(x):
        return None if x is None or not norm64 else abs(x - norm64) / norm64

    def clip_of(x):
        return mx / (x + 1e-6) if x is not None and mx > 0 and x > mx else 1.0
    _progress("cpu baseline: torch.optim.AdamW(fused=True)")
    t_fused, _, n_fused = torch_route(max(2, steps // 2), fused=True)

    _progress("cpu baseline: the C oracle port")
    p = master_h.numpy().copy()
    m = np.zeros(ns, np.float32)
    v = np.zeros(ns, np.float32)
    p16 = np.empty(ns, np.uint16)
    h = O.Hyper(lr=hyper.lr, beta1=hyper.beta1, beta2=hyper.beta2, eps=hyper.eps,
                weight_decay=hyper.weight_decay, max_grad_norm=mx)
    times = []
    for t in range(1, 2 + steps):
        t0 = time.perf_counter()
        ss = O.sumsq_parallel(g16, O.BF16, 1.0, 1024)
        coef = O.clip_coef(ss ** 0.5, h.max_grad_norm, h.clip_eps)
        O.adamw(p, m, v, p16, O.BF16, g16, O.BF16, O.step_scalars(h, t, 1.0, coef))
        times.append(time.perf_counter() - t0)
    t_port = sorted(times[1:])[len(times[1:]) // 2]
    del p, m, v, p16
    return {
        "value": round(ns / t_ref / 1e9, 4),
        "unit": "Gparam/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "what": "the reference's CPU route (cpu_offload -> torch.optim.AdamW, default single-tensor dispatch, "
                "foreach=False) on CPU fp32: bf16 -> fp32 grads, norm as compute_norm takes it, clip, "
                "AdamW.step(), bf16 cast",
        "sample": (f"{ns} elements: " + ("the whole shard" if shard in (None, ns) else f"the first {ns} of the "
                                         f"{shard}-element shard") +
                   f", the GPU run's own inputs (bf16 grads N(0,5e-4^2), fp32 master N(0,0.02^2)) copied to host "
                   f"memory; median of {n_ref} steps after 1 warm-up"),
        "ms_per_step": round(t_ref * 1e3, 1),
        "threads": {"used": torch.get_num_threads(), "why": why},
        "host": host_info(),
        "norm": {
            "fp64": {"value": norm64, "what": "sqrt of the fp64 sum of squares (the oracle's 1024 compensated "
                                              "block sums, added in block order)"},
            "gpu_step": {"value": gpu_norm, "rel_err_vs_fp64": rel(gpu_norm),
                         "what": "the GPU step's norm over the same values (DsxStepScalars.norm: K1's fp64 "
                                 "partials reduced by the finalize)"},
            "reference_style": {"value": norm_ref, "rel_err_vs_fp64": rel(norm_ref),
                                "what": "the reference's compute_norm on the CPU: t.norm(dtype=float32).item() "
                                        "** 2, then ** 0.5 (Src/zero/utils.py:146-154), torch's fp32 reduction"},
            "torch_linalg_vector_norm": {"value": norm_vec, "rel_err_vs_fp64": rel(norm_vec),
                                         "what": "torch.linalg.vector_norm on the CPU fp32 grads"},
            "clip_coef": {"reference_cpu_route": clip_of(norm_ref), "from_fp64_norm": clip_of(norm64),
                          "gpu_step": clip_of(gpu_norm) if gpu_norm is not None else None},
            "note": "the timed reference CPU route clips by max_norm / (its own norm + 1e-6); torch's CPU fp32 "
                    "reduction undercounts large samples, so that coefficient differs from the fp64 one by the "
                    "norm's relative error; the GPU step's norm is held to 1e-6 of fp64",
        },
        "torch_adamw_cpu_fused": {"value": round(ns / t_fused / 1e9, 4), "unit": "Gparam/s",
                                  "ms_per_step": round(t_fused * 1e3, 1), "steps": n_fused,
                                  "what": "torch.optim.AdamW(fused=True) on CPU, same sample and step"},
        "port": {"value": round(ns / t_port / 1e9, 4), "unit": "Gparam/s", "ms_per_step": round(t_port * 1e3, 1),
                 "threads": int(O.lib().dsxo_num_threads()), "steps": len(times) - 1,
                 "what": "this repository's C oracle on OpenMP threads: the norm as 1024 compensated block sums, "
                         "clip, the AdamW loop (vectorised), bf16 cast"},
    }


def main() -> int:
    a = _args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1",
                          "gpus_requested": a.gpus}))
        return 2
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, FlatStep, ScalerConfig

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lib = _lib.load()
    if a.tuning:
        vals = [int(x) for x in a.tuning.split(",")]
        _lib.call("dsx_set_tuning", *vals[:4])
        if len(vals) > 4:
            _lib.call("dsx_set_tuning_k2", vals[4], vals[5] if len(vals) > 5 else -1)
    if a.tuning_multi:
        _lib.call("dsx_set_tuning_multi", *[int(x) for x in a.tuning_multi.split(",")])
    if a.k2_chunk is not None:
        _lib.call("dsx_set_tuning_k2_chunk", a.k2_chunk)
    if a.fold is not None:
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(a.fold))
    n = int(a.numel)
    if a.profile_kernels:
        if a.workload in ("llama-ragged", "gpt2-small"):
            return profile_ragged(a.workload, dev)
        return profile_kernels(n, dev)
    if a.workload == "llama-ragged":
        return bench_ragged(a, dev)
    if a.workload == "llama70b-offload":
        return bench_offload(a, dev)
    if a.workload in ("gpt2-small", "mlp"):
        return bench_dropin(a, dev)
    if a.workload == "mlp-train":
        return bench_mlp_train(a, dev)
    if a.workload == "ffn-train":
        return bench_ffn_train(a, dev)
    if a.workload == "llama8b-dropin":
        return bench_dropin_headline(a, dev)
    hyper = AdamWHyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    _progress(f"generating {n} elements")
    master, exp_avg, exp_avg_sq, p16, grad = make_inputs(n, 2, dev)
    fs = FlatStep(n, dev, hyper, ScalerConfig(mode="none"))
    # the CPU baseline's inputs: the same values, copied to host memory now
    ns = n if a.cpu_sample < 0 else min(a.cpu_sample, n)
    cpu_in = (master[:ns].cpu(), grad[:ns].cpu()) if ns > 0 else (None, None)
    torch.cuda.synchronize()

    # Warm-up and timed steps: K1 -> K0 -> K2 through the library's three
    # entry points (the one-call step, FlatStep.step, folds K0 into K2's
    # first part instead), so that every step issues the same kernels and a
    # kernel trace of this run holds K1, K0 and 15 K2 parts per step.
    hc, sc = hyper.to_c(), fs.scaler.to_c()
    fs.bc.ensure(fs.steps_issued + a.warmup + a.steps)
    _progress(f"warmup {a.warmup}")
    for _ in range(a.warmup):
        fs.steps_issued += 1
        ops.unscale_norm(grad, fs.state, fs.partials, fs.nparts)
        ops.finalize(fs.partials, fs.nparts, fs.state, sc, hc, fs.bc.table, fs.bc.length, fs.scalars)
        ops.adamw_flat(master, exp_avg, exp_avg_sq, p16, grad, fs.scalars)
    torch.cuda.synchronize()

    # The timed region: K steps, with an event before and after every launch
    # on the stream the kernels run on (torch's current stream). ms_per_step
    # spans the whole region; the per-kernel averages (roofline.achieved)
    # come from the same launches.
    _progress(f"timing {a.steps} steps")
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(a.steps)]
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        fs.steps_issued += 1
        e = ev[i]
        e[0].record()
        ops.unscale_norm(grad, fs.state, fs.partials, fs.nparts)
        e[1].record()
        ops.finalize(fs.partials, fs.nparts, fs.state, sc, hc, fs.bc.table, fs.bc.length, fs.scalars)
        e[2].record()
        ops.adamw_flat(master, exp_avg, exp_avg_sq, p16, grad, fs.scalars)
        e[3].record()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev[0][0].elapsed_time(stop) / a.steps
    k1_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / a.steps
    k0_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / a.steps
    k2_ms = sum(e[2].elapsed_time(e[3]) for e in ev) / a.steps
    st = fs.read_state()
    scal = fs.read_scalars()
    if st.error or scal.skip:
        print(json.dumps({"error": f"step state error={st.error} skip={scal.skip}"}))
        return 1

    # The GPU step's norm over the CPU baseline's sample: the step's own
    # record when the sample is the whole shard (every timed step saw the
    # same grads), else K1 over the sample's grads, its fp64 partials summed
    # here.
    gpu_norm = None
    if ns == n:
        gpu_norm = float(scal.norm)
    elif ns > 0:
        import math
        np_s = ops.suggest_partials(ns)
        ps = torch.zeros(np_s, dtype=torch.float64, device=dev)
        ops.unscale_norm(grad[:ns], fs.state, ps, np_s)
        gpu_norm = math.sqrt(math.fsum(ps.cpu().tolist()))
        del ps

    gparams = n / (ms_step * 1e-3) / 1e9
    e2e_gbs = (K1_BYTES + K2_BYTES) * n / (ms_step * 1e-3) / 1e9
    k2_gbs = K2_BYTES * n / (k2_ms * 1e-3) / 1e9
    k1_gbs = K1_BYTES * n / (k1_ms * 1e-3) / 1e9

    # K2's own access pattern without its math: the same bytes in the same
    # launch shape on the same buffers (dsx_traffic_probe_flat), timed after
    # the measured steps. K2 at or above it means the math costs nothing and
    # the memory system sets the bound.
    _progress("traffic probe")
    pev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(a.steps)]
    for i in range(a.steps):
        pev[i][0].record()
        ops.traffic_probe_flat(master, exp_avg, exp_avg_sq, p16, grad)
        pev[i][1].record()
    torch.cuda.synchronize()
    probe_ms = sum(e[0].elapsed_time(e[1]) for e in pev) / a.steps
    probe_gbs = K2_BYTES * n / (probe_ms * 1e-3) / 1e9

    traffic = None
    if os.path.exists(a.traffic):
        try:
            with open(a.traffic) as f:
                tj = json.load(f)
            if int(tj.get("numel", -1)) == n:
                traffic = tj.get("k2_hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    # The other BASELINE configs in the same run, after the headline's timed
    # region. configs[4] goes first, while nothing large has been returned to
    # the HIP runtime: on these boxes, once a process has freed a large
    # allocation (hipFree of 16 GB), its simultaneous host-to-device and
    # device-to-host copies run one at a time (28.8 instead of 48.6 GB/s each
    # way), which would halve that line.
    secondary = {}

    def run_secondary(key, fn):
        try:
            secondary[key] = fn()
        except Exception as e:  # a secondary line must not cost the headline
            secondary[key] = {"error": f"{type(e).__name__}: {e}"}
            torch.cuda.empty_cache()

    if a.secondary:
        run_secondary("configs[4]", lambda: measure_offload(dev, 8_819_213_312, a.pinned_budget_gib, 3))
    torch_gpu = torch_gpu_reference(master, grad, hyper, ms_step) if a.torch_gpu else None
    if a.secondary:
        del master, exp_avg, exp_avg_sq, p16, grad, fs
        torch.cuda.empty_cache()
        run_secondary("configs[2]", lambda: measure_dropin_headline(
            dev, n, a.steps, a.warmup, ms_step, 3 << 23 if a.fold is None else a.fold))
        run_secondary("configs[0]", lambda: measure_dropin(dev, False, max(a.steps, 200), max(a.warmup, 20),
                                                           modes=("flat_eager",)))
        run_secondary("configs[1]", lambda: measure_dropin(dev, True, a.steps, a.warmup, modes=("flat_eager",)))
        run_secondary("configs[3]", lambda: measure_ragged(dev, max(3, min(a.steps, 10)), min(a.warmup, 3)))
        secondary = {k: secondary[k] for k in sorted(secondary)}
    else:
        secondary = None
    cpu = cpu_baseline(*cpu_in, hyper, a.cpu_steps, shard=n, gpu_norm=gpu_norm)

    out = {
        "metric": "AdamW step Gparam/s + achieved HBM TB/s (% of 8 TB/s), 1.0B-elt bf16 shard",
        "value": round(gparams, 3),
        "unit": "Gparam/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch generator on the GPU)",
        "config": {"workload": "llama3-8b zero2 one-rank shard (BASELINE configs[2])", "numel": n,
                   "grad_dtype": "bf16", "param_dtype": "bf16", "state_dtype": "f32", "lr": hyper.lr, "betas": [hyper.beta1, hyper.beta2],
                   "eps": hyper.eps, "weight_decay": hyper.weight_decay, "max_grad_norm": hyper.max_grad_norm,
                   "parallelism": "dp1 (one rank's ZeRO shard)"},
        "achieved_tbps_end_to_end": round(e2e_gbs / 1000, 4),
        "pct_of_8tbps_end_to_end": round(100 * e2e_gbs / HBM_PEAK_GBS, 2),
        "kernels_ms": {"k1_unscale_norm": round(k1_ms, 4), "k0_finalize": round(k0_ms, 4),
                       "k2_adamw_flat": round(k2_ms, 4)},
        "k1_gbs": round(k1_gbs, 1),
        "k2_traffic_probe": {"what": "K2's loads, stores and launch shape without the AdamW math, same buffers",
                             "ms": round(probe_ms, 4), "gbs": round(probe_gbs, 1),
                             "k2_over_probe": round(k2_gbs / probe_gbs, 4)},
        "roofline": {"bound": "hbm", "achieved": round(k2_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k2_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k2_adamw_flat", "algorithmic_bytes_per_launch": K2_BYTES * n,
                     "dispatches_per_launch": k2_parts(n, a.k2_chunk)},
        "cpu_baseline": cpu,
        "gpu_over_cpu_reference_route": round(gparams / cpu["value"], 1) if cpu else None,
        "secondary_configs": secondary,
        "torch_gpu_reference_path": torch_gpu,
        "wall_s_timed": round(wall, 3),
        "torch": torch.__version__, "hip": torch.version.hip,
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
