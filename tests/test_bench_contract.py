"""bench.py keeps its output contract: one JSON line with the metric, value,
unit, roofline and cpu_baseline objects (GPU run on a small shard), and a
refusal with a message for more than one GPU (CPU)."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, timeout):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, capture_output=True, text=True,
                          timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run(["--gpus", "2"], 120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"] and line["gpus_requested"] == 2


@pytest.mark.gpu
def test_bench_line_contract(gpu):
    r = _run(["--numel", str((1 << 22) + 3), "--steps", "3", "--warmup", "1", "--cpu-sample", str(1 << 20),
              "--cpu-steps", "1", "--torch-gpu", "1", "--secondary", "0"], 300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [x for x in r.stdout.splitlines() if x.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1 and d["value"] > 0
    assert "workload" in d["config"]
    rf = d["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    cb = d["cpu_baseline"]
    assert cb["kind"] == "reference" and cb["cores"] >= 1 and cb["value"] > 0 and cb["sample"]
    assert cb["threads"]["used"] == cb["cores"] and cb["host"]["os_cpu_count"] >= 1
    assert cb["port"]["value"] > 0 and cb["torch_adamw_cpu_fused"]["value"] > 0
    nm = cb["norm"]
    # the GPU step's norm against the fp64 one, at the north star's 1e-6
    assert nm["gpu_step"]["value"] > 0 and nm["gpu_step"]["rel_err_vs_fp64"] <= 1e-6, nm
    for k in ("reference_style", "torch_linalg_vector_norm"):
        assert nm[k]["rel_err_vs_fp64"] == abs(nm[k]["value"] - nm["fp64"]["value"]) / nm["fp64"]["value"], k
    assert d["secondary_configs"] is None
    assert d["torch_gpu_reference_path"]["foreach_ms_per_step"] > 0
    tp = d["k2_traffic_probe"]
    assert tp["ms"] > 0 and abs(tp["k2_over_probe"] - rf["achieved"] / tp["gbs"]) < 1e-3


def test_cpu_baseline_host_facts():
    """The CPU baseline states its thread count and why, and the host's core
    counts and CPU model, without a GPU."""
    sys.path.insert(0, ROOT)
    import bench
    info = bench.host_info()
    assert info["os_cpu_count"] >= 1 and info["affinity_cpus"] >= 1
    assert info["cpu_model"]
    n, why = bench.cpu_threads()
    assert n >= 1 and why


@pytest.mark.gpu
@pytest.mark.parametrize("workload", ["mlp", "mlp-train", "gpt2-small", "ffn-train", "llama8b-dropin"])
def test_secondary_workloads_print_one_line(gpu, workload):
    """The secondary workloads (configs[0] and [1] through the drop-in
    classes, the training iterations) still run and print one JSON line with
    a positive value. configs[3] and [4] run inside the headline line's
    secondary_configs."""
    print(f"[gpu-test] bench.py --workload {workload}", file=sys.stderr, flush=True)
    extra = ["--numel", str((1 << 25) + 5)] if workload == "llama8b-dropin" else []
    r = _run(["--workload", workload, "--steps", "3", "--warmup", "1"] + extra, 280)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [x for x in r.stdout.splitlines() if x.startswith("{")]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])
    assert d["metric"] and d["unit"] and d["value"] > 0, d
    assert isinstance(d["config"], dict) and d["config"], d


@pytest.mark.gpu
def test_dropin_headline_measurement(gpu):
    """The headline line's secondary_configs["configs[2]"] entry: the
    drop-in AdamWOptimizer.step() and ZeROOptimizer.step() on one shard (here
    2^25 + 5 elements: above the fold bound, so the fold-first form), every
    step clean (also with the fold switched off), and ZeROOptimizer's
    current_step counting every form's steps."""
    sys.path.insert(0, ROOT)
    import bench
    n = (1 << 25) + 5
    print(f"[gpu-test] measure_dropin_headline n={n}", file=sys.stderr, flush=True)
    r = bench.measure_dropin_headline(gpu, n, 3, 1, 1.0)
    assert r["numel"] == n and "folded into the first" in r["path"]
    assert set(r["modes"]) == {"AdamWOptimizer.step", "AdamWOptimizer.step, fold off (three launches)",
                               "ZeROOptimizer.step", "the headline's three entry points on these buffers"}
    for k, m in r["modes"].items():
        assert m["ms_per_step"] > 0 and m["state_error"] == 0 and m["last_skip"] == 0, m
        assert m["over_headline_ms"] > 0
    assert r["modes"]["ZeROOptimizer.step"]["current_step"] == 12
    # whatever happened above, the tests after this one (same process) see
    # the library's default fold bound
    from distributedspeed_amd import _lib
    assert _lib.load().dsx_set_tuning_fold(3 << 23) == 0
