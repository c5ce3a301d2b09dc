"""Host-side logic without a GPU: ds_config parsing (mirroring
Src/config.py's defaults, deep merge, unknown-key TypeError, validation
messages and env overrides), the flat partition layout (on CPU tensors), the
bias-correction table, the loss-scaler mapping and the ops' argument checks."""
from __future__ import annotations

import json
import math

import numpy as np
import pytest
import torch

from distributedspeed_amd import config as C
from distributedspeed_amd.flat import ALIGN, FlatPartition
from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig


# ---- ds_config ------------------------------------------------------------------------

def test_defaults_match_reference():
    c = C.DistributedSpeedConfig()
    assert c.max_grad_norm == 1.0 and c.gradient_accumulation_steps == 1 and c.train_batch_size == 32
    assert c.adamw_params() == {"lr": 1e-4, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.01}
    assert (c.fp16.loss_scale, c.fp16.initial_scale_power, c.fp16.loss_scale_window, c.fp16.hysteresis,
            c.fp16.min_loss_scale) == (0.0, 16, 1000, 2, 1.0)
    assert c.zero_optimization.stage == 0 and c.zero_optimization.contiguous_gradients
    assert c.precision == "fp32" and c.loss_scaler() == {"mode": "none", "init_scale": 1.0}


def test_deep_merge_keeps_unspecified_params():
    c = C.DistributedSpeedConfig({"optimizer": {"params": {"lr": 3e-4, "betas": [0.9, 0.95]}}})
    assert c.adamw_params() == {"lr": 3e-4, "betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.01}


def test_loss_scaler_mapping():
    dyn = C.DistributedSpeedConfig(C.fp16_config()).loss_scaler()
    assert dyn == {"mode": "dynamic", "init_scale": 65536.0, "window": 1000, "hysteresis": 2, "min_scale": 1.0}
    static = C.DistributedSpeedConfig({"fp16": {"enabled": True, "loss_scale": 128}}).loss_scaler()
    assert static == {"mode": "static", "init_scale": 128.0}
    assert C.DistributedSpeedConfig(C.bf16_config()).loss_scaler()["mode"] == "none"
    ScalerConfig(**dyn).validate()


def test_unknown_key_raises_typeerror_like_the_reference():
    with pytest.raises(TypeError):
        C.DistributedSpeedConfig({"fp16": {"enabled": True, "not_a_key": 1}})
    with pytest.raises(TypeError):
        C.DistributedSpeedConfig({"zero_optimization": {"stagee": 2}})


@pytest.mark.parametrize("cfg,msg", [
    ({"fp16": {"enabled": True}, "bf16": {"enabled": True}}, "Cannot enable both FP16 and BF16"),
    ({"zero_optimization": {"stage": 4}}, "ZeRO stage must be 0, 1, 2, or 3"),
    ({"gradient_accumulation_steps": 0}, "gradient_accumulation_steps must be positive"),
    ({"fp16": {"enabled": True, "hysteresis": 0}}, "hysteresis must be >= 1"),
])
def test_validation_messages(cfg, msg):
    with pytest.raises(ValueError, match="Configuration validation failed") as e:
        C.DistributedSpeedConfig(cfg)
    assert msg in str(e.value)


def test_gradient_clipping_alias_and_extra_sections():
    c = C.DistributedSpeedConfig({"gradient_clipping": 0.5, "scheduler": {"type": "WarmupLR"}})
    assert c.max_grad_norm == 0.5 and c.extra["scheduler"] == {"type": "WarmupLR"}
    assert c["scheduler"]["type"] == "WarmupLR" and c.get("nope", 7) == 7


def test_env_overrides(monkeypatch):
    monkeypatch.setenv("DISTRIBUTEDSPEED_LEARNING_RATE", "0.005")
    monkeypatch.setenv("DISTRIBUTEDSPEED_BF16_ENABLED", "true")
    monkeypatch.setenv("DISTRIBUTEDSPEED_ZERO_STAGE", "2")
    c = C.DistributedSpeedConfig({})
    assert c.adamw_params()["lr"] == 0.005 and c.bf16.enabled and c.zero_optimization.stage == 2


def test_load_config_json_and_yaml(tmp_path):
    d = {"fp16": {"enabled": True}, "gradient_accumulation_steps": 4}
    j = tmp_path / "ds.json"
    j.write_text(json.dumps(d))
    y = tmp_path / "ds.yaml"
    y.write_text("fp16:\n  enabled: true\ngradient_accumulation_steps: 4\n")
    for path in (j, y):
        c = C.load_config(str(path))
        assert c.fp16.enabled and c.gradient_accumulation_steps == 4
    with pytest.raises(FileNotFoundError):
        C.load_config(str(tmp_path / "missing.json"))
    with pytest.raises(TypeError):
        C.load_config(3.0)


# ---- flat partition (CPU tensors) ----------------------------------------------------------

def _params(shapes, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.nn.Parameter(torch.randn(s, generator=g) * 0.02) for s in shapes]


def test_flat_layout_alignment_and_views():
    ps = _params([(3, 5), (7,), (4, 4), (1,), (10,)])
    orig = [p.detach().clone() for p in ps]
    fp = FlatPartition([ps[:2], ps[2:]], torch.device("cpu"), torch.bfloat16)
    offs = [s.offset for s in fp.slots]
    assert offs == [0, 16, 24, 40, 48] and all(o % ALIGN == 0 for o in offs)
    assert fp.group_ranges == [(0, 24), (24, 64)] and fp.numel == 64
    for s, p, o in zip(fp.slots, ps, orig):
        assert p.dtype == torch.bfloat16 and p.grad is not None and p.grad.dtype == torch.bfloat16
        assert torch.equal(fp.master[s.offset:s.offset + s.numel], o.reshape(-1))  # master keeps fp32 values
        assert torch.equal(p.detach().float().reshape(-1), o.reshape(-1).to(torch.bfloat16).float())
        assert p.data_ptr() == fp.param16[s.offset:].data_ptr()
    # padding is zero everywhere
    used = torch.zeros(fp.numel, dtype=torch.bool)
    for s in fp.slots:
        used[s.offset:s.offset + s.numel] = True
    assert (fp.master[~used] == 0).all() and (fp.param16[~used].float() == 0).all()


def test_autograd_accumulates_into_flat_views_on_cpu():
    lin = torch.nn.Linear(6, 3)
    fp = FlatPartition([list(lin.parameters())], torch.device("cpu"), None)
    x = torch.randn(4, 6)
    lin(x).sum().backward()
    lin(x).sum().backward()  # accumulates in place
    for s, p in zip(fp.slots, fp.params):
        assert p.grad.data_ptr() == fp.grad[s.offset:].data_ptr()
    assert torch.allclose(fp.grad[fp.slots[1].offset:fp.slots[1].offset + 3], torch.full((3,), 8.0))
    fp.check_grads_bound()
    # a replaced grad is copied back into the flat buffer and the view restored
    lin.bias.grad = torch.ones(3)
    fp.check_grads_bound()
    assert torch.equal(fp.grad[fp.slots[1].offset:fp.slots[1].offset + 3], torch.ones(3))
    assert lin.bias.grad.data_ptr() == fp.grad[fp.slots[1].offset:].data_ptr()
    lin.weight.grad = None
    fp.check_grads_bound()
    assert lin.weight.grad is not None and float(lin.weight.grad.abs().sum()) == 0.0
    fp.zero_grad()
    assert float(fp.grad.abs().sum()) == 0.0


def test_grads_handed_over_after_set_to_none():
    """zero_grad(set_to_none=True): autograd's own grads are copied into the
    flat views by the post-accumulate hook and p.grad is the view again, so a
    second micro-batch accumulates in the flat buffer; a parameter without a
    grad is zeroed in its view before the step; set_to_none=False zeroes the
    buffer in place and keeps the views bound. Values equal plain autograd."""
    import gc
    torch.manual_seed(0)
    lin, unused = torch.nn.Linear(6, 3), torch.nn.Parameter(torch.ones(5))
    ref = torch.nn.Linear(6, 3)
    ref.load_state_dict(lin.state_dict())
    fp = FlatPartition([list(lin.parameters()) + [unused]], torch.device("cpu"), None)
    views = [fp.grad[s.offset:s.offset + s.numel] for s in fp.slots]
    fp.grad.fill_(7.0)  # stale values from an earlier step
    fp.zero_grad(set_to_none=True)
    assert all(p.grad is None for p in fp.params)
    xs = [torch.randn(4, 6) for _ in range(2)]
    for x in xs:
        lin(x).pow(2).sum().backward()
        ref(x).pow(2).sum().backward()
    for p, v in zip(list(lin.parameters()), views):
        assert p.grad.data_ptr() == v.data_ptr()
    assert torch.equal(lin.weight.grad, ref.weight.grad) and torch.equal(lin.bias.grad, ref.bias.grad)
    assert unused.grad is None
    fp.check_grads_bound()
    assert unused.grad.data_ptr() == views[2].data_ptr() and float(unused.grad.abs().sum()) == 0.0
    fp.zero_grad(set_to_none=False)
    assert float(fp.grad.abs().sum()) == 0.0
    assert all(p.grad.data_ptr() == v.data_ptr() for p, v in zip(fp.params, views))
    lin(xs[0]).sum().backward()
    assert torch.equal(lin.bias.grad, torch.full((3,), 4.0))
    # the partition can go while the parameters live on: its hooks go with it
    del fp
    gc.collect()
    lin.weight.grad = None
    lin(xs[0]).sum().backward()
    assert lin.weight.grad is not None and lin.weight.grad.data_ptr() != views[0].data_ptr()


def test_flat_rejects_duplicates_and_bad_dtype():
    p = torch.nn.Parameter(torch.zeros(3))
    with pytest.raises(ValueError):
        FlatPartition([[p], [p]], torch.device("cpu"), None)
    with pytest.raises(ValueError):
        FlatPartition([[torch.nn.Parameter(torch.zeros(3))]], torch.device("cpu"), torch.float64)
    with pytest.raises(ValueError):
        FlatPartition([[torch.nn.Parameter(torch.zeros(3))]], torch.device("cpu"), None, offload=True)


def test_storage_bytes_of_both_forms():
    """What get_memory_info / estimate_memory_usage report: 16-bit params and
    grads plus 12 bytes of fp32 state per element (padding included in the
    flat form); with fp32 training the params are the master (no extra bytes)."""
    from distributedspeed_amd.ragged import RaggedParams
    fp = FlatPartition([_params([(3, 5), (7,)])], torch.device("cpu"), torch.bfloat16)
    assert fp.numel == 24
    assert fp.storage_bytes() == {"params": 48, "grads": 48, "optimizer_states": 288,
                                  "optimizer_states_on_host": False}
    f32 = FlatPartition([_params([(9,)])], torch.device("cpu"), None)
    assert f32.numel == 16
    assert f32.storage_bytes() == {"params": 0, "grads": 64, "optimizer_states": 192,
                                   "optimizer_states_on_host": False}
    rp = RaggedParams([_params([(3, 5), (7,)])], torch.device("cpu"), torch.float16)
    assert rp.storage_bytes() == {"params": 44, "grads": 44, "optimizer_states": 264,
                                  "optimizer_states_on_host": False}
    r32 = RaggedParams([_params([(9,)])], torch.device("cpu"), None)
    assert r32.storage_bytes()["params"] == 0 and r32.storage_bytes()["grads"] == 36


def test_layout_manifest_names():
    lin = torch.nn.Linear(2, 2)
    names = {id(p): n for n, p in lin.named_parameters()}
    fp = FlatPartition([list(lin.parameters())], torch.device("cpu"), None, names)
    assert [e["name"] for e in fp.layout()] == ["weight", "bias"]


# ---- bias corrections, hyper-parameters ----------------------------------------------------

def test_bias_correction_table_matches_torch_expression():
    tab = BiasCorrectionTable(torch.device("cpu"), 0.9, 0.95, capacity=8)
    assert tab.length >= 8
    t = tab.table.numpy()
    for step in range(1, 9):
        assert t[2 * (step - 1)] == 1 - 0.9 ** float(step)
        assert t[2 * (step - 1) + 1] == (1 - 0.95 ** float(step)) ** 0.5
    tab.ensure(5000)
    assert tab.length >= 5000 and tab.table.numel() == 2 * tab.length
    tab.ensure(10, betas=(0.8, 0.99))
    assert tab.table[0].item() == 1 - 0.8 ** 1.0


def test_hyper_validation_messages():
    for kw, msg in ((dict(lr=-1), "Invalid learning rate"), (dict(eps=-1), "Invalid epsilon"),
                    (dict(beta1=1.0), "index 0"), (dict(beta2=-0.1), "index 1"),
                    (dict(weight_decay=-1), "Invalid weight_decay"), (dict(max_grad_norm=math.nan), "NaN")):
        with pytest.raises(ValueError, match=msg):
            AdamWHyper(**kw).validate()
    c = AdamWHyper(lr=1e-3).to_c()
    assert (c.lr, c.beta1, c.clip_eps) == (1e-3, 0.9, 1e-6)


def test_ops_reject_cpu_tensors():
    from distributedspeed_amd import ops
    t = torch.zeros(16)
    with pytest.raises(ValueError, match="GPU"):
        ops.adamw_flat(t, t, t, None, t, torch.zeros(64, dtype=torch.uint8))
    with pytest.raises(TypeError):
        ops.grad_code(torch.int32)
    assert ops.grad_code(torch.float32) == 0 and ops.dtype_code(torch.bfloat16) == 2


def test_initialize_fails_loudly_without_gpu():
    import distributedspeed_amd as ds
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="GPU"):
        ds.initialize(torch.nn.Linear(2, 2), {})


def test_oracle_not_imported_by_product():
    import pathlib
    root = pathlib.Path(__file__).resolve().parents[1] / "distributedspeed_amd"
    for f in root.rglob("*.py"):
        text = f.read_text()
        assert "import oracle" not in text and "from oracle" not in text, f
    assert np.__version__  # numpy is the only array dependency of the oracle


def test_pack_groups_checks_on_host():
    """The graph path's per-step group block: table checks in Python (the
    hyper-parameters are checked by dsx_groups_upload, tested with the ABI)."""
    from distributedspeed_amd import ops
    t = torch.zeros(8, dtype=torch.float64)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.pack_groups([AdamWHyper().to_c()], [t], [0], 4)
    with pytest.raises(ValueError, match="groups"):
        ops.pack_groups([], [], [], 4)
    assert ops.GROUPS_BYTES == 1112


# ---- ragged parameter store (CPU tensors) ------------------------------------------------

def test_ragged_store_keeps_storage_and_masters():
    from distributedspeed_amd.ragged import RaggedParams
    ps = _params([(3, 5), (7,), (4, 4)])
    orig = [p.detach().clone() for p in ps]
    rp = RaggedParams([ps[:1], ps[1:]], torch.device("cpu"), torch.float16, {id(ps[1]): "b"})
    assert rp.numel == 15 + 7 + 16 and rp.group_of == [0, 1, 1]
    for p, o, m in zip(ps, orig, rp.master):
        assert p.dtype == torch.float16 and m.dtype == torch.float32
        assert torch.equal(m, o) and torch.equal(p.detach(), o.to(torch.float16))
        assert p.data_ptr() != m.data_ptr()
    assert [e["name"] for e in rp.layout()] == ["param0", "b", "param2"]
    assert [e["offset"] for e in rp.layout()] == [0, 15, 22]
    rp.ensure_grads()
    assert all(p.grad is not None and p.grad.dtype == torch.float16 and float(p.grad.abs().sum()) == 0 for p in ps)
    ps[0].grad = torch.ones(5, 3, dtype=torch.float16).t()  # a strided grad is made contiguous
    rp.ensure_grads()
    assert ps[0].grad.is_contiguous() and float(ps[0].grad.sum()) == 15
    rp.zero_grad()
    assert float(ps[0].grad.abs().sum()) == 0
    rp.master[1].fill_(1.0 + 2 ** -12)  # rounds to 1.0 in fp16 (RNE, tie to even)
    rp.refresh_params16()
    assert torch.equal(ps[1].detach(), torch.ones(7, dtype=torch.float16))


def test_ragged_store_fp32_master_is_the_param():
    from distributedspeed_amd.ragged import RaggedParams
    ps = _params([(5,), (2, 3)])
    rp = RaggedParams([ps], torch.device("cpu"), None)
    for p, m in zip(ps, rp.master):
        assert p.data_ptr() == m.data_ptr() and p.dtype == torch.float32
    with pytest.raises(ValueError):
        RaggedParams([[torch.nn.Parameter(torch.zeros(2, dtype=torch.float16))]], torch.device("cpu"), None)


def test_ragged_chunk_size_fills_the_gpu():
    from distributedspeed_amd.ragged import auto_chunk_elems
    assert auto_chunk_elems(8_310_226_944) == 65536 and auto_chunk_elems(124_439_808) == 16384
    # small lists: one trip of K3's slot loop per chunk while the list fits in 1024 chunks of 2048
    assert auto_chunk_elems(1_863_690) == 2048 and auto_chunk_elems(10) == 2048
    assert auto_chunk_elems(1024 * 2048) == 2048 and auto_chunk_elems(1024 * 2048 + 1) == 4096
    assert auto_chunk_elems(3_900_000) == 4096
    for n in (1 << 20, 1 << 22, 1 << 27, 3 << 28):
        c = auto_chunk_elems(n)
        assert c % 8 == 0 and (c == 4096 or n // c >= 4096 or (c == 2048 and -(-n // c) <= 1024))


def test_optimizer_step_hooks_still_run():
    """AdamWOptimizer.step skips torch's per-call wrapper when nothing needs
    it, and runs the step pre / post hooks (and the closure) when they are
    registered; checked without a GPU by replacing the fused step."""
    from distributedspeed_amd.optimizers import AdamWOptimizer
    assert getattr(AdamWOptimizer.step, "hooked", False)  # torch does not wrap it again
    calls = []

    class Probe(AdamWOptimizer):
        def __init__(self):  # no device state: only the protocol is exercised
            torch.optim.Optimizer.__init__(self, [torch.nn.Parameter(torch.zeros(2))], dict(lr=1.0))

        def step_fused(self):
            calls.append("fused")

    o = Probe()
    assert o.step() is None and calls == ["fused"]
    h1 = o.register_step_pre_hook(lambda opt, a, k: calls.append("pre"))
    from torch.optim.optimizer import register_optimizer_step_post_hook
    h2 = register_optimizer_step_post_hook(lambda opt, a, k: calls.append("post"))
    try:
        assert o.step(lambda: 3.0) == 3.0
        assert calls == ["fused", "pre", "fused", "post"]
    finally:
        h1.remove()
        h2.remove()
    o.step()
    assert calls[-1] == "fused" and calls.count("pre") == 1


def test_more_than_sixteen_groups_is_refused():
    from distributedspeed_amd.optimizers import AdamWOptimizer
    groups = [{"params": [torch.nn.Parameter(torch.zeros(2))]} for _ in range(17)]
    with pytest.raises(ValueError, match="at most 16 parameter groups"):
        AdamWOptimizer(groups)


def test_k2_parts_per_call_follow_the_library_rule():
    """K2 above the part size runs as ceil(n / part) consecutive dispatches
    (dsx_set_tuning_k2_chunk; default 2^26): the rocprof summary and bench.py
    turn per-dispatch figures into per-call ones with the same count."""
    import os
    import sys
    from distributedspeed_amd.rocprof_summary import parts_per_call
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    from bench import k2_parts
    assert parts_per_call(1003782656, 1 << 26) == 15 == k2_parts(1003782656, None)
    assert parts_per_call(124439808, 1 << 26) == 2 == k2_parts(124439808, None)
    assert parts_per_call(1 << 26, 1 << 26) == 1 == k2_parts(1 << 26, None)
    assert parts_per_call(1003782656, 0) == 1 == k2_parts(1003782656, 0)
    assert parts_per_call(1003782656, 1 << 25) == 30 == k2_parts(1003782656, 1 << 25)



def test_rocprof_call_spans_include_the_gaps_between_parts(tmp_path):
    """call_spans (the summary's events-like figure for a parted kernel)
    takes each call as `parts` consecutive dispatches of that kernel and
    measures from the first start to the last end, gaps included; other
    kernels in between do not count."""
    import csv
    from distributedspeed_amd.rocprof_summary import call_spans
    k2 = "void (anonymous namespace)::k2_adamw_flat<2, 2, 2, true, false>(float*)"
    k1 = "void (anonymous namespace)::k1_unscale_norm<2, 4, true>(void const*, long)"
    rows, t = [], 0
    for call in range(3):
        rows.append({"Start_Timestamp": t, "End_Timestamp": t + 50, "Kernel_Name": k1})
        t += 60
        for part in range(3):  # 100 ns each, 7 ns gaps
            rows.append({"Start_Timestamp": t, "End_Timestamp": t + 100, "Kernel_Name": k2})
            t += 107
    with open(tmp_path / "t_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Start_Timestamp", "End_Timestamp", "Kernel_Name"])
        w.writeheader()
        w.writerows(rows[::-1])  # the trace need not be in time order
    assert call_spans(str(tmp_path), "k2_adamw_flat", 3) == [314, 314, 314]
    assert call_spans(str(tmp_path), "k2_adamw_flat", 1) == [100] * 9


def test_rocprof_step_chains_count_the_parts_after_a_folded_first_part(tmp_path):
    """The kernel-trace summary (rocprof_summary --chains) groups a step's
    launches by form: K1 then the folded K2 and the plain K2 parts after it
    (one step above the fold's bound), K1/K0/K2 parts (three launches), K1
    over a chunk table then the folded K3; K2's column sums every part."""
    import csv
    from distributedspeed_amd.rocprof_summary import step_chains
    names = {"k1": "void (anonymous namespace)::k1_unscale_norm<2, 4, true>(void const*, long)",
             "k2f": "void (anonymous namespace)::k2_adamw_fold<2, 2, 2, true, DsxGroupsDev>(float*)",
             "k2": "void (anonymous namespace)::k2_adamw_flat<2, 2, 2, true, false>(float*)",
             "k0": "(anonymous namespace)::k0_finalize(double const*, int)",
             "k1m": "void (anonymous namespace)::k1_unscale_norm_multi<1, true>(DsxTensorRef const*)",
             "k3f": "void (anonymous namespace)::k3_adamw_fold<1, 1, true>(DsxTensorRef const*)"}
    rows, t = [], 0

    def launch(k, dur):
        nonlocal t
        rows.append({"Start_Timestamp": t, "End_Timestamp": t + dur, "Kernel_Name": names[k]})
        t += dur + 1000

    for _ in range(4):  # folded first part + two plain parts
        launch("k1", 10_000), launch("k2f", 100_000), launch("k2", 90_000), launch("k2", 80_000)
    for _ in range(3):  # three launches, two parts
        launch("k1", 10_000), launch("k0", 4_000), launch("k2", 95_000), launch("k2", 95_000)
    for _ in range(3):  # ragged, folded
        launch("k1m", 5_000), launch("k3f", 9_000)
    with open(tmp_path / "t_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Start_Timestamp", "End_Timestamp", "Kernel_Name"])
        w.writeheader()
        w.writerows(rows)
    res = step_chains(str(tmp_path))
    two = res["flat, eager, two launches (K0 folded into K2)"]
    assert two["steps"] == 4 and two["kernels_us"]["k2_adamw_fold"] == 270.0
    assert two["kernels_us"]["k1_unscale_norm"] == 10.0 and two["kernel_busy_us"] == 280.0
    three = res["flat, eager, three launches"]
    assert three["steps"] == 3 and three["kernels_us"]["k2_adamw_flat"] == 190.0
    assert three["kernels_us"]["k0_finalize"] == 4.0
    rag = res["ragged, two launches (K0 folded into K3)"]
    assert rag["steps"] == 3 and rag["kernels_us"]["k3_adamw_fold"] == 9.0
