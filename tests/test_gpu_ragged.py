"""GPU tests of the ragged form (MultiTensorAdamWOptimizer: K1 over a chunk
table, K0, K3) against the flat form (K1, K0, K2 over one buffer), whose
parity with the oracle is tested elsewhere. The update is elementwise, so
the two must agree bit for bit on master / exp_avg / exp_avg_sq / 16-bit
params and on every skip and loss-scale decision; only the fp64 norm may
differ in its last bits (the partial sums are grouped differently)."""
from __future__ import annotations

import sys

import pytest

pytestmark = pytest.mark.gpu

SHAPES = ((257, 33), (1000,), (64, 64), (5,), (3, 7, 11))


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _pair(gpu, dtype, scaler, shapes=SHAPES):
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    out = []
    for cls in (AdamWOptimizer, MultiTensorAdamWOptimizer):
        g = torch.Generator().manual_seed(5)
        ps = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.05).to(gpu)) for s in shapes]
        groups = [{"params": ps[:2]}, {"params": ps[2:], "lr": 3e-4, "weight_decay": 0.0, "betas": (0.8, 0.95)}]
        out.append(cls(groups, lr=1e-3, weight_decay=0.01, max_grad_norm=1.0, param_dtype=dtype,
                       loss_scaler=scaler, device=gpu))
    return out


def _check(flat, rag, tag):
    import torch
    for i, p in enumerate(rag.dsx_params):
        fv, rv = flat.flat.views_of(i), rag.store.views_of(i)
        for k in ("master", "exp_avg", "exp_avg_sq"):
            assert torch.equal(fv[k].view(torch.int32), rv[k].view(torch.int32)), f"{tag}: {k}[{i}]"
        fp = flat.dsx_params[i]
        if p.dtype != torch.float32:
            assert torch.equal(fp.detach().view(torch.int16), p.detach().view(torch.int16)), f"{tag}: param16[{i}]"
    a, b = flat.read_state(), rag.read_state()
    for k in ("scale", "good_steps", "hyst_left", "t", "iter", "overflow_count", "error", "last_skip"):
        assert getattr(a, k) == getattr(b, k), f"{tag}: state.{k} {getattr(a, k)} vs {getattr(b, k)}"
    assert abs(a.last_norm - b.last_norm) <= 1e-12 * max(a.last_norm, 1e-30) or a.last_norm == b.last_norm


def _set_grads(flat, rag, gen, scale, dtype, inf_at=None):
    import torch
    for i, (pf, pr) in enumerate(zip(flat.dsx_params, rag.dsx_params)):
        g = (torch.randn(pf.shape, generator=gen, device=pf.device) * 1e-2 * scale).to(dtype)
        if inf_at == i:
            g.view(-1)[g.numel() // 2] = float("inf")
        pf.grad.copy_(g)  # the flat form's grads are views into its buffer
        pr.grad = g.clone()  # the ragged form takes autograd-style fresh tensors


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16", "float32"])
def test_ragged_matches_flat(gpu, dtype_name):
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    dtype = getattr(torch, dtype_name)
    _say(f"ragged vs flat {dtype_name}")
    sc = (ScalerConfig(mode="dynamic", init_scale=2.0 ** 12, window=4, hysteresis=2)
          if dtype == torch.float16 else ScalerConfig(mode="none"))
    flat, rag = _pair(gpu, None if dtype == torch.float32 else dtype, sc)
    gen = torch.Generator(device=gpu).manual_seed(2)
    for step in range(12):
        scale = float(flat.read_state().scale)
        inf_at = (step % 5) if (dtype == torch.float16 and step in (3, 4, 8)) else None
        _set_grads(flat, rag, gen, scale if dtype == torch.float16 else 1.0, flat.flat.grad.dtype, inf_at)
        for o in (flat, rag):
            o.param_groups[1]["lr"] = 3e-4 * (1 + step)
            o.step()
        _check(flat, rag, f"step {step}")
    st = rag.read_state()
    assert st.t == (9 if dtype == torch.float16 else 12)


def test_ragged_large_tensors_through_k2_match_flat(gpu):
    """A list in K3's one-block-per-CU range (here ~29 chunks per CU) steps
    its tensors of >= 2^24 elements through K2 one by one and the rest
    through K3: bit-identical to the flat form over four steps with fp16
    grads, a dynamic loss scale with an overflow skip at step 2, two groups
    and clipping; a large tensor's grad given as a misaligned view is
    realigned (copied) before K2 reads it, and a large tensor whose param.data
    becomes a misaligned view leaves K2 for K3's table."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    from distributedspeed_amd.ragged import K2_TENSOR_ELEMS
    _say("ragged: large tensors through K2")
    shapes = [(4096, 4096), (3000, 4001), (4099,), (1024, 1023)]
    gen = torch.Generator(device=gpu).manual_seed(31)
    init = [torch.randn(*sh, device=gpu, generator=gen) * 0.02 for sh in shapes]
    grads = [[(torch.randn(*sh, device=gpu, generator=gen) * 1e-3 * 1024).half() for sh in shapes] for _ in range(4)]
    grads[1][2][7] = float("inf")

    def make(cls):
        ps = [torch.nn.Parameter(t.clone()) for t in init]
        groups = [{"params": ps[:2]}, {"params": ps[2:], "lr": 3e-4, "weight_decay": 0.0}]
        return ps, cls(groups, lr=1e-3, weight_decay=0.01, param_dtype=torch.float16, device=gpu, max_grad_norm=1.0,
                       loss_scaler=ScalerConfig(mode="dynamic", init_scale=1024.0, hysteresis=1))

    pf, flat = make(AdamWOptimizer)
    pr, rag = make(MultiTensorAdamWOptimizer)
    for step in range(4):
        for i, (a, b) in enumerate(zip(pf, pr)):
            a.grad = grads[step][i].clone()
            if i == 0:
                buf = torch.empty(grads[step][i].numel() + 8, dtype=torch.float16, device=gpu)
                view = buf[1:1 + grads[step][i].numel()].view(shapes[0])
                view.copy_(grads[step][i])
                assert view.data_ptr() % 16
                b.grad = view
            else:
                b.grad = grads[step][i].clone()
        if step == 3:
            # param.data replaced by a misaligned view of the same values: the
            # rebuilt table keeps the tensor in K3 (K2 needs 16-byte alignment)
            pbuf = torch.empty(pr[0].numel() + 8, dtype=torch.float16, device=gpu)
            pview = pbuf[1:1 + pr[0].numel()].view(shapes[0])
            pview.copy_(pr[0].data)
            assert pview.data_ptr() % 16
            pr[0].data = pview
        flat.step()
        rag.step()
        if step == 0:
            assert rag.store.k2_tensors == [0] and K2_TENSOR_ELEMS <= shapes[0][0] * shapes[0][1]
            assert rag.store.small_table is not None and rag.store.small_table.nchunks > 0
        if step == 3:
            assert rag.store.k2_tensors == [] and rag.store.small_table is None
    torch.cuda.synchronize()
    assert flat.read_state().overflow_count == rag.read_state().overflow_count == 1
    for i in range(len(shapes)):
        vf, vr = flat.store.views_of(i), rag.store.views_of(i)
        for name in ("master", "exp_avg", "exp_avg_sq"):
            assert torch.equal(vf[name].view(torch.int32), vr[name].view(torch.int32)), (i, name)
        assert torch.equal(pf[i].detach().view(torch.int16), pr[i].detach().view(torch.int16)), (i, "param16")


def test_ragged_misaligned_grads_and_table_rebuild(gpu):
    """Grads at odd element offsets take the kernels' unaligned paths; a
    grad replaced between steps moves storage and rebuilds the table."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    _say("ragged misaligned + rebuild")
    flat, rag = _pair(gpu, torch.bfloat16, ScalerConfig(mode="none"))
    gen = torch.Generator(device=gpu).manual_seed(9)
    keys = set()
    for step in range(4):
        _set_grads(flat, rag, gen, 1.0, torch.bfloat16)
        if step % 2:
            big = torch.empty(sum(p.numel() for p in rag.dsx_params) + 8, dtype=torch.bfloat16, device=gpu)
            off = 1
            for p in rag.dsx_params:
                v = big[off:off + p.numel()].view(p.shape)
                v.copy_(p.grad)
                p.grad = v
                off += p.numel() + 1
        for o in (flat, rag):
            o.step()
        keys.add(rag.store._key)
        _check(flat, rag, f"step {step}")
    assert len(keys) == 4


def test_engine_non_contiguous_gradients_matches_contiguous(gpu):
    import torch
    import distributedspeed_amd as ds
    _say("engine contiguous_gradients false")
    base = {"train_batch_size": 8, "optimizer": {"type": "AdamW", "params": {"lr": 1e-3}},
            "fp16": {"enabled": True, "initial_scale_power": 12}, "max_grad_norm": 1.0}
    opts = []
    for contiguous in (True, False):
        torch.manual_seed(0)
        model = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.GELU(), torch.nn.Linear(128, 8))
        cfg = dict(base, zero_optimization={"stage": 2, "contiguous_gradients": contiguous})
        engine, opt, _, _ = ds.initialize(model, cfg)
        gen = torch.Generator(device=gpu).manual_seed(1)
        for _ in range(5):
            x = torch.randn(8, 64, device=gpu, generator=gen)
            loss = engine(x).float().pow(2).mean()
            engine.backward(loss)
            engine.step()
        torch.cuda.synchronize()
        opts.append(opt.base_optimizer)
    from distributedspeed_amd.optimizers import MultiTensorAdamWOptimizer
    assert isinstance(opts[1], MultiTensorAdamWOptimizer) and not isinstance(opts[0], MultiTensorAdamWOptimizer)
    _check(opts[0], opts[1], "engine")
    assert opts[1].read_state().t == 5


def test_ragged_reads_autograd_grads_in_place_after_set_to_none(gpu):
    """zero_grad(set_to_none=True) in the ragged form: the next step reads the
    grads autograd allocated, refreshing only the tensor table's grad
    pointers (the chunk table object and its bound launches are kept), and
    trains bit-identically to the flat form; a parameter with no grad gets a
    zero grad as in the flat form."""
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    _say("ragged set_to_none")
    opts, tables = [], []
    for cls in (AdamWOptimizer, MultiTensorAdamWOptimizer):
        torch.manual_seed(7)
        model = torch.nn.Sequential(torch.nn.Linear(48, 80), torch.nn.GELU(), torch.nn.Linear(80, 8)).to(gpu)
        spare = torch.nn.Parameter(torch.randn(19, device=gpu) * 0.1)
        opt = cls(list(model.parameters()) + [spare], lr=1e-3, weight_decay=0.05, max_grad_norm=1.0,
                  param_dtype=torch.bfloat16, device=gpu)
        gen = torch.Generator(device=gpu).manual_seed(2)
        seen = []
        for _ in range(4):
            opt.zero_grad(set_to_none=True)
            assert all(p.grad is None for p in opt.dsx_params)
            x = torch.randn(12, 48, device=gpu, generator=gen).to(torch.bfloat16)
            model(x).float().pow(2).mean().backward()
            opt.step()
            if cls is MultiTensorAdamWOptimizer:
                seen.append(opt.store.table())
        torch.cuda.synchronize()
        opts.append(opt)
        tables.append(seen)
    assert all(t is tables[1][0] for t in tables[1])  # one chunk table throughout
    _check(opts[0], opts[1], "set_to_none")
    assert opts[1].read_state().t == 4


def test_bound_launches_keep_their_buffers_alive(gpu):
    """A launch bound by ops.plan_* holds raw device addresses; it keeps the
    objects behind them alive (a chunk table and, through it, the state and
    parameter tensors; a flat partition's buffers), so a caller that drops
    its own references cannot leave the launch pointing at freed memory. No
    kernel runs here: only object lifetimes are checked."""
    import gc
    import weakref
    import torch
    from distributedspeed_amd import ops
    _say("bound launches keep their buffers alive")
    ts = [torch.zeros(n, device=gpu) for n in (1000, 4096)]
    table = ops.ChunkTable(ts, [torch.zeros_like(t) for t in ts], [torch.zeros_like(t) for t in ts],
                           [t.half() for t in ts], [t.half() for t in ts])
    scalars = torch.zeros(ops.SCALARS_BYTES, dtype=torch.uint8, device=gpu)
    k3 = ops.plan_adamw_multi(table, scalars)
    wt, wm = weakref.ref(table), weakref.ref(ts[0])
    del table, ts
    gc.collect()
    assert wt() is not None and wm() is not None
    del k3
    gc.collect()
    assert wt() is None
    p, g = torch.zeros(4096, device=gpu), torch.zeros(4096, device=gpu, dtype=torch.float16)
    k2 = ops.plan_adamw_flat(p, torch.zeros_like(p), torch.zeros_like(p), None, g, scalars)
    wp = weakref.ref(p)
    del p, g
    gc.collect()
    assert wp() is not None
    del k2



@pytest.mark.parametrize("seed", range(8))
def test_ragged_random_lists_match_flat(gpu, seed):
    """Random lists through the ragged form's one-call step against the flat
    form, bit for bit, five steps each. Lists of 2e4-2e6 elements (2048-element
    chunks, K3 one chunk per block), 3e6-8e6 (4096-element chunks) and
    2.2e7-3e7 (over 20 chunks per CU: K1, K0 and K3 as one block per CU
    walking the list), split at random over 2 to 60 tensors, or 150 to 300
    tensors of at most 60 elements; a third of the tensors one element off
    the 16-byte grid, two groups with their own lr and betas, clipping, fp16
    with a dynamic scale and an inf at step 2 or bf16; odd seeds with the fold
    switched off (K1, K0, K3)."""
    import ctypes

    import numpy as np
    import torch
    from distributedspeed_amd import _lib
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    rng = np.random.default_rng(100 + seed)
    if seed == 3:  # many tiny tensors
        nt = int(rng.integers(150, 301))
        sizes = [int(x) for x in rng.integers(1, 61, size=nt)]
    else:
        lo, hi = ((2e4, 2e6), (3e6, 8e6), (2.2e7, 3e7))[seed % 3]
        total = int(rng.uniform(lo, hi))
        nt = int(rng.integers(2, 61))
        w = rng.dirichlet(np.ones(nt))
        sizes = [max(1, int(x)) for x in w * total]
    shapes = [(s,) if rng.random() < 0.5 or s < 4 else (s // 3, 3) if s >= 3 else (s,) for s in sizes]
    dt = torch.float16 if seed % 2 == 0 else torch.bfloat16
    fp16 = dt == torch.float16
    sc = (ScalerConfig(mode="dynamic", init_scale=2.0 ** 10, window=2, hysteresis=1) if fp16
          else ScalerConfig(mode="none"))
    gen = torch.Generator().manual_seed(seed)
    init = [torch.randn(s, generator=gen) * 0.05 for s in shapes]

    def build(cls):
        ps = []
        for k, t in enumerate(init):
            if k % 3 == 1:  # one element past a 16-byte boundary
                buf = torch.empty(t.numel() + 1, dtype=dt, device=gpu)
                v = buf[1:].view(t.shape)
                v.copy_(t)
                ps.append(torch.nn.Parameter(v))
            else:
                ps.append(torch.nn.Parameter(t.to(gpu, dt)))
        cut = max(1, len(ps) // 3)
        groups = [{"params": ps[:cut]}, {"params": ps[cut:], "lr": 3e-4, "betas": (0.8, 0.95)}]
        return cls(groups, lr=1e-3, weight_decay=0.05, max_grad_norm=0.3, param_dtype=dt, device=gpu,
                   loss_scaler=sc)

    flat, rag = build(AdamWOptimizer), build(MultiTensorAdamWOptimizer)
    _say(f"random list seed {seed}: {nt} tensors, {sum(sizes)} elements, {dt}, "
         f"chunks of {rag.store.chunk_elems}, fold {'off' if seed % 2 else 'on'}")
    ggen = torch.Generator(device=gpu).manual_seed(seed)
    fold_default = 3 << 23  # the library's default bound
    try:
        if seed % 2:
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(0))
        for step in range(5):
            scale = float(flat.read_state().scale) if fp16 else 1.0
            _set_grads(flat, rag, ggen, scale, dt, inf_at=(nt // 2 if fp16 and step == 2 else None))
            flat.step()
            rag.step()
            _check(flat, rag, f"seed {seed} step {step}")
    finally:
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(fold_default))
    st = rag.read_state()
    assert st.t == (4 if fp16 else 5) and st.error == 0


@pytest.mark.parametrize("handover", [False, True], ids=["grads-copied", "autograd-set-to-none"])
def test_zero_element_parameters(gpu, handover):
    """Parameters with no elements (torch's AdamW takes them) in both storage
    forms: among others, first and last in the list, and a whole group of
    them. They get no chunks and no elements of the flat buffer; every other
    tensor steps bit for bit as in the flat form. With `handover` the grads
    come from autograd after zero_grad(set_to_none=True), so the flat form's
    hook copies (an empty grad included) and its segment reduce replace K1."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    shapes = ((0,), (257, 33), (0, 5), (1000,), (5,), (0,))
    dt = torch.float16
    sc = ScalerConfig(mode="dynamic", init_scale=2.0 ** 8, window=2, hysteresis=1)
    opts = []
    for cls in (AdamWOptimizer, MultiTensorAdamWOptimizer):
        g = torch.Generator().manual_seed(11)
        ps = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.05).to(gpu, dt)) for s in shapes]
        groups = [{"params": [ps[0], ps[2]]}, {"params": [ps[1], ps[3]], "lr": 3e-4},
                  {"params": [ps[4], ps[5]], "betas": (0.8, 0.95)}]
        opts.append(cls(groups, lr=1e-3, weight_decay=0.01, max_grad_norm=0.5, param_dtype=dt, loss_scaler=sc,
                        device=gpu))
    flat, rag = opts
    before = [p.detach().clone() for p in rag.dsx_params]
    ggen = torch.Generator(device=gpu).manual_seed(12)
    _say(f"zero-element params, handover={handover}")
    for step in range(4):
        scale = float(flat.read_state().scale)
        if handover:
            w = [torch.randn(p.shape, generator=ggen, device=gpu) * 1e-2 for p in flat.dsx_params]
            for opt in opts:
                opt.zero_grad(set_to_none=True)
                loss = sum((p.float() * wi).sum() for p, wi in zip(opt.dsx_params, w))
                (loss * scale).backward()
            assert flat.flat.hook_norm_ready(), "the flat step would take K1, not the hooks' partials"
        else:
            _set_grads(flat, rag, ggen, scale, dt, inf_at=(3 if step == 1 else None))
        flat.step()
        rag.step()
        _check(flat, rag, f"zero-element step {step}")
    # dsx_params are in group order
    order = [0, 2, 1, 3, 4, 5]
    assert [tuple(p.shape) for p in rag.dsx_params] == [tuple(shapes[k]) for k in order]
    for p, b in zip(rag.dsx_params, before):
        if p.numel():
            assert not torch.equal(p.detach(), b), f"tensor of shape {tuple(p.shape)} did not step"
    st = rag.read_state()
    assert st.error == 0 and st.t == (4 if handover else 3)


def test_only_zero_element_parameters(gpu):
    """A model whose parameters all have no elements: an empty flat buffer and
    an empty chunk table. Both forms step (norm 0, no skip, t advances) and
    report no error, as torch's AdamW does nothing and raises nothing."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    sc = ScalerConfig(mode="dynamic", init_scale=2.0 ** 8, window=2, hysteresis=1)
    for cls in (AdamWOptimizer, MultiTensorAdamWOptimizer):
        ps = [torch.nn.Parameter(torch.zeros(s, device=gpu, dtype=torch.float16)) for s in ((0,), (0, 5))]
        opt = cls(ps, lr=1e-3, max_grad_norm=1.0, param_dtype=torch.float16, loss_scaler=sc, device=gpu)
        _say(f"only zero-element params: {cls.__name__}")
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            sum(p.float().sum() for p in opt.dsx_params).backward()
            opt.step()
        st = opt.read_state()
        assert st.error == 0 and st.t == 2 and st.last_skip == 0 and st.last_norm == 0.0, cls.__name__
