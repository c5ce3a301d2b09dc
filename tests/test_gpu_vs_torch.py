"""GPU parity against the reference's own update rule on the same device: the
fused step (K1/K0/K2 through AdamWOptimizer) against the step the reference
takes at world size 1 -- unscale by 1/scale (GradScaler.unscale_), skip on a
non-finite grad, per-tensor fp32 norm combined in Python double
(Src/zero/utils.py:126-154), g *= max/(norm + 1e-6) when norm > max
(Src/zero/utils.py:187-216), then torch.optim.AdamW.step on fp32 GPU tensors
(Src/zero/stage2.py:609-612) -- with torch's default dispatch (on GPU
tensors the multi-tensor path) and with the single-tensor path.

Bar: skip decisions and the loss-scale sequence
bit-exact; fp32 master / exp_avg / exp_avg_sq within 2 ulp; 16-bit params
within 1 ulp; grad norm within 1e-6 relative. Against torch's default path
the kernels follow its roundings, so the state is required bit-identical;
the single-tensor path (foreach=False, not the default on a GPU) divides
by the bias correction through a reciprocal (x * fl(1/b), up to 1.5 ulp
from x / b), which moves the update by up to ~3 ulp: it is held to 2 ulp on
exp_avg / exp_avg_sq and 4 ulp on the master, one step at a time from
torch's state. Where a result comes out of
cancellation (p*decay + update, m + w*(g - m)) the ulp is taken of the
largest operand of that last operation, as for the CPU pins of the oracle.
The reference's norm is an fp32 reduction, ours an fp64 sum of exact
squares; they are compared to 1e-6, and the clip coefficient on the
reference side is then taken (by the reference's formula) from our norm, so
that a last-bit difference between the two norms does not leak into the
AdamW comparison as a 1-ulp difference of every clipped grad."""
from __future__ import annotations

import math
import sys

import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _ulp(x):
    """ulp of fp32 values (of their magnitude), as float64, computed exactly
    on the host (np.frexp / np.ldexp; torch's ldexp goes through pow)."""
    import numpy as np
    a = np.abs(x.detach().float().cpu().numpy())
    _, e = np.frexp(a)  # a = m * 2^e, m in [0.5, 1)
    return np.ldexp(np.float64(1.0), np.maximum(e - 24, -149))


def _within(ours, ref, scale_of, k, what):
    """|ours - ref| <= k * ulp(scale_of) elementwise; returns the max ratio."""
    import numpy as np
    d = np.abs(ours.detach().cpu().numpy().astype(np.float64) - ref.detach().cpu().numpy().astype(np.float64))
    u = _ulp(scale_of)
    bad = ~(d <= k * u)  # k * u is exact (u is a power of two); NaN counts as bad
    r = d / u
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} elements beyond {k} ulp "
                                 f"(max {float(np.max(r[np.isfinite(r)])):.3f})")
    return float(np.max(r))


def _ulp16_diff(a, b, dt):
    """max ulp distance between two 16-bit tensors of the same sign pattern."""
    import torch
    ia = a.view(torch.int16).int()
    ib = b.view(torch.int16).int()
    # map sign-magnitude to a monotone integer line
    ma = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    mb = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return int((ma - mb).abs().max())


@pytest.mark.parametrize("dtype_name,foreach", [("bfloat16", None), ("float16", None), ("bfloat16", False),
                                                ("float16", False)])
def test_fused_step_matches_torch_adamw_on_gpu(gpu, dtype_name, foreach):
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    dt = getattr(torch, dtype_name)
    _say(f"fused step vs torch AdamW (foreach={foreach}) {dtype_name}")
    n = 1 << 22
    lr, betas, eps, wd, max_norm = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0
    gen = torch.Generator(device=gpu).manual_seed(21)
    p0 = torch.randn(n, device=gpu, generator=gen) * 0.02
    fp16 = dt == torch.float16
    sc = (ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=3, hysteresis=1, min_scale=1.0) if fp16
          else ScalerConfig(mode="none"))
    mine = AdamWOptimizer([torch.nn.Parameter(p0.clone())], lr=lr, betas=betas, eps=eps, weight_decay=wd,
                          max_grad_norm=max_norm, param_dtype=dt, loss_scaler=sc, device=gpu)
    ref_p = torch.nn.Parameter(p0.clone())
    ref = torch.optim.AdamW([ref_p], lr=lr, betas=betas, eps=eps, weight_decay=wd, foreach=foreach)
    scale, good = (2.0 ** 16 if fp16 else 1.0), 0
    worst = {"master": 0.0, "exp_avg": 0.0, "exp_avg_sq": 0.0}
    for step in range(8):
        sigma = 2e-4 if step % 2 else 3e-2  # alternate unclipped / clipped steps
        g32 = torch.randn(n, device=gpu, generator=gen) * sigma * scale
        g16 = g32.to(dt)
        inject = fp16 and step == 3
        if inject:
            g16[12345] = float("inf")
        mine.flat.grad.copy_(g16)
        # -- ours --
        mine.step()
        s = mine.read_state()
        # -- the reference's step at world size 1 --
        p_before = ref_p.detach().clone()
        st = ref.state.get(ref_p, {})
        m_before = st["exp_avg"].clone() if st else torch.zeros_like(p0)
        g = g16.float() * float(torch.tensor(1.0 / scale, dtype=torch.float32))
        skipped = not bool(torch.isfinite(g).all())
        if not skipped:
            norm = math.sqrt(float(g.norm(2).item()) ** 2)
            assert abs(s.last_norm - norm) <= 1e-6 * norm, f"step {step}: norm {s.last_norm} vs {norm}"
            if s.last_norm > max_norm:
                g.mul_(max_norm / (s.last_norm + 1e-6))
            ref_p.grad = g
            ref.step()
        if fp16:  # GradScaler.update with growth_interval = window, hysteresis 1
            if skipped:
                scale, good = max(scale * 0.5, 1.0), 0
            else:
                good += 1
                if good == 3:
                    scale, good = scale * 2.0, 0
        assert bool(s.last_skip) == skipped, f"step {step}: skip"
        assert s.scale == scale, f"step {step}: scale {s.scale} vs {scale}"
        if skipped:
            continue
        rs = ref.state[ref_p]
        if foreach is None:  # torch's default: bit for bit
            for name, a, b in (("master", mine.flat.master, ref_p.detach()), ("exp_avg", mine.flat.exp_avg, rs["exp_avg"]),
                               ("exp_avg_sq", mine.flat.exp_avg_sq, rs["exp_avg_sq"])):
                assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"step {step}: {name} not bit-identical"
            assert torch.equal(mine.flat.param16.view(torch.int16), ref_p.detach().to(dt).view(torch.int16))
            continue
        # exp_avg: m + w*(g - m); exp_avg_sq: no cancellation
        gc = ref_p.grad
        worst["exp_avg"] = max(worst["exp_avg"], _within(
            mine.flat.exp_avg, rs["exp_avg"], torch.maximum(torch.maximum(m_before.abs(), gc.abs()),
                                                            rs["exp_avg"].abs()), 2, f"step {step} exp_avg"))
        worst["exp_avg_sq"] = max(worst["exp_avg_sq"], _within(
            mine.flat.exp_avg_sq, rs["exp_avg_sq"], rs["exp_avg_sq"], 2, f"step {step} exp_avg_sq"))
        # master: p*decay + update
        upd = (ref_p.detach() - p_before * (1 - lr * wd)).abs()
        big = torch.maximum(torch.maximum((p_before * (1 - lr * wd)).abs(), upd), ref_p.detach().abs())
        worst["master"] = max(worst["master"], _within(mine.flat.master, ref_p.detach(), big, 4,
                                                       f"step {step} master"))
        # 16-bit params: the cast of the master; compare with the cast of torch's fp32 param
        assert _ulp16_diff(mine.flat.param16, ref_p.detach().to(dt), dt) <= 1, f"step {step}: param16"
        # next step from torch's state: two trajectories that run apart would
        # count a within-bar difference again wherever |p| is far below the update
        with torch.no_grad():
            mine.flat.master.copy_(ref_p.detach())
            mine.flat.exp_avg.copy_(rs["exp_avg"])
            mine.flat.exp_avg_sq.copy_(rs["exp_avg_sq"])
            mine.flat.param16.copy_(mine.flat.master)
    _say(f"worst ulp: {worst}")


def test_headline_shard_full_size_bit_identical_to_torch(gpu):
    """configs[2] at its full size -- 1,003,782,656 elements, bf16 grads
    N(0, 5e-4^2), lr 3e-4, betas (0.9, 0.95), eps 1e-8, wd 0.1, clip 1.0
    (active: the norm is about 15.8) -- two steps of the fused step against
    torch.optim.AdamW (default dispatch) on the same GPU: master, exp_avg,
    exp_avg_sq and bf16 params bit-identical."""
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer
    _say("configs[2] full size vs torch AdamW")
    n = 1_003_782_656
    lr, betas, eps, wd, max_norm = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0
    gen = torch.Generator(device=gpu).manual_seed(2)
    p0 = torch.empty(n, device=gpu).normal_(0.0, 0.02, generator=gen)
    mine = AdamWOptimizer([torch.nn.Parameter(p0)], lr=lr, betas=betas, eps=eps, weight_decay=wd,
                          max_grad_norm=max_norm, param_dtype=torch.bfloat16, device=gpu)
    ref_p = torch.nn.Parameter(mine.flat.master.clone())  # same fp32 start (p0's storage was re-homed)
    del p0
    ref = torch.optim.AdamW([ref_p], lr=lr, betas=betas, eps=eps, weight_decay=wd)
    for step in range(2):
        g16 = mine.flat.grad
        chunk = 1 << 27
        for s in range(0, n, chunk):
            e = min(n, s + chunk)
            g16[s:e].copy_(torch.empty(e - s, device=gpu).normal_(0.0, 5e-4, generator=gen))
        mine.step()
        st = mine.read_state()
        g = g16.float()
        norm = float(g.norm(2).item())
        assert abs(st.last_norm - norm) <= 1e-6 * norm and st.last_norm > max_norm, (st.last_norm, norm)
        g.mul_(max_norm / (st.last_norm + 1e-6))
        ref_p.grad = g
        ref.step()
        del g
        ref_p.grad = None
        rs = ref.state[ref_p]
        for name, a, b in (("master", mine.flat.master, ref_p.detach()), ("exp_avg", mine.flat.exp_avg, rs["exp_avg"]),
                           ("exp_avg_sq", mine.flat.exp_avg_sq, rs["exp_avg_sq"])):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"step {step}: {name}"
        assert torch.equal(mine.flat.param16.view(torch.int16), ref_p.detach().to(torch.bfloat16).view(torch.int16))
        torch.cuda.synchronize()


def _random_case(rng):
    import torch
    dt = [torch.float16, torch.bfloat16, None][int(rng.integers(3))]
    ngroups = int(rng.integers(1, 4))
    groups = []
    for _ in range(ngroups):
        sizes = [int(x) for x in rng.integers(1, 40_000, size=int(rng.integers(1, 4)))]
        b1 = float(rng.choice([0.9, 0.5, 0.0, 0.3, 0.99, 0.8]))
        b2 = float(rng.choice([0.999, 0.95, 0.0, 0.5, 0.9999]))
        groups.append(dict(sizes=sizes, lr=float(10 ** rng.uniform(-5, -1.5)), betas=(b1, b2),
                           eps=float(rng.choice([1e-8, 1e-6, 1e-3, 0.0])),
                           weight_decay=float(rng.choice([0.0, 0.01, 0.1, 0.5]))))
    max_norm = float(rng.choice([0.0, 1.0, 1e3]))
    sigma = float(10 ** rng.uniform(-5, -1))
    return dt, groups, max_norm, sigma


@pytest.mark.parametrize("case", range(24))
def test_random_configurations_bit_identical_to_torch(gpu, case):
    """Seeded random configurations -- sizes (odd, tiny), grad dtype fp16 /
    bf16 / fp32, 1-3 parameter groups with their own lr / betas (both lerp
    branches, beta1 = 0.5 exactly, beta = 0) / eps (0 included) / weight
    decay, clipping off / active / inactive -- three steps against
    torch.optim.AdamW (default dispatch) on the same GPU, bit for bit."""
    import numpy as np
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer
    rng = np.random.default_rng(9000 + case)
    dt, groups, max_norm, sigma = _random_case(rng)
    _say(f"random case {case}: dtype={dt} groups={len(groups)} max_norm={max_norm} sigma={sigma:.2e}")
    gen = torch.Generator(device=gpu).manual_seed(case)
    inits = [[torch.randn(n, device=gpu, generator=gen) * 0.05 for n in g["sizes"]] for g in groups]
    mine_groups, ref_groups, ref_params = [], [], []
    for g, ini in zip(groups, inits):
        hp = dict(lr=g["lr"], betas=g["betas"], eps=g["eps"], weight_decay=g["weight_decay"])
        mine_groups.append(dict(hp, params=[torch.nn.Parameter(t.clone()) for t in ini]))
        rp = [torch.nn.Parameter(t.clone()) for t in ini]
        ref_params += rp
        ref_groups.append(dict(hp, params=rp))
    mine = AdamWOptimizer(mine_groups, max_grad_norm=max_norm, param_dtype=dt, device=gpu)
    ref = torch.optim.AdamW(ref_groups)
    # start from the master the flat partition holds (fp32 values of the inits)
    for i, p in enumerate(ref_params):
        with torch.no_grad():
            p.copy_(mine.flat.views_of(i)["master"])
    gdt = dt or torch.float32
    for step in range(3):
        gs = [(torch.randn(p.shape, device=gpu, generator=gen) * sigma).to(gdt) for p in ref_params]
        for p, g in zip(mine.dsx_params, gs):
            p.grad.copy_(g)
        mine.step()
        st = mine.read_state()
        gf = [g.float() for g in gs]
        norm = float(torch.linalg.vector_norm(torch.cat(gf)).item())
        assert abs(st.last_norm - norm) <= 1e-6 * max(norm, 1e-30), (st.last_norm, norm)
        if max_norm > 0 and st.last_norm > max_norm:
            coef = max_norm / (st.last_norm + 1e-6)
            for g in gf:
                g.mul_(coef)
        for p, g in zip(ref_params, gf):
            p.grad = g
        ref.step()
        for i, p in enumerate(ref_params):
            v = mine.flat.views_of(i)
            s = ref.state[p]
            for name, a, b in (("master", v["master"], p.detach()), ("exp_avg", v["exp_avg"], s["exp_avg"]),
                               ("exp_avg_sq", v["exp_avg_sq"], s["exp_avg_sq"])):
                assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"step {step} param {i}: {name}"
            if dt is not None:
                assert torch.equal(mine.dsx_params[i].detach().view(torch.int16), p.detach().to(dt).view(torch.int16))


def test_sixteen_groups_with_empty_and_single_element_groups(gpu):
    """DSX_MAX_GROUPS parameter groups, one of them empty and one holding a
    single element, each with its own lr / betas / eps / weight decay: three
    steps bit for bit against torch.optim.AdamW (default dispatch)."""
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer
    _say("16 groups")
    gen = torch.Generator(device=gpu).manual_seed(16)
    sizes = [[37, 5], [], [1], [4096], [3, 3, 3], [1000], [8], [9], [17, 1], [2048], [513], [7], [64, 64], [1], [100],
             [31]]
    mine_groups, ref_groups, ref_params = [], [], []
    for k, sz in enumerate(sizes):
        hp = dict(lr=1e-4 * (k + 1), betas=(0.9 - 0.02 * k, 0.999 - 0.01 * k), eps=10.0 ** (-8 + k % 4),
                  weight_decay=0.01 * (k % 3))
        ini = [torch.randn(n, device=gpu, generator=gen) * 0.05 for n in sz]
        mine_groups.append(dict(hp, params=[torch.nn.Parameter(t.clone()) for t in ini]))
        rp = [torch.nn.Parameter(t.clone()) for t in ini]
        ref_params += rp
        ref_groups.append(dict(hp, params=rp))
    mine = AdamWOptimizer(mine_groups, max_grad_norm=1.0, param_dtype=torch.bfloat16, device=gpu)
    ref = torch.optim.AdamW(ref_groups)
    for i, p in enumerate(ref_params):
        with torch.no_grad():
            p.copy_(mine.flat.views_of(i)["master"])
    for step in range(3):
        gs = [(torch.randn(p.shape, device=gpu, generator=gen) * 0.05).to(torch.bfloat16) for p in ref_params]
        for p, g in zip(mine.dsx_params, gs):
            p.grad.copy_(g)
        mine.step()
        st = mine.read_state()
        gf = [g.float() for g in gs]
        if st.last_norm > 1.0:
            for g in gf:
                g.mul_(1.0 / (st.last_norm + 1e-6))
        for p, g in zip(ref_params, gf):
            p.grad = g
        ref.step()
        for i, p in enumerate(ref_params):
            v = mine.flat.views_of(i)
            s = ref.state[p]
            for name, a, b in (("master", v["master"], p.detach()), ("exp_avg", v["exp_avg"], s["exp_avg"]),
                               ("exp_avg_sq", v["exp_avg_sq"], s["exp_avg_sq"])):
                assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"step {step} param {i}: {name}"


WARM_FORMS = {"flat": ("AdamWOptimizer", {}), "graph": ("AdamWOptimizer", {"graph": True}),
              "capturable": ("AdamWOptimizer", {"capturable": True}),
              "offload": ("AdamWOptimizer", {"offload": True, "offload_chunk_elems": 4096}),
              "ragged": ("MultiTensorAdamWOptimizer", {})}


@pytest.mark.parametrize("form", list(WARM_FORMS))
def test_init_warm_step_follows_the_reference_trajectory(gpu, form):
    """ZeROOptimizer.init_warm_step() reproduces the reference stages'
    construction-time warm step (Src/zero/stage1.py:330-374: zero grads, one
    step of the torch optimizer, its state kept): against torch.optim.AdamW
    (default dispatch) on this GPU taking a zero-grad step and then the same
    four steps, every master value, exp_avg and exp_avg_sq bit for bit, in
    every storage form; the step count is 1 after the warm step while
    current_step stays 0; the loss scaler is untouched."""
    import torch
    from distributedspeed_amd import optimizers as O
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.zero import ZeROOptimizer
    _say(f"init warm step vs torch, {form}")
    cls_name, kw = WARM_FORMS[form]
    gen = torch.Generator(device=gpu).manual_seed(44)
    shapes = [(96, 33), (33,), (50, 17)]
    p0 = [torch.randn(s, device=gpu, generator=gen) * 0.05 for s in shapes]
    lr, betas, eps = 2e-3, (0.9, 0.98), 1e-8
    sc = ScalerConfig(mode="dynamic", init_scale=2.0 ** 10, window=2, hysteresis=1)
    ps = [torch.nn.Parameter(t.clone()) for t in p0]
    opt = getattr(O, cls_name)([{"params": ps[:2], "weight_decay": 0.1}, {"params": ps[2:], "weight_decay": 0.0}],
                               lr=lr, betas=betas, eps=eps, param_dtype=torch.bfloat16, loss_scaler=sc, device=gpu,
                               **kw)
    zero = ZeROOptimizer(opt, {"stage": 2})
    ref_ps = [torch.nn.Parameter(t.clone()) for t in p0]
    ref = torch.optim.AdamW([{"params": ref_ps[:2], "weight_decay": 0.1},
                             {"params": ref_ps[2:], "weight_decay": 0.0}], lr=lr, betas=betas, eps=eps)
    for p in ref_ps:
        p.grad = torch.zeros_like(p)
    ref.step()
    zero.init_warm_step()
    st = opt.read_state()
    assert st.t == 1 and zero.current_step == 0 and st.scale == 2.0 ** 10 and st.good_steps == 0
    assert all(p.grad is None for p in opt.dsx_params) or form == "capturable"
    with pytest.raises(RuntimeError, match="before any other step"):
        zero.init_warm_step()

    def check(tag):
        torch.cuda.synchronize()
        for i, rp in enumerate(ref_ps):
            v = opt.store.views_of(i)
            rs = ref.state[rp]
            for name, a, b in (("master", v["master"], rp.detach()), ("exp_avg", v["exp_avg"], rs["exp_avg"]),
                               ("exp_avg_sq", v["exp_avg_sq"], rs["exp_avg_sq"])):
                a = a.reshape(b.shape).to(b.device)
                assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"{tag}: tensor {i} {name}"

    check("after the warm step")
    for step in range(4):
        scale = float(opt.read_state().scale)
        for p, rp in zip(opt.dsx_params, ref_ps):
            g = (torch.randn(p.shape, device=gpu, generator=gen) * 1e-2).to(torch.bfloat16)
            if p.grad is None:
                p.grad = (g.float() * scale).to(torch.bfloat16)
            else:
                p.grad.copy_((g.float() * scale).to(torch.bfloat16))
            rp.grad = p.grad.float() * (1.0 / scale)
        zero.step()
        ref.step()
        check(f"step {step}")
    st = opt.read_state()
    assert st.t == 5 and zero.current_step == 4
