"""The fused optimizer step captured once as a HIP graph and replayed.

The launches of one dsx_zero_step_dev call -- K1 (unscale + norm partials)
then K2 per parameter group with the finalize folded in, or on partitions
above the fold's bound K1 -> K0 (dsx_finalize_dev) -> K2 per group -- are
recorded into one torch.cuda.CUDAGraph on the first step. Every buffer the
kernels touch (flat partition, DsxState, partials, scalars) keeps its
address for the optimizer's life, so the recorded launches stay valid. What
changes from step to step -- learning rate and the other per-group
hyper-parameters a scheduler may set, the bias-correction tables as they
grow -- lives in a DsxGroupsDev block in device memory, which the kernels
read at replay time. When those values changed since the last replay, the host
enqueues dsx_groups_upload before the replay (a one-wave kernel that takes
the block as its argument: no staging buffer, no DMA copy, no host wait);
the upload is not part of the graph, and nothing in the graph is a memset
or a host copy.

A GraphedStep keeps no reference to its optimizer (the optimizer holds the
GraphedStep), so the pair is freed by reference counting when the optimizer
goes away, never later by the cyclic garbage collector -- which could
otherwise destroy a graph in the middle of another graph's capture. The
capture itself runs with the cyclic collector paused for the same reason.

This path has no counterpart in the reference, which launches the step
eagerly every iteration (Src/zero/optimizer.py:212-274).
"""
from __future__ import annotations

import gc

import torch

from . import _lib, ops


class GraphedStep:
    """Captures the fused step of `opt` (an AdamWOptimizer with HBM-resident
    state) and replays it. Construction synchronises the device once."""

    def __init__(self, opt):
        if opt.streamer is not None:
            raise NotImplementedError("graph capture covers HBM-resident state; the offloaded step streams "
                                      "host chunks under host control")
        dev = opt.device
        self.device = dev
        self.ngroups = len(opt.param_groups)
        self.groups_dev = torch.zeros(ops.GROUPS_BYTES, dtype=torch.uint8, device=dev)
        self._uploaded = None  # the values groups_dev holds
        self.replays = 0
        self.uploads = 0
        plans = self._plans(opt)
        self._warm(opt, dev)
        self.graph = torch.cuda.CUDAGraph()
        gc.collect()
        was_enabled = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.device(dev), torch.cuda.graph(self.graph):
                s = ops.stream_of(dev)
                for launch in plans:
                    launch(s)
        finally:
            if was_enabled:
                gc.enable()

    def _plans(self, opt) -> list:
        """The step's launches, checked and bound before the capture: one
        dsx_zero_step_dev call (K1, then each group's K2 with the finalize
        folded in, or K1, K0, K2 on larger partitions), its group block read
        from self.groups_dev when the graph replays."""
        return [ops.plan_zero_step_dev(opt.pack_plan(), self.groups_dev,
                                       keep=(opt.flat, opt.partials, opt.dstate, opt.scalars))]

    @staticmethod
    def _warm(opt, dev: torch.device) -> None:
        """Launch the same kernel instantiations once, eagerly, on small
        scratch buffers (K0 sees an empty group block and writes skip, so K2
        returns at once), so that loading the code object happens outside
        the capture."""
        gd = opt.flat.grad.dtype
        pd = opt.flat.param16.dtype if opt.flat.param16 is not None else None
        st = ops.new_state(dev)
        parts = torch.zeros(1, dtype=torch.float64, device=dev)
        sc = torch.zeros(ops.SCALARS_BYTES, dtype=torch.uint8, device=dev)
        groups = torch.zeros(ops.GROUPS_BYTES, dtype=torch.uint8, device=dev)
        g = torch.zeros(16, dtype=gd, device=dev)
        f = [torch.zeros(16, dtype=torch.float32, device=dev) for _ in range(3)]
        p16 = torch.zeros(16, dtype=pd, device=dev) if pd is not None else None
        ops.unscale_norm(g, st, parts, 1)
        ops.finalize_dev(parts, 1, st, opt.scaler.to_c(), groups, 1, sc)
        ops.adamw_flat(f[0], f[1], f[2], p16, g, sc)
        # the two-launch form's kernels (the empty group block makes it a skip)
        P = _lib.DsxFlatPlan()
        P.master, P.exp_avg, P.exp_avg_sq = f[0].data_ptr(), f[1].data_ptr(), f[2].data_ptr()
        P.param16 = p16.data_ptr() if p16 is not None else None
        P.grad, P.n = g.data_ptr(), g.numel()
        P.param_dtype = ops.dtype_code(pd) if pd is not None else _lib.DSX_F16
        P.grad_dtype = ops.grad_code(gd)
        P.state, P.partials, P.out = st.data_ptr(), parts.data_ptr(), sc.data_ptr()
        P.nparts, P.ngroups, P.scaler = 1, 1, opt.scaler.to_c()
        P.group_end[0] = g.numel()
        ops.plan_zero_step_dev(P, groups)(ops.stream_of(dev))
        torch.cuda.synchronize(dev)

    def replay(self, hypers, tables, t_offsets, bc_len: int) -> None:
        """Upload this step's group block if it differs from the one on the
        device, then replay, both on the current stream (no host wait)."""
        key = (tuple((h.lr, h.beta1, h.beta2, h.eps, h.weight_decay, h.max_grad_norm, h.clip_eps) for h in hypers),
               tuple(t.data_ptr() for t in tables), tuple(t_offsets), int(bc_len))
        if key != self._uploaded:
            ops.groups_upload(ops.pack_groups(hypers, tables, t_offsets, bc_len), self.groups_dev)
            self._uploaded = key
            self.uploads += 1
        self.graph.replay()
        self.replays += 1
