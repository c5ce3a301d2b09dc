"""The fused optimizer step captured once as a HIP graph and replayed.

K1 (unscale + norm partials) -> K0 (dsx_finalize_dev) -> K2 per parameter
group are recorded into one torch.cuda.CUDAGraph on the first step. Every
buffer the kernels touch (flat partition, DsxState, partials, scalars) keeps
its address for the optimizer's life, so the recorded launches stay valid.
What changes from step to step -- learning rate and the other per-group
hyper-parameters a scheduler may set, the bias-correction tables as they
grow -- lives in a DsxGroupsDev block in device memory, which K0 reads at
replay time. Before each replay the host packs that block into a pinned
staging slot and enqueues an async copy on the replay stream; the copy is
not part of the graph, so nothing in the graph is a memset or a host copy.

This path has no counterpart in the reference, which launches the step
eagerly every iteration (Src/zero/optimizer.py:212-274).
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops


class PinnedRing:
    """A few pinned staging slots for small host->device uploads. A slot is
    reused only after the copy that last read it has completed (its event),
    so the host never overwrites bytes a pending copy still needs."""

    def __init__(self, nbytes: int, slots: int = 4):
        self.bufs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(slots)]
        self.events: list[torch.cuda.Event | None] = [None] * slots
        self.i = 0

    def upload(self, data: bytes, dst: torch.Tensor) -> None:
        k = self.i
        self.i = (k + 1) % len(self.bufs)
        if self.events[k] is not None:
            self.events[k].synchronize()
        self.bufs[k].numpy()[:] = np.frombuffer(data, dtype=np.uint8)
        dst.copy_(self.bufs[k], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dst.device))
        self.events[k] = ev


class GraphedStep:
    """Captures `opt`'s fused step (an AdamWOptimizer with HBM-resident
    state) and replays it. Construction synchronises the device once."""

    def __init__(self, opt):
        if opt.streamer is not None:
            raise NotImplementedError("graph capture covers HBM-resident state; the offloaded step streams "
                                      "host chunks under host control")
        self.opt = opt
        dev = opt.device
        self.ngroups = len(opt.param_groups)
        self.groups_dev = torch.zeros(ops.GROUPS_BYTES, dtype=torch.uint8, device=dev)
        self.ring = PinnedRing(ops.GROUPS_BYTES)
        self._warm(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.device(dev), torch.cuda.graph(self.graph):
            self._record()
        self.replays = 0

    def _launches(self):
        opt = self.opt
        yield lambda: ops.unscale_norm(opt.flat.grad, opt.dstate, opt.partials, opt.nparts)
        yield lambda: ops.finalize_dev(opt.partials, opt.nparts, opt.dstate, opt.scaler.to_c(), self.groups_dev,
                                       self.ngroups, opt.scalars)
        for gi in range(self.ngroups):
            master, m, v, p16, g = opt.flat.group_views(gi)
            if master.numel() == 0:
                continue
            sc = opt.scalars[gi * ops.SCALARS_BYTES:(gi + 1) * ops.SCALARS_BYTES]
            yield lambda master=master, m=m, v=v, p16=p16, g=g, sc=sc: ops.adamw_flat(master, m, v, p16, g, sc)

    def _record(self) -> None:
        for launch in self._launches():
            launch()

    def _warm(self, dev: torch.device) -> None:
        """Launch the same kernel instantiations once, eagerly, on small
        scratch buffers (K0 sees an empty group block and writes skip, so K2
        returns at once), so that loading the code object happens outside
        the capture."""
        opt = self.opt
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
        torch.cuda.synchronize(dev)

    def replay(self, hypers, tables, bc_len: int) -> None:
        """Upload this step's group block, then replay, both on the current
        stream (no host synchronisation beyond a staging slot's reuse)."""
        blob = ops.pack_groups(hypers, tables, self.opt._t_offsets, bc_len)
        self.ring.upload(blob, self.groups_dev)
        self.graph.replay()
        self.replays += 1
