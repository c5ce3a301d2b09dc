"""One flat partition holding every trainable parameter of a rank.

The reference packs per-parameter grads into fp32 flat buffers every step
(OptimizedGradientBucket, Src/zero/stage1.py:109-151; AdvancedGradientPartitioner
with per-parameter views, Src/zero/stage2.py:108-193) and computes partition
bounds element-granular (Src/zero/partition.py:102-141). Here the layout is
built once and the copies disappear:

  param16  n x fp16/bf16   the model's parameters (param.data are views)
  grad     n x fp16/bf16   the model's grads (param.grad are views; autograd
                           accumulates into them in place)
  master   n x fp32        the optimizer's master weights
  exp_avg, exp_avg_sq      n x fp32

With fp32 training there is no param16: param.data are views of master and
grads are fp32. With `offload=True` master / exp_avg / exp_avg_sq are pinned
host tensors instead (the step streams them through HBM; param16 and grad
stay in HBM), which needs a 16-bit param dtype.

Grads reach the flat buffer one of two ways. After zero_grad(set_to_none=
False) the views stay bound and autograd accumulates into them: a zeroing
pass (2 B/elt written) and then, per micro-batch, the view read, the new
grad read and the sum written (6 B/elt). After zero_grad(set_to_none=True),
the default, p.grad is None, so autograd hands over the grad it produced
and a post-accumulate-grad hook copies it into the view (2 B read, 2 B
written) and rebinds p.grad to the view, which later micro-batches then
accumulate into: 4 B/elt instead of 8 for the first micro-batch, and the
copies run during backward. When the partition collects the norm
(enable_hook_norm, the optimizer's eager step), the hook's copy also writes
the norm's partial sums, and a step whose grads all arrived that way skips
its own pass over the grads (hook_norm_ready). A parameter that received no grad is zeroed in
its view before the step (check_grads_bound) and takes an AdamW step with a
zero grad, as torch does after zero_grad(set_to_none=False). Code that
writes grads straight into the flat buffer keeps the views bound with
zero_grad(set_to_none=False).

Parameters are laid out group by group in model order; every
parameter (and so every group) starts on an 8-element boundary, so each
group's range is 16-byte aligned in every buffer. Padding elements have zero
grad and zero master and stay zero under AdamW.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch

ALIGN = 8


def _round_up(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def _bind_hook(ref, i: int):
    """Post-accumulate-grad hook of parameter i: a grad autograd produced
    outside the flat buffer (p.grad was None) is copied into the parameter's
    view -- with the norm's partial sums taken on the way when the partition
    collects them -- and p.grad becomes the view again. A grad accumulated
    into the bound view makes any collected partials stale."""
    def hook(p):
        part = ref()
        if part is None:
            return
        view = part._grad_views[i]
        g = p.grad
        if g is view:
            part._hn_armed = False
            return
        if view.numel() == 0:
            # Nothing to copy (and an empty tensor's data_ptr() is 0, the
            # same as any other empty tensor's): the parameter's one partial
            # stays the zero it was allocated with.
            if part._hn_on:
                part._hn_fired[i] += 1
            p.grad = view
            return
        if g is not None and g.data_ptr() != view.data_ptr():
            if not (part._hn_armed and part._copy_with_norm(i, g)):
                view.copy_(g)
                part._hn_armed = False
        else:
            part._hn_armed = False
        p.grad = view
    return hook


@dataclass
class Slot:
    offset: int
    numel: int
    shape: torch.Size
    group: int
    name: str


class FlatPartition:
    def __init__(self, groups: list[list[torch.nn.Parameter]], device: torch.device,
                 param_dtype: torch.dtype | None, names: dict | None = None, offload: bool = False):
        """groups: parameter lists (one per optimizer param group).
        param_dtype: torch.float16 / torch.bfloat16 for mixed precision, None
        for fp32 training."""
        if param_dtype not in (None, torch.float16, torch.bfloat16):
            raise ValueError(f"param_dtype must be float16, bfloat16 or None, got {param_dtype}")
        if offload and param_dtype is None:
            raise ValueError("offloaded optimizer state needs fp16 or bf16 parameters (fp32 params would have to "
                             "live in host memory)")
        names = names or {}
        self.offload = bool(offload)
        self.device = torch.device(device)
        self.param_dtype = param_dtype
        self.grad_dtype = param_dtype or torch.float32
        self.slots: list[Slot] = []
        self.params: list[torch.nn.Parameter] = []
        self.group_ranges: list[tuple[int, int]] = []
        seen = set()
        off = 0
        for gi, plist in enumerate(groups):
            start = off
            for p in plist:
                if id(p) in seen:
                    raise ValueError("a parameter appears in more than one group")
                seen.add(id(p))
                n = p.numel()
                self.slots.append(Slot(off, n, p.shape, gi, names.get(id(p), f"param{len(self.params)}")))
                self.params.append(p)
                off = _round_up(off + n, ALIGN)
            self.group_ranges.append((start, off))
        self.numel = off
        dev = self.device
        if self.offload:
            from .offload import pinned_zeros
            self.master, self.exp_avg, self.exp_avg_sq = (pinned_zeros(self.numel) for _ in range(3))
        else:
            self.master, self.exp_avg, self.exp_avg_sq = (
                torch.zeros(self.numel, dtype=torch.float32, device=dev) for _ in range(3))
        self.grad = torch.zeros(self.numel, dtype=self.grad_dtype, device=dev)
        self.param16 = torch.zeros(self.numel, dtype=param_dtype, device=dev) if param_dtype else None
        with torch.no_grad():
            for s, p in zip(self.slots, self.params):
                src = p.detach().reshape(-1)
                self.master[s.offset:s.offset + s.numel].copy_(src.to(self.master.device, torch.float32))
                if self.offload:
                    self.param16[s.offset:s.offset + s.numel].copy_(src.to(dev, torch.float32))
            if self.param16 is not None and not self.offload:
                self.param16.copy_(self.master)  # round to nearest even
        self.rebind()
        # The hooks reach the partition through a weak reference, so a
        # parameter that outlives its optimizer does not keep the flat
        # buffers alive; they are removed when the partition goes.
        self._hn_on = False  # norm partials taken by the hooks' copies (enable_hook_norm)
        self._hn_armed = False
        ref = weakref.ref(self)
        self._hooks = [p.register_post_accumulate_grad_hook(_bind_hook(ref, i))
                       for i, p in enumerate(self.params) if p.requires_grad]

    def __del__(self):
        for h in getattr(self, "_hooks", ()):
            h.remove()

    def rebind(self) -> None:
        """Point every param.data / param.grad at its view of the flat buffers."""
        home = self.param16 if self.param16 is not None else self.master
        self._grad_views = []
        for s, p in zip(self.slots, self.params):
            p.data = home[s.offset:s.offset + s.numel].view(s.shape)
            gv = self.grad[s.offset:s.offset + s.numel].view(s.shape)
            p.grad = gv
            self._grad_views.append(gv)

    def check_grads_bound(self) -> None:
        """Autograd accumulates into an existing .grad in place, so p.grad stays
        the view rebind() set. If something replaced it (set it to None or to
        a new tensor), copy that into the flat buffer and restore the view."""
        for i, (s, p) in enumerate(zip(self.slots, self.params)):
            g = p.grad
            view = self._grad_views[i]
            if g is view:
                continue
            if g is None:
                view.zero_()
            elif g.data_ptr() != view.data_ptr():
                view.copy_(g)
            p.grad = view

    def group_views(self, gi: int):
        a, b = self.group_ranges[gi]
        return (self.master[a:b], self.exp_avg[a:b], self.exp_avg_sq[a:b],
                self.param16[a:b] if self.param16 is not None else None, self.grad[a:b])

    def views_of(self, i: int) -> dict:
        s = self.slots[i]
        sl = slice(s.offset, s.offset + s.numel)
        return {"master": self.master[sl].view(s.shape), "exp_avg": self.exp_avg[sl].view(s.shape),
                "exp_avg_sq": self.exp_avg_sq[sl].view(s.shape)}

    def zero_grad(self, set_to_none: bool = False) -> None:
        """set_to_none: p.grad = None, so the next backward hands its grads
        over (copied into the views by the hook); otherwise the flat grad
        buffer is zeroed in place and the views stay bound."""
        self._hn_armed = False
        if set_to_none:
            for p in self.params:
                p.grad = None
            if self._hn_on:
                self._hn_fired = [0] * len(self.params)
                self._hn_version = self.grad._version
                self._hn_armed = True
        else:
            self.grad.zero_()
            for p, view in zip(self.params, self._grad_views):
                if p.grad is not view:
                    p.grad = view

    def refresh_params16(self) -> None:
        """param16 <- master (RNE), after the master was loaded."""
        if self.param16 is not None:
            with torch.no_grad():
                self.param16.copy_(self.master.to(self.device))

    def refresh_master(self, indices=None) -> None:
        """master <- fp32(param) for the given parameters (all by default),
        after the 16-bit params were written from outside the step (a model
        state dict loaded after construction). The step reads only the
        master, so it would otherwise write the old values back over them.
        With fp32 training the params are views into the master: nothing to
        do."""
        if self.param16 is None:
            return
        with torch.no_grad():
            for i in (range(len(self.slots)) if indices is None else indices):
                s = self.slots[i]
                self.master[s.offset:s.offset + s.numel].copy_(self.param16[s.offset:s.offset + s.numel])

    def layout(self) -> list[dict]:
        return [{"name": s.name, "offset": s.offset, "numel": s.numel, "shape": list(s.shape), "group": s.group}
                for s in self.slots]

    def storage_bytes(self) -> dict:
        """Bytes held by the partition's buffers (padding included). With fp32
        training the params are views into the master: no separate bytes."""
        state = sum(t.numel() * t.element_size() for t in (self.master, self.exp_avg, self.exp_avg_sq))
        return {"params": self.param16.numel() * self.param16.element_size() if self.param16 is not None else 0,
                "grads": self.grad.numel() * self.grad.element_size(),
                "optimizer_states": state, "optimizer_states_on_host": self.offload}

    # ---- the norm taken by the hooks' copies ---------------------------------------------

    def enable_hook_norm(self, state: torch.Tensor) -> bool:
        """From now on the hooks copy grads with dsx_copy_unscale_norm, which
        also writes the norm's fp64 block partials (a segment per parameter,
        unscaled by the loss scale in `state`, a DsxState). hook_norm_ready()
        says when they describe the flat buffer exactly; reduce_hook_norm()
        then sums each segment into hook_norm_partials (one per parameter),
        from which K0 finalizes without a K1 pass. False (and off) for more
        parameters than K0 reads."""
        from . import _lib, ops
        if not self.params or len(self.params) > _lib.DSX_MAX_PARTIALS:
            return False
        counts = [ops.suggest_partials(s.numel) for s in self.slots]
        offs = [0]
        for c in counts:
            offs.append(offs[-1] + c)
        dev = self.device
        self._hn_block = torch.zeros(offs[-1], dtype=torch.float64, device=dev)
        self._hn_offsets = torch.tensor(offs, dtype=torch.int64).to(dev)
        self.hook_norm_partials = torch.zeros(len(self.params), dtype=torch.float64, device=dev)
        base = self._hn_block.data_ptr()
        self._hn_args = [(v.data_ptr(), s.numel, base + 8 * o, c)
                         for v, s, o, c in zip(self._grad_views, self.slots, offs, counts)]
        self._hn_state = state.data_ptr()
        self._hn_state_ref = state
        self._hn_gdt = ops.grad_code(self.grad_dtype)
        lib = _lib.load()
        self._hn_copy = lib.dsx_copy_unscale_norm
        self._hn_reduce = lib.dsx_reduce_segments
        self._hn_stream = ops.stream_of
        self._hn_fired = [0] * len(self.params)
        self._hn_version = -1
        self._hn_on = True
        return True

    def _copy_with_norm(self, i: int, g: torch.Tensor) -> bool:
        """The hook's copy of parameter i's grad with its norm partials (the
        caller checked that they are being collected); False when g does not
        qualify (the hook then copies with torch and the step runs K1).
        Autograd hands over a grad of the parameter's dtype, device and
        shape, so what is left to check is its layout."""
        ptr = g.data_ptr()
        if ptr & 15 or not g.is_contiguous():
            return False
        dst, n, blk, cnt = self._hn_args[i]
        rc = self._hn_copy(ptr, dst, self._hn_gdt, n, self._hn_state, blk, cnt, self._hn_stream(self.device))
        if rc:
            from . import _lib
            raise _lib.DsxError("dsx_copy_unscale_norm", rc, _lib.last_error())
        self._hn_fired[i] += 1
        self._hn_version = self.grad._version
        return True

    def hook_norm_ready(self) -> bool:
        """Whether the hooks' partials describe the flat grad buffer: since
        zero_grad(set_to_none=True) every parameter was copied by the hook with
        its partials, nothing accumulated into a bound view, and no torch
        in-place write touched the buffer afterwards (its version counter)."""
        return (self._hn_on and self._hn_armed and all(self._hn_fired)
                and self.grad._version == self._hn_version)

    def reduce_hook_norm(self, stream) -> None:
        """hook_norm_partials[i] <- sum of parameter i's block partials (one
        small launch, fixed order)."""
        from . import _lib
        rc = self._hn_reduce(self._hn_block.data_ptr(), self._hn_offsets.data_ptr(), len(self.params),
                             self.hook_norm_partials.data_ptr(), stream)
        if rc:
            raise _lib.DsxError("dsx_reduce_segments", rc, _lib.last_error())

    def disarm_hook_norm(self) -> None:
        """The partials were used (or passed over) by a step: the next one
        needs new grads."""
        self._hn_armed = False
