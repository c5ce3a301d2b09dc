"""Parameters left where they lie: the ragged-list form of the step (K3).

With `zero_optimization.contiguous_gradients: false` the reference keeps each
parameter's grad as its own tensor and steps them one by one (torch
AdamW's per-tensor loop, Src/zero/stage1.py:522-525); here every parameter
keeps its own storage and its own autograd-allocated grad, and the step runs
over the list through a device chunk table (dsx_unscale_norm_multi /
dsx_adamw_multi): one launch each for the norm and the update whatever the
number of tensors. When the list falls in K3's one-block-per-CU range, its
tensors of at least K2_TENSOR_ELEMS elements step through K2
(dsx_adamw_flat) one by one instead, and K3 takes the rest.

Per parameter: master / exp_avg / exp_avg_sq are fp32 tensors of the
parameter's shape owned here; with a 16-bit param dtype, param.data is the
16-bit copy K3 writes, and with fp32 training param.data is the master
itself. The chunk table holds raw addresses, so it is rebuilt whenever a
param's or a grad's storage has moved (checked every step on the host).
"""
from __future__ import annotations

import torch

from . import ops


# Tensors of at least this many elements step through K2 one by one (the
# rest through K3) when the whole list would put K3 in its one-block-per-CU
# regime (K3_SPLIT_RANGE chunks per CU). Measured on MI355X: a 12-layer Llama
# list (2.9e9 elements, 174 chunks per CU) 15.66 -> 13.64 ms; configs[1]'s
# GPT-2-small list (30 per CU) 0.6437 -> 0.6404 ms; configs[3]'s list (496
# per CU, K3's many-blocks regime) is faster as one K3 launch (37.72 against
# 38.72 ms) and stays so.
K2_TENSOR_ELEMS = 1 << 24
K3_SPLIT_RANGE = (20, 256)


def auto_chunk_elems(numel: int) -> int:
    """Chunk size for a list of `numel` elements: 65536 for large lists; for
    smaller ones a power of two down to 4096, so that the list still splits
    into about 4096 chunks (the kernels hand chunks to blocks statically, and
    a GPU of 256 CUs needs several rounds of them to balance). A list that
    fits in at most 1024 chunks of 2048 elements (2.1e6 elements) takes 2048:
    one trip of K3's slot loop per chunk (256 threads x 2 slots x 4
    elements), so that in K3's one-chunk-per-block shape, and in the
    two-launch step with K0 folded into K3, all of a chunk's loads are in
    flight at once. Eager drop-in steps on MI355X, one process: configs[0]'s
    MLP list (1.86e6 elements) 17.1-17.6 us per step in 4096-element chunks,
    14.9-15.2 in 2048 (1024: 19.8-20.0; 8192: 18.8-19.2); larger lists lose
    with 2048 (K1 walks twice the chunks): 3.9e6 elements 27.2 against 26.0
    us, 6.3e6 39.8 against 38.3."""
    c = 65536
    while c > 4096 and numel // c < 4096:
        c //= 2
    if c == 4096 and -(-numel // 2048) <= 1024:
        c = 2048
    return c


def k3_chunk_elems(numel: int) -> int:
    """Chunk size of K3's own table when a list's large tensors step through
    K2: a power of two from 65536 down to 4096 that gives at least 16384
    chunks where possible. What K3 then takes is many mid-size and small
    tensors (configs[1]'s 147 GPT-2-small tensors besides wte: 85.8e6
    elements), which it runs faster in small chunks: on two MI355X boxes, in
    one process each, 4096-element chunks against the 16384 of
    auto_chunk_elems took 407 against 414 us and 429 against 463 us (the
    whole 148-tensor list: 613 against 641 us)."""
    c = 65536
    while c > 4096 and numel // c < 16384:
        c //= 2
    return c


class RaggedParams:
    def __init__(self, groups: list[list[torch.nn.Parameter]], device: torch.device,
                 param_dtype: torch.dtype | None, names: dict | None = None, chunk_elems: int | None = None):
        if param_dtype not in (None, torch.float16, torch.bfloat16):
            raise ValueError(f"param_dtype must be float16, bfloat16 or None, got {param_dtype}")
        names = names or {}
        self.device = torch.device(device)
        self.param_dtype = param_dtype
        self.grad_dtype = param_dtype or torch.float32
        self.params: list[torch.nn.Parameter] = []
        self.group_of: list[int] = []
        self.names: list[str] = []
        self.master: list[torch.Tensor] = []
        self.exp_avg: list[torch.Tensor] = []
        self.exp_avg_sq: list[torch.Tensor] = []
        seen = set()
        with torch.no_grad():
            for gi, plist in enumerate(groups):
                for p in plist:
                    if id(p) in seen:
                        raise ValueError("a parameter appears in more than one group")
                    seen.add(id(p))
                    src = p.detach()
                    if param_dtype is None:
                        if src.dtype != torch.float32:
                            raise ValueError(f"fp32 training needs fp32 parameters, got {src.dtype}")
                        master = src.to(self.device).contiguous().clone()
                        p.data = master
                    else:
                        master = src.to(self.device, torch.float32).contiguous().clone()
                        p.data = master.to(param_dtype)  # round to nearest even
                    self.params.append(p)
                    self.group_of.append(gi)
                    self.names.append(names.get(id(p), f"param{len(self.params) - 1}"))
                    self.master.append(master)
                    self.exp_avg.append(torch.zeros_like(master))
                    self.exp_avg_sq.append(torch.zeros_like(master))
                    if p.grad is not None:
                        p.grad = p.grad.to(self.device, self.grad_dtype).contiguous()
        self.numel = sum(m.numel() for m in self.master)
        self.chunk_elems = int(chunk_elems) if chunk_elems else auto_chunk_elems(self.numel)
        self.ngroups = len(groups)
        self._table = None
        self._key = None
        self.k2_tensors: list[int] = []  # tensors the step runs through K2 (decided with each table)
        self.small_table = None  # K3's table over the other tensors when k2_tensors is not empty

    def ensure_grads(self) -> None:
        """Give every param a contiguous grad of the grad dtype on the device
        (zeros where autograd produced none, as the flat form does), 16-byte
        aligned for the tensors of K2's size (K2 takes them one by one)."""
        for p in self.params:
            g = p.grad
            if g is None:
                p.grad = torch.zeros_like(p, dtype=self.grad_dtype)
            elif g.dtype != self.grad_dtype or g.device != self.device or not g.is_contiguous():
                p.grad = g.to(self.device, self.grad_dtype).contiguous()
        for p, m in zip(self.params, self.master):
            if m.numel() >= K2_TENSOR_ELEMS and p.grad.data_ptr() % 16:
                p.grad = p.grad.clone()  # a fresh allocation is aligned

    def table(self) -> ops.ChunkTable:
        """The device chunk table for the current storage: rebuilt when a
        param's address changed; when only grads moved (autograd's own grads
        after zero_grad(set_to_none=True)), only the tensor table's grad
        pointers are refreshed, in place."""
        self.ensure_grads()
        key = tuple((p.data_ptr(), p.grad.data_ptr()) for p in self.params)
        if (self._table is not None and key != self._key
                and all(a[0] == b[0] for a, b in zip(key, self._key))):
            self._table.update_grads([p.grad for p in self.params])
            if self.small_table is not None:
                self.small_table.update_grads([self.params[i].grad for i in self._small])
            self._key = key
        if key != self._key:
            for p, m in zip(self.params, self.master):
                if p.data.shape != m.shape or (self.param_dtype is None and p.data.data_ptr() != m.data_ptr()):
                    raise RuntimeError("a parameter's storage was replaced after the optimizer was built")
                if self.param_dtype is not None and (p.dtype != self.param_dtype or not p.data.is_contiguous()):
                    raise RuntimeError("a parameter's dtype or layout was changed after the optimizer was built")
            p16 = None if self.param_dtype is None else [p.data for p in self.params]
            self._table = ops.ChunkTable(self.master, self.exp_avg, self.exp_avg_sq, p16,
                                         [p.grad for p in self.params], self.group_of, self.chunk_elems)
            self._split(p16)
            self._key = key
        return self._table

    def _split(self, p16) -> None:
        """Choose the tensors that step through K2 for the table just built,
        and build K3's table over the rest."""
        cus = torch.cuda.get_device_properties(self.device).multi_processor_count
        per_cu = self._table.nchunks / cus
        big = []
        if K3_SPLIT_RANGE[0] <= per_cu < K3_SPLIT_RANGE[1]:
            # K2 needs every array 16-byte aligned. master / exp_avg / exp_avg_sq
            # are allocated here and ensure_grads realigns a large tensor's grad
            # before each step, but param.data may have been replaced by a
            # misaligned view: such a tensor stays in K3's table, whose scalar
            # loop takes any address.
            big = [i for i, m in enumerate(self.master) if m.numel() >= K2_TENSOR_ELEMS
                   and all(t.data_ptr() % 16 == 0 for t in (m, self.exp_avg[i], self.exp_avg_sq[i]))
                   and (p16 is None or p16[i].data_ptr() % 16 == 0)]
        self.k2_tensors = big
        taken = set(big)
        self._small = [i for i in range(len(self.params)) if i not in taken]
        self.small_table = None
        if big and self._small:
            sub = self._small
            n_small = sum(self.master[i].numel() for i in sub)
            self.small_table = ops.ChunkTable(
                [self.master[i] for i in sub], [self.exp_avg[i] for i in sub], [self.exp_avg_sq[i] for i in sub],
                None if p16 is None else [p16[i] for i in sub], [self.params[i].grad for i in sub],
                [self.group_of[i] for i in sub], k3_chunk_elems(n_small))

    def zero_grad(self, set_to_none: bool = False) -> None:
        """set_to_none: p.grad = None, so the next backward's grads are read
        where autograd puts them (the tensor table's grad pointers are
        refreshed at the next step; nothing is copied or zeroed); otherwise
        the grads are zeroed in place and their addresses stay."""
        if set_to_none:
            for p in self.params:
                p.grad = None
            return
        gs = [p.grad for p in self.params if p.grad is not None]
        if gs:
            torch._foreach_zero_(gs)

    def views_of(self, i: int) -> dict:
        return {"master": self.master[i], "exp_avg": self.exp_avg[i], "exp_avg_sq": self.exp_avg_sq[i]}

    def refresh_params16(self) -> None:
        """param.data <- master (RNE), after the master was loaded."""
        if self.param_dtype is None:
            return
        with torch.no_grad():
            for p, m in zip(self.params, self.master):
                p.data.copy_(m)

    def refresh_master(self, indices=None) -> None:
        """master <- fp32(param) for the given parameters (all by default),
        after the 16-bit params were written from outside the step; with fp32
        training the param is the master."""
        if self.param_dtype is None:
            return
        with torch.no_grad():
            for i in (range(len(self.params)) if indices is None else indices):
                self.master[i].copy_(self.params[i].data)

    def storage_bytes(self) -> dict:
        """Bytes held per the layout: 16-bit params (with fp32 training the
        param is the master), grads of the grad dtype, fp32 master/m/v."""
        elt16 = 2 if self.param_dtype is not None else 0
        return {"params": elt16 * self.numel,
                "grads": self.numel * torch.empty(0, dtype=self.grad_dtype).element_size(),
                "optimizer_states": 12 * self.numel, "optimizer_states_on_host": False}

    def layout(self) -> list[dict]:
        out, off = [], 0
        for p, name, gi in zip(self.params, self.names, self.group_of):
            out.append({"name": name, "offset": off, "numel": p.numel(), "shape": list(p.shape), "group": gi})
            off += p.numel()
        return out
