"""torch-tensor wrappers over the libdsx C ABI (include/dsx.h).

Every function checks shapes, dtypes, devices and alignment on the host
before anything is launched, then enqueues on torch's current HIP stream.
Nothing here synchronises the host with the device.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import (DSX_BF16, DSX_F16, DSX_F32, DSX_MAX_GROUPS, DsxAdamwHyper, DsxScalerConfig, DsxStepScalars,
                   DsxState)

_DT = {torch.float16: DSX_F16, torch.bfloat16: DSX_BF16}
_GDT = {torch.float16: DSX_F16, torch.bfloat16: DSX_BF16, torch.float32: DSX_F32}

STATE_BYTES = ctypes.sizeof(DsxState)
SCALARS_BYTES = ctypes.sizeof(DsxStepScalars)


def dtype_code(dt: torch.dtype) -> int:
    """Code of a 16-bit parameter dtype."""
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"expected a float16 or bfloat16 tensor, got {dt}") from None


def grad_code(dt: torch.dtype) -> int:
    """Code of a grad dtype (fp16, bf16 or fp32)."""
    try:
        return _GDT[dt]
    except KeyError:
        raise TypeError(f"expected a float16, bfloat16 or float32 grad, got {dt}") from None


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t: torch.Tensor, name: str, dtype: torch.dtype | None, numel: int | None, device: torch.device,
          align: int = 16) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name} has {t.numel()} elements, expected {numel}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() and t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")


def _device(t: torch.Tensor) -> torch.device:
    if t.device.type != "cuda":
        raise ValueError(f"libdsx runs on the GPU; got a tensor on {t.device}")
    return t.device


def new_state(device: torch.device, init_scale: float = 1.0, hysteresis: int = 1) -> torch.Tensor:
    """A DsxState on `device` (uint8[64]), initialised on the current stream."""
    st = torch.empty(STATE_BYTES, dtype=torch.uint8, device=device)
    _lib.call("dsx_state_init", _ptr(st), ctypes.c_float(init_scale), int(hysteresis), _stream(st.device))
    return st


def new_scalars(device: torch.device) -> torch.Tensor:
    return torch.zeros(SCALARS_BYTES, dtype=torch.uint8, device=device)


def scalars_from_host(sc: DsxStepScalars, device: torch.device) -> torch.Tensor:
    """Upload a host-built DsxStepScalars (for driving K2 directly)."""
    raw = torch.frombuffer(bytearray(bytes(sc)), dtype=torch.uint8)
    return raw.to(device)


def read_state(st: torch.Tensor) -> DsxState:
    """Copy a DsxState to the host (synchronises with the stream)."""
    return DsxState.from_buffer_copy(bytes(st.cpu().numpy().tobytes()))


def read_scalars(sc: torch.Tensor) -> DsxStepScalars:
    return DsxStepScalars.from_buffer_copy(bytes(sc.cpu().numpy().tobytes()))


def scale_view(st: torch.Tensor) -> torch.Tensor:
    """fp32 one-element device view of DsxState.scale (no host sync)."""
    return st[0:4].view(torch.float32)


class Launch:
    """One entry point with its arguments checked and bound once; calling it
    with a stream handle enqueues the launch. For buffers that never move
    (a flat partition) this takes the per-step host cost down to the ctypes
    call itself. `keep` holds the tensors (or tables) whose addresses are
    bound, so that they live as long as the launch does."""

    __slots__ = ("name", "fn", "args", "keep")

    def __init__(self, name: str, *args, keep=()):
        self.name = name
        self.fn = getattr(_lib.load(), name)
        self.args = args
        self.keep = tuple(keep)

    def __call__(self, stream: ctypes.c_void_p) -> None:
        rc = self.fn(*self.args, stream)
        if rc:
            raise _lib.DsxError(self.name, rc, _lib.last_error())


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> ctypes.c_void_p:
    """torch's current HIP stream on `device` as the void* the ABI takes
    (the raw handle query, without building a Stream object)."""
    if _RAW_STREAM is not None and device.index is not None:
        return ctypes.c_void_p(_RAW_STREAM(device.index))
    return _stream(device)


def suggest_partials(n: int) -> int:
    return int(_lib.load().dsx_suggest_partials(int(n)))


def plan_unscale_norm(grad: torch.Tensor, state: torch.Tensor, partials: torch.Tensor,
                      nparts: int | None = None) -> Launch:
    dev = _device(grad)
    _need(grad, "grad", None, None, dev)
    gdt = grad_code(grad.dtype)
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    nparts = nparts or partials.numel()
    _need(partials, "partials", torch.float64, None, dev, 8)
    if nparts > partials.numel():
        raise ValueError("nparts exceeds the partials buffer")
    return Launch("dsx_unscale_norm", _ptr(grad), gdt, ctypes.c_int64(grad.numel()), _ptr(state), _ptr(partials),
                  int(nparts), keep=(grad, state, partials))


def unscale_norm(grad: torch.Tensor, state: torch.Tensor, partials: torch.Tensor, nparts: int | None = None) -> None:
    """K1: partials[:nparts] = per-block fp64 sums of (grad * inv_scale)^2."""
    plan_unscale_norm(grad, state, partials, nparts)(_stream(grad.device))


def norm_type_of(norm_type) -> float:
    """clip_grad_norm_'s norm_type as a float: any p > 0 or inf (also the
    string "inf", as torch.nn.utils.clip_grad_norm_ takes it)."""
    try:
        p = float(norm_type)
    except (TypeError, ValueError):
        raise ValueError(f"norm_type must be a number > 0 or inf, got {norm_type!r}") from None
    if not p > 0:  # also NaN
        raise ValueError(f"norm_type must be > 0 (finite or inf), got {norm_type!r}")
    return p


def plan_norm_partials(grad: torch.Tensor, state: torch.Tensor, norm_type: float, partials: torch.Tensor,
                       nparts: int) -> Launch:
    """K1 for a norm of type norm_type: partials[:nparts] = per-block fp64
    sums of |grad * inv_scale|^p (maxima for p = inf)."""
    dev = _device(grad)
    _need(grad, "grad", None, None, dev)
    gdt = grad_code(grad.dtype)
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(partials, "partials", torch.float64, None, dev, 8)
    if not 1 <= nparts <= partials.numel():
        raise ValueError("nparts must be in [1, partials.numel()]")
    return Launch("dsx_norm_partials", _ptr(grad), gdt, ctypes.c_int64(grad.numel()), _ptr(state),
                  ctypes.c_double(norm_type_of(norm_type)), _ptr(partials), int(nparts), keep=(grad, state, partials))


def clip_prepare(partials: torch.Tensor, nparts: int, norm_type: float, max_norm: float, clip_eps: float,
                 state: torch.Tensor, norm_out: torch.Tensor) -> None:
    """The norm from plan_norm_partials' partials into norm_out (fp64, one
    element) and the one-shot clip coefficient the next finalize applies."""
    dev = _device(state)
    _need(partials, "partials", torch.float64, None, dev, 8)
    if not 1 <= nparts <= partials.numel():
        raise ValueError("nparts must be in [1, partials.numel()]")
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(norm_out, "norm_out", torch.float64, 1, dev, 8)
    _lib.call("dsx_clip_prepare", _ptr(partials), int(nparts), ctypes.c_double(norm_type_of(norm_type)),
              ctypes.c_double(max_norm), ctypes.c_double(clip_eps), _ptr(state), _ptr(norm_out), _stream(dev))


def finalize(partials: torch.Tensor, nparts: int, state: torch.Tensor, scaler: DsxScalerConfig,
             hyper: DsxAdamwHyper, bc_table: torch.Tensor, bc_len: int, out: torch.Tensor) -> None:
    """K0: norm, skip decision, clip coefficient, step scalars, scaler update."""
    dev = _device(state)
    _need(partials, "partials", torch.float64, None, dev, 8)
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(out, "scalars", torch.uint8, SCALARS_BYTES, dev, 8)
    _need(bc_table, "bc_table", torch.float64, None, dev, 8)
    if bc_table.numel() < 2 * bc_len:
        raise ValueError("bc_table shorter than bc_len")
    _lib.call("dsx_finalize", _ptr(partials), int(nparts), _ptr(state), scaler, hyper, _ptr(bc_table), int(bc_len),
              _ptr(out), _stream(dev))


def adamw_flat(master: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
               param16: torch.Tensor | None, grad: torch.Tensor, scalars: torch.Tensor) -> None:
    """K2: AdamW + 16-bit cast over a flat partition (in place)."""
    plan_adamw_flat(master, exp_avg, exp_avg_sq, param16, grad, scalars)(_stream(master.device))


def plan_adamw_flat(master: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
                    param16: torch.Tensor | None, grad: torch.Tensor, scalars: torch.Tensor) -> Launch:
    dev = _device(master)
    n = master.numel()
    for name, t in (("master", master), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        _need(t, name, torch.float32, n, dev)
    _need(grad, "grad", None, n, dev)
    gdt = grad_code(grad.dtype)
    pdt = DSX_F16
    if param16 is not None:
        _need(param16, "param16", None, n, dev)
        pdt = dtype_code(param16.dtype)
    _need(scalars, "scalars", torch.uint8, SCALARS_BYTES, dev, 8)
    return Launch("dsx_adamw_flat", _ptr(master), _ptr(exp_avg), _ptr(exp_avg_sq), _ptr(param16), pdt, _ptr(grad),
                  gdt, ctypes.c_int64(n), _ptr(scalars), keep=(master, exp_avg, exp_avg_sq, param16, grad, scalars))


def traffic_probe_flat(master: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
                       param16: torch.Tensor, grad: torch.Tensor) -> None:
    """Measurement only: K2's traffic in K2's launch shape without the AdamW
    math (values written back unchanged, param16 = RNE(master)); grad and
    param16 of one 16-bit type."""
    dev = _device(master)
    n = master.numel()
    for name, t in (("master", master), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        _need(t, name, torch.float32, n, dev)
    _need(grad, "grad", None, n, dev)
    _need(param16, "param16", grad.dtype, n, dev)
    Launch("dsx_traffic_probe_flat", _ptr(master), _ptr(exp_avg), _ptr(exp_avg_sq), _ptr(param16),
           dtype_code(param16.dtype), _ptr(grad), ctypes.c_int64(n))(_stream(dev))


def zero_step_flat(master: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
                   param16: torch.Tensor | None, grad: torch.Tensor, state: torch.Tensor,
                   scaler: DsxScalerConfig, hyper: DsxAdamwHyper, bc_table: torch.Tensor, bc_len: int,
                   partials: torch.Tensor, nparts: int, out: torch.Tensor) -> None:
    """K1 -> K0 -> K2 in one call (three launches on the current stream)."""
    dev = _device(master)
    n = master.numel()
    for name, t in (("master", master), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        _need(t, name, torch.float32, n, dev)
    _need(grad, "grad", None, n, dev)
    gdt = grad_code(grad.dtype)
    pdt = DSX_F16
    if param16 is not None:
        _need(param16, "param16", None, n, dev)
        pdt = dtype_code(param16.dtype)
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(out, "scalars", torch.uint8, SCALARS_BYTES, dev, 8)
    _need(partials, "partials", torch.float64, None, dev, 8)
    if nparts > partials.numel():
        raise ValueError("nparts exceeds the partials buffer")
    _need(bc_table, "bc_table", torch.float64, None, dev, 8)
    if bc_table.numel() < 2 * bc_len:
        raise ValueError("bc_table shorter than bc_len")
    _lib.call("dsx_zero_step_flat", _ptr(master), _ptr(exp_avg), _ptr(exp_avg_sq), _ptr(param16), pdt, _ptr(grad),
              gdt, n, _ptr(state), scaler, hyper, _ptr(bc_table), int(bc_len), _ptr(partials), int(nparts), _ptr(out),
              _stream(dev))


# ---- parameter groups ---------------------------------------------------------------

def finalize_groups(partials: torch.Tensor, nparts: int, state: torch.Tensor, scaler: DsxScalerConfig,
                    hypers: list[DsxAdamwHyper], bc_tables: list[torch.Tensor], t_offsets: list[int], bc_len: int,
                    out: torch.Tensor) -> None:
    """K0 for several parameter groups: out holds len(hypers) DsxStepScalars."""
    dev = _device(state)
    k = len(hypers)
    if not 1 <= k <= DSX_MAX_GROUPS or len(bc_tables) != k or len(t_offsets) != k:
        raise ValueError(f"need 1..{DSX_MAX_GROUPS} groups with one table and offset each")
    _need(partials, "partials", torch.float64, None, dev, 8)
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(out, "scalars", torch.uint8, SCALARS_BYTES * k, dev, 8)
    for i, t in enumerate(bc_tables):
        _need(t, f"bc_table[{i}]", torch.float64, None, dev, 8)
        if t.numel() < 2 * bc_len:
            raise ValueError("bc_table shorter than bc_len")
    FinalizeGroups(partials, nparts, state, out, k)(scaler, hypers, bc_tables, t_offsets, bc_len, _stream(dev))


class FinalizeGroups:
    """K0 over `ngroups` parameter groups with its buffers checked once;
    each call passes that step's scaler, hyper-parameters and tables."""

    def __init__(self, partials: torch.Tensor, nparts: int, state: torch.Tensor, out: torch.Tensor, ngroups: int):
        dev = _device(state)
        if not 1 <= ngroups <= DSX_MAX_GROUPS:
            raise ValueError(f"need 1..{DSX_MAX_GROUPS} groups")
        _need(partials, "partials", torch.float64, None, dev, 8)
        if not 1 <= nparts <= partials.numel():
            raise ValueError("nparts must be in [1, partials.numel()]")
        _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
        _need(out, "scalars", torch.uint8, SCALARS_BYTES * ngroups, dev, 8)
        self.k = ngroups
        self.name = "dsx_finalize_groups"
        self._keep = (partials, state, out)  # their addresses are bound below
        self.head = (_ptr(partials), int(nparts), _ptr(state))
        self.fn = getattr(_lib.load(), self.name)
        self.out = _ptr(out)
        self.hyper_t = DsxAdamwHyper * ngroups
        self.tab_t = ctypes.c_void_p * ngroups
        self.off_t = ctypes.c_int32 * ngroups

    def __call__(self, scaler: DsxScalerConfig, hypers, bc_tables, t_offsets, bc_len: int,
                 stream: ctypes.c_void_p) -> None:
        k = self.k
        if len(hypers) != k or len(bc_tables) != k or len(t_offsets) != k:
            raise ValueError(f"expected {k} groups with one table and offset each")
        key = (tuple(map(id, bc_tables)), tuple(t_offsets), bc_len)
        if key != getattr(self, "_key", None):  # tables / offsets checked and packed once per change
            for i, t in enumerate(bc_tables):
                if t.dtype != torch.float64 or t.device.type != "cuda" or t.numel() < 2 * bc_len:
                    raise ValueError(f"bc_table[{i}] must be a float64 GPU tensor of at least {2 * bc_len} entries")
            self._tabs = self.tab_t(*[t.data_ptr() for t in bc_tables])
            self._offs = self.off_t(*[int(x) for x in t_offsets])
            self._held = list(bc_tables)  # keep the tables (and their ids) alive while cached
            self._key = key
        rc = self.fn(*self.head, scaler, self.hyper_t(*hypers), self._tabs, self._offs, k, int(bc_len), self.out,
                     stream)
        if rc:
            raise _lib.DsxError(self.name, rc, _lib.last_error())


GROUPS_BYTES = ctypes.sizeof(_lib.DsxGroupsDev)


def pack_groups(hypers: list[DsxAdamwHyper], bc_tables: list[torch.Tensor], t_offsets: list[int],
                bc_len: int) -> _lib.DsxGroupsDev:
    """A host DsxGroupsDev for dsx_groups_upload (which checks the
    hyper-parameters as dsx_finalize_groups does)."""
    k = len(hypers)
    if not 1 <= k <= DSX_MAX_GROUPS or len(bc_tables) != k or len(t_offsets) != k:
        raise ValueError(f"need 1..{DSX_MAX_GROUPS} groups with one table and offset each")
    g = _lib.DsxGroupsDev()
    for i in range(k):
        h = hypers[i]
        t = bc_tables[i]
        if t.dtype != torch.float64 or t.device.type != "cuda" or t.numel() < 2 * bc_len:
            raise ValueError(f"bc_table[{i}] must be a float64 GPU tensor of at least {2 * bc_len} entries")
        if int(t_offsets[i]) < 0:
            raise ValueError(f"negative t_offset for group {i}")
        g.hyper[i] = h
        g.bc_table[i] = t.data_ptr()
        g.t_offset[i] = int(t_offsets[i])
    g.ngroups = k
    g.bc_len = int(bc_len)
    return g


def groups_upload(block: _lib.DsxGroupsDev, dst: torch.Tensor) -> None:
    """dst (device, GROUPS_BYTES) <- block, in stream order."""
    dev = _device(dst)
    _need(dst, "groups", torch.uint8, GROUPS_BYTES, dev, 8)
    _lib.call("dsx_groups_upload", ctypes.byref(block), _ptr(dst), _stream(dev))


def finalize_dev(partials: torch.Tensor, nparts: int, state: torch.Tensor, scaler: DsxScalerConfig,
                 groups_dev: torch.Tensor, max_groups: int, out: torch.Tensor) -> None:
    """K0 reading its per-group inputs from `groups_dev` (a DsxGroupsDev in
    device memory), the form a captured graph replays; `out` holds max_groups
    DsxStepScalars, all written."""
    plan_finalize_dev(partials, nparts, state, scaler, groups_dev, max_groups, out)(_stream(state.device))


def plan_finalize_dev(partials: torch.Tensor, nparts: int, state: torch.Tensor, scaler: DsxScalerConfig,
                      groups_dev: torch.Tensor, max_groups: int, out: torch.Tensor) -> Launch:
    dev = _device(state)
    if not 1 <= max_groups <= DSX_MAX_GROUPS:
        raise ValueError(f"max_groups must be in [1, {DSX_MAX_GROUPS}]")
    _need(partials, "partials", torch.float64, None, dev, 8)
    if nparts > partials.numel():
        raise ValueError("nparts exceeds the partials buffer")
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(groups_dev, "groups", torch.uint8, GROUPS_BYTES, dev, 8)
    _need(out, "scalars", torch.uint8, SCALARS_BYTES * max_groups, dev, 8)
    return Launch("dsx_finalize_dev", _ptr(partials), int(nparts), _ptr(state), scaler, _ptr(groups_dev),
                  int(max_groups), _ptr(out), keep=(partials, state, groups_dev, out))


def plan_zero_step_dev(plan: _lib.DsxFlatPlan, groups_dev: torch.Tensor, keep=()) -> Launch:
    """dsx_zero_step_dev bound to a packed flat plan and a device group
    block (uint8[GROUPS_BYTES]): the flat step whose per-group inputs the
    kernels read from device memory, so that it can be captured into a graph.
    `keep` holds the tensors the plan points into."""
    if groups_dev.dtype != torch.uint8 or groups_dev.numel() < GROUPS_BYTES or not groups_dev.is_cuda:
        raise ValueError("groups_dev must be a uint8 device tensor of GROUPS_BYTES bytes")
    if groups_dev.data_ptr() % 8:
        raise ValueError("groups_dev must be 8-byte aligned")
    return Launch("dsx_zero_step_dev", ctypes.byref(plan), _ptr(groups_dev), keep=(plan, groups_dev) + tuple(keep))


# ---- ragged lists (K3) --------------------------------------------------------------

class ChunkTable:
    """Device-resident tensor and chunk tables of a ragged list (built once;
    the tensors must stay in place while the table is used). The table keeps
    the state and parameter tensors alive; the grads must be alive whenever
    a launch that reads them runs (update_grads re-points the table).

    masters/exp_avgs/exp_avg_sqs are fp32; grads share one dtype (fp16, bf16
    or fp32); params16 (optional) share one 16-bit dtype; groups[i] is the
    parameter group of tensor i (indexes the scalars array)."""

    def __init__(self, masters, exp_avgs, exp_avg_sqs, params16, grads, groups=None, chunk_elems: int = 65536):
        k = len(masters)
        if not (len(exp_avgs) == len(exp_avg_sqs) == len(grads) == k) or (params16 is not None and len(params16) != k):
            raise ValueError("tensor lists must have equal lengths")
        if k == 0:
            raise ValueError("empty tensor list")
        groups = list(groups) if groups is not None else [0] * k
        if len(groups) != k or min(groups) < 0 or max(groups) >= DSX_MAX_GROUPS:
            raise ValueError("groups must give one index in [0, DSX_MAX_GROUPS) per tensor")
        dev = _device(masters[0])
        self.device = dev
        self.gdt = grad_code(grads[0].dtype)
        self.pdt = dtype_code(params16[0].dtype) if params16 is not None else DSX_F16
        self.ngroups = max(groups) + 1
        refs = (_lib.DsxTensorRef * k)()
        numels = (ctypes.c_int64 * k)()
        for i in range(k):
            n = masters[i].numel()
            for name, t in (("master", masters[i]), ("exp_avg", exp_avgs[i]), ("exp_avg_sq", exp_avg_sqs[i])):
                _need(t, f"{name}[{i}]", torch.float32, n, dev, 4)
            _need(grads[i], f"grad[{i}]", grads[0].dtype, n, dev, grads[0].element_size())
            p16 = None
            if params16 is not None:
                p16 = params16[i]
                _need(p16, f"param16[{i}]", params16[0].dtype, n, dev, 2)
            refs[i] = _lib.DsxTensorRef(masters[i].data_ptr(), exp_avgs[i].data_ptr(), exp_avg_sqs[i].data_ptr(),
                                        p16.data_ptr() if p16 is not None else None, grads[i].data_ptr(), n,
                                        int(groups[i]), 0)
            numels[i] = n
        L = _lib.load()
        cnt = L.dsx_count_chunks(numels, k, int(chunk_elems))
        if cnt < 0:
            raise ValueError(_lib.last_error())
        chunks = (_lib.DsxChunk * max(cnt, 1))()
        got = L.dsx_build_chunks(numels, k, int(chunk_elems), chunks, cnt)
        if got != cnt:
            raise RuntimeError(_lib.last_error())
        self.nchunks = int(cnt)
        self.numel = int(sum(numels))
        # The table holds raw addresses: it keeps the state and parameter
        # tensors alive. Not the grads: after zero_grad(set_to_none=True) the
        # old grads must be freeable during the next backward; nothing reads
        # them before update_grads points the table at the new ones.
        self._held = (list(masters), list(exp_avgs), list(exp_avg_sqs),
                      list(params16) if params16 is not None else None)
        self._refs = refs
        self._gdtype = grads[0].dtype
        self.tensors = torch.frombuffer(bytearray(bytes(refs)), dtype=torch.uint8).to(dev)
        self.chunks = torch.frombuffer(bytearray(bytes(chunks)), dtype=torch.uint8).to(dev)

    def update_grads(self, grads) -> None:
        """Point the tensor table at new grad tensors (same count, numels and
        dtype) in place: the chunk table and every launch bound to this table
        stay valid. The new table is copied from pinned memory on the current
        stream, so launches already queued read the old one and later ones the
        new one."""
        refs = self._refs
        if len(grads) != len(refs):
            raise ValueError(f"expected {len(refs)} grads, got {len(grads)}")
        esz = torch.empty(0, dtype=self._gdtype).element_size()
        for i, g in enumerate(grads):
            _need(g, f"grad[{i}]", self._gdtype, refs[i].numel, self.device, esz)
            refs[i].grad = g.data_ptr()
        host = torch.frombuffer(bytearray(bytes(refs)), dtype=torch.uint8).pin_memory()
        self.tensors.copy_(host, non_blocking=True)


def plan_unscale_norm_multi(table: ChunkTable, state: torch.Tensor, partials: torch.Tensor, nparts: int) -> Launch:
    dev = table.device
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(partials, "partials", torch.float64, None, dev, 8)
    if nparts > partials.numel():
        raise ValueError("nparts exceeds the partials buffer")
    return Launch("dsx_unscale_norm_multi", _ptr(table.tensors), _ptr(table.chunks), ctypes.c_int64(table.nchunks),
                  table.gdt, _ptr(state), _ptr(partials), int(nparts), keep=(table, state, partials))


def plan_norm_partials_multi(table: ChunkTable, state: torch.Tensor, norm_type: float, partials: torch.Tensor,
                             nparts: int) -> Launch:
    """plan_norm_partials over a ragged list's chunk table."""
    dev = table.device
    _need(state, "state", torch.uint8, STATE_BYTES, dev, 8)
    _need(partials, "partials", torch.float64, None, dev, 8)
    if not 1 <= nparts <= partials.numel():
        raise ValueError("nparts must be in [1, partials.numel()]")
    return Launch("dsx_norm_partials_multi", _ptr(table.tensors), _ptr(table.chunks), ctypes.c_int64(table.nchunks),
                  table.gdt, _ptr(state), ctypes.c_double(norm_type_of(norm_type)), _ptr(partials), int(nparts),
                  keep=(table, state, partials))


def unscale_norm_multi(table: ChunkTable, state: torch.Tensor, partials: torch.Tensor, nparts: int) -> None:
    """K1 over a ragged list: partials[:nparts] as unscale_norm."""
    plan_unscale_norm_multi(table, state, partials, nparts)(_stream(table.device))


def plan_adamw_multi(table: ChunkTable, scalars: torch.Tensor) -> Launch:
    dev = table.device
    _need(scalars, "scalars", torch.uint8, None, dev, 8)
    if scalars.numel() < SCALARS_BYTES * table.ngroups:
        raise ValueError(f"scalars must hold {table.ngroups} DsxStepScalars")
    return Launch("dsx_adamw_multi", _ptr(table.tensors), _ptr(table.chunks), ctypes.c_int64(table.nchunks),
                  table.pdt, table.gdt, _ptr(scalars), keep=(table, scalars))


def adamw_multi(table: ChunkTable, scalars: torch.Tensor) -> None:
    """K3: AdamW + cast over the list; scalars holds table.ngroups entries."""
    plan_adamw_multi(table, scalars)(_stream(table.device))
