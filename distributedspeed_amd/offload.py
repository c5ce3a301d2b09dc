"""Optimizer state offloaded to pinned host memory.

The reference's `cpu_offload` parks optimizer state on the host and copies
all of it back to the GPU before stepping (Src/zero/stage1.py:376-398,
482-498; Src/zero/stage2.py:432-454, 563-582), and ZeRO-3 keeps a pinned-host
tier (Src/zero/stage3.py:881-898, 1189-1207). Here the fp32 master /
exp_avg / exp_avg_sq live in pinned host memory for good; the 16-bit params
and grads stay in HBM. A step is

    K1 over the device grads -> K0 (skip decision stays on the device)
    for each chunk k of every parameter group's range:
        copy stream in :  state[k] host -> staging[k % nbuf]     (hipMemcpyAsync)
        compute stream :  K2 on staging[k % nbuf] + grad/param16 views
        copy stream out:  staging[k % nbuf] -> state[k] host

with events so that chunk k+1 is copied in and chunk k-1 copied out while
chunk k computes; on a skipped step K2 leaves each chunk unchanged. The host
link, not HBM, bounds it: 12 B/elt each way.
All streams have the default priority.
"""
from __future__ import annotations

import ctypes
import time
import weakref

import torch

from . import ops

_hip = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime torch already loaded (same soname, so the same copy)."""
    global _hip
    if _hip is None:
        torch.cuda.init()
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipHostMalloc.restype = ctypes.c_int
        _hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        _hip.hipHostFree.restype = ctypes.c_int
        _hip.hipHostFree.argtypes = [ctypes.c_void_p]
    return _hip


def pinned_empty(n: int) -> torch.Tensor:
    """An fp32 CPU tensor of exactly n elements in pinned host memory from
    hipHostMalloc, freed with hipHostFree when the last tensor or view using
    it is released. (torch's pinned allocator rounds every request up to a
    power of two, which doubles the footprint of a 35 GB state array.) Raises
    MemoryError when the machine's pinned-memory limit is reached.

    Lifetime: torch.from_numpy keeps the ndarray alive for as long as the
    storage lives, the ndarray keeps the ctypes array alive, and the
    finalizer on the ctypes array frees the memory."""
    n = int(n)
    if n == 0:
        return torch.empty(0, dtype=torch.float32)
    import numpy as np
    hip = _hip_runtime()
    ptr = ctypes.c_void_p()
    rc = hip.hipHostMalloc(ctypes.byref(ptr), 4 * n, 0)
    if rc != 0 or not ptr.value:
        raise MemoryError(f"hipHostMalloc of {4 * n / 2**30:.1f} GiB failed (status {rc}): the pinned host memory "
                          "this machine allows is exhausted")
    buf = (ctypes.c_float * n).from_address(ptr.value)
    weakref.finalize(buf, hip.hipHostFree, ptr.value)
    return torch.from_numpy(np.ctypeslib.as_array(buf))


_COPY_STREAMS: dict = {}


def copy_streams(device: torch.device) -> tuple:
    """One (copy-in, copy-out) stream pair per device, created once. HIP maps
    streams onto a small number of hardware queues (4 by default); every extra
    stream raises the chance that copy-in and copy-out share a queue and
    serialise, so all offload work on a device uses this one pair."""
    device = torch.device(device)
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _COPY_STREAMS:
        _COPY_STREAMS[key] = (torch.cuda.Stream(device), torch.cuda.Stream(device))
    return _COPY_STREAMS[key]


class HostStateStreamer:
    def __init__(self, device: torch.device, chunk_elems: int = 64 << 20, nbuf: int = 3):
        if chunk_elems <= 0 or chunk_elems % 8:
            raise ValueError("chunk_elems must be a positive multiple of 8")
        if nbuf < 2:
            raise ValueError("nbuf must be >= 2")
        self.device = torch.device(device)
        self.chunk = int(chunk_elems)
        self.nbuf = int(nbuf)
        self.stage = [[torch.empty(self.chunk, dtype=torch.float32, device=self.device) for _ in range(3)]
                      for _ in range(self.nbuf)]
        self.s_in, self.s_out = copy_streams(self.device)
        self.ev_in = [torch.cuda.Event() for _ in range(self.nbuf)]
        self.ev_done = [torch.cuda.Event() for _ in range(self.nbuf)]
        self.ev_out = [torch.cuda.Event() for _ in range(self.nbuf)]
        self.last_bytes = 0  # host<->HBM bytes the last run() moved (both directions)

    def run(self, host_state: tuple[torch.Tensor, torch.Tensor, torch.Tensor], param16: torch.Tensor | None,
            grad: torch.Tensor | None, pieces: list[tuple[int, int, torch.Tensor | None]], *,
            copy_only: bool = False) -> None:
        """pieces: (start, end, scalars) ranges of the flat partition, each
        with the DsxStepScalars (device uint8[64]) of its parameter group.
        copy_only (measurement only): the same copies, streams and events
        with the AdamW launch left out, so every chunk goes back unchanged;
        param16, grad and the scalars are then unused."""
        compute = torch.cuda.current_stream(self.device)
        # Everything earlier on the compute stream (K0, the previous step's
        # K2s) and every earlier copy out is ordered before this step's copies.
        self.s_in.wait_stream(compute)
        self.s_in.wait_stream(self.s_out)
        k = 0
        moved = 0
        for a, b, scal in pieces:
            for s in range(a, b, self.chunk):
                e = min(b, s + self.chunk)
                n = e - s
                slot = k % self.nbuf
                st = [t[:n] for t in self.stage[slot]]
                with torch.cuda.stream(self.s_in):
                    if k >= self.nbuf:
                        self.s_in.wait_event(self.ev_out[slot])
                    for dst, src in zip(st, host_state):
                        dst.copy_(src[s:e], non_blocking=True)
                    self.ev_in[slot].record(self.s_in)
                compute.wait_event(self.ev_in[slot])
                if not copy_only:
                    ops.adamw_flat(st[0], st[1], st[2], param16[s:e] if param16 is not None else None, grad[s:e],
                                   scal)
                self.ev_done[slot].record(compute)
                with torch.cuda.stream(self.s_out):
                    self.s_out.wait_event(self.ev_done[slot])
                    for dst, src in zip(host_state, st):
                        dst[s:e].copy_(src, non_blocking=True)
                    self.ev_out[slot].record(self.s_out)
                moved += 24 * n
                k += 1
        # the step is complete, in stream order, once the last copy out is
        compute.wait_stream(self.s_out)
        self.last_bytes = moved


def pinned_zeros(n: int) -> torch.Tensor:
    t = pinned_empty(n)
    t.zero_()
    return t


def measure_link(device: torch.device, nbytes: int = 1 << 30) -> dict:
    """Plain pinned-host <-> HBM copy bandwidth (GB/s), one direction at a
    time and both at once: the ceiling the streamed step is compared to."""
    n = nbytes // 4
    h1 = pinned_empty(n)
    h2 = pinned_empty(n)
    d1 = torch.empty(n, dtype=torch.float32, device=device)
    d2 = torch.empty(n, dtype=torch.float32, device=device)
    s1, s2 = copy_streams(device)
    out = {}
    for name, fn in (("h2d", lambda: d1.copy_(h1, non_blocking=True)),
                     ("d2h", lambda: h2.copy_(d2, non_blocking=True))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        out[name] = 3 * nbytes / (time.perf_counter() - t0) / 1e9
    reps = 8
    for timed in (False, True):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps if timed else 1):
            with torch.cuda.stream(s1):
                d1.copy_(h1, non_blocking=True)
            with torch.cuda.stream(s2):
                h2.copy_(d2, non_blocking=True)
        torch.cuda.synchronize()
    out["both_each_way"] = reps * nbytes / (time.perf_counter() - t0) / 1e9
    return out


def measure_streamer_link(streamer: HostStateStreamer, host_state: tuple, reps: int = 4, trials: int = 3,
                          pipeline_passes: int = 2, lead=None) -> dict:
    """The host link as the streamed step sees it, on the streamer's own
    copy-in and copy-out streams, staging buffers and the pinned state
    arrays:
      h2d, d2h        one direction alone (three arrays of one chunk per
                      repetition), best of `trials`;
      pairs_each_way  both at once, the same copies, best of `trials`;
      copy_pipeline_each_way  the step's whole copy schedule over every
                      chunk of the state with the AdamW launch left out
                      (run(copy_only=True)), best of `pipeline_passes`;
      sweep_each_way  both directions free-running, no dependency between
                      them, a step's bytes each way: copies in of every
                      chunk of the state (its own host addresses) into
                      staging slots 1 and 2 (slot 1 alone with two slots),
                      while copies out of slot 0 write the first chunk back;
                      best of `pipeline_passes`;
      copy_pipeline_behind_lead_each_way  with `lead` (a callable that
                      enqueues work on the current stream and changes no
                      state, e.g. the step's own K1): the copy-only schedule
                      started behind it, as a step's copies start behind K1
                      and K0, best of `pipeline_passes` (the lead's time is
                      not counted out: a lead of a few hundred microseconds
                      against a schedule of hundreds of milliseconds);
      both_each_way   the largest of the both-ways figures.
    Every copy out writes back the values a copy in read (staging slot 0 is
    first loaded from the arrays' first chunk), so the state is unchanged.
    Needs at least two chunks of state."""
    c = streamer.chunk
    if min(t.numel() for t in host_state) < 2 * c:
        raise ValueError("measure_streamer_link needs at least two chunks of state")
    a_slot, b_slot = streamer.stage[0], streamer.stage[1]
    s_in, s_out = streamer.s_in, streamer.s_out
    for d, h in zip(a_slot, host_state):
        d.copy_(h[:c])
    torch.cuda.synchronize(streamer.device)

    def copy_in():
        with torch.cuda.stream(s_in):
            for d, h in zip(b_slot, host_state):
                d.copy_(h[c:2 * c], non_blocking=True)

    def copy_out():
        with torch.cuda.stream(s_out):
            for d, h in zip(a_slot, host_state):
                h[:c].copy_(d, non_blocking=True)

    def timed(fns) -> float:
        best = 0.0
        for _ in range(trials):
            torch.cuda.synchronize(streamer.device)
            t0 = time.perf_counter()
            for _ in range(reps):
                for fn in fns:
                    fn()
            torch.cuda.synchronize(streamer.device)
            best = max(best, reps * 12 * c / (time.perf_counter() - t0) / 1e9)
        return best

    copy_in()
    copy_out()
    out = {"h2d": timed([copy_in]), "d2h": timed([copy_out]), "pairs_each_way": timed([copy_in, copy_out]),
           "bytes_each_way_per_rep": 12 * c}
    n = min(t.numel() for t in host_state)
    best = 0.0
    for _ in range(max(1, pipeline_passes)):
        torch.cuda.synchronize(streamer.device)
        t0 = time.perf_counter()
        streamer.run(tuple(host_state), None, None, [(0, n, None)], copy_only=True)
        torch.cuda.synchronize(streamer.device)
        best = max(best, 12 * n / (time.perf_counter() - t0) / 1e9)
    out["copy_pipeline_each_way"] = best
    out["copy_pipeline_bytes_each_way"] = 12 * n
    nch = -(-n // c)
    # copies in never land in slot 0, which the copies out read (with two
    # slots they all go to slot 1)
    slots = (streamer.stage[1], streamer.stage[2 if streamer.nbuf > 2 else 1])

    def sweep():
        with torch.cuda.stream(s_in):
            for k in range(nch):
                s0, e0 = k * c, min(n, (k + 1) * c)
                for d, h in zip(slots[k % 2], host_state):
                    d[:e0 - s0].copy_(h[s0:e0], non_blocking=True)
        with torch.cuda.stream(s_out):
            for k in range(nch):
                e0 = min(n, (k + 1) * c) - k * c
                for d, h in zip(a_slot, host_state):
                    h[:e0].copy_(d[:e0], non_blocking=True)

    # the pipeline passed every chunk through the staging slots: slot 0 gets
    # the first chunk again, which the sweep's copies out write back
    for d, h in zip(a_slot, host_state):
        d.copy_(h[:c])
    best = 0.0
    for _ in range(max(1, pipeline_passes)):
        torch.cuda.synchronize(streamer.device)
        t0 = time.perf_counter()
        sweep()
        torch.cuda.synchronize(streamer.device)
        best = max(best, 12 * n / (time.perf_counter() - t0) / 1e9)
    out["sweep_each_way"] = best
    ways = [out["pairs_each_way"], out["copy_pipeline_each_way"], best]
    if lead is not None:
        best = 0.0
        for _ in range(max(1, pipeline_passes)):
            torch.cuda.synchronize(streamer.device)
            t0 = time.perf_counter()
            lead()
            streamer.run(tuple(host_state), None, None, [(0, n, None)], copy_only=True)
            torch.cuda.synchronize(streamer.device)
            best = max(best, 12 * n / (time.perf_counter() - t0) / 1e9)
        out["copy_pipeline_behind_lead_each_way"] = best
        ways.append(best)
    out["both_each_way"] = max(ways)
    return out
