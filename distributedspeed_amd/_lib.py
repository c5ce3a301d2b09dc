"""ctypes binding of libdsx.so (C ABI declared in include/dsx.h).

The library is loaded after torch so that its libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded (one runtime per process:
torch's streams and device pointers are then valid in libdsx).

There is no fallback: if libdsx.so is missing or fails to load, every entry
point raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdsx.so")

DSX_F32, DSX_F16, DSX_BF16 = 0, 1, 2
DSX_SCALE_NONE, DSX_SCALE_STATIC, DSX_SCALE_DYNAMIC = 0, 1, 2
DSX_EINVAL = 1
DSX_STATE_ERR_BC_TABLE = 1
DSX_STATE_ERR_GROUPS = 2
DSX_MAX_PARTIALS = 8192
DSX_MAX_GROUPS = 16
DSX_NOALLOC_MAX_PARTIALS = 8192
DSX_NOALLOC_SCRATCH_BYTES = 8 * DSX_NOALLOC_MAX_PARTIALS + 256
ABI_VERSION = 2

_c = ctypes
_P = _c.c_void_p


class DsxState(_c.Structure):
    _fields_ = [("scale", _c.c_float), ("good_steps", _c.c_int32), ("hyst_left", _c.c_int32),
                ("t", _c.c_int32), ("iter", _c.c_int64), ("overflow_count", _c.c_int64),
                ("error", _c.c_int32), ("last_skip", _c.c_int32), ("last_norm", _c.c_double),
                ("clip_once_coef", _c.c_float), ("clip_once", _c.c_int32), ("step_scale", _c.c_float),
                ("step_t2", _c.c_int32)]


class DsxScalerConfig(_c.Structure):
    _fields_ = [("mode", _c.c_int32), ("window", _c.c_int32), ("hysteresis", _c.c_int32),
                ("reserved", _c.c_int32), ("min_scale", _c.c_float), ("growth_factor", _c.c_float),
                ("backoff_factor", _c.c_float), ("reserved2", _c.c_float)]


class DsxAdamwHyper(_c.Structure):
    _fields_ = [(k, _c.c_double) for k in
                ("lr", "beta1", "beta2", "eps", "weight_decay", "max_grad_norm", "clip_eps")]


class DsxStepScalars(_c.Structure):
    _fields_ = [("skip", _c.c_int32), ("t", _c.c_int32)] + \
               [(k, _c.c_float) for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2",
                                          "eps", "bc2s", "nss")] + \
               [("sumsq", _c.c_double), ("norm", _c.c_double)]


class DsxTensorRef(_c.Structure):
    _fields_ = [("master", _P), ("exp_avg", _P), ("exp_avg_sq", _P), ("param16", _P), ("grad", _P),
                ("numel", _c.c_int64), ("group", _c.c_int32), ("reserved", _c.c_int32)]


class DsxChunk(_c.Structure):
    _fields_ = [("tensor", _c.c_int32), ("reserved", _c.c_int32), ("start", _c.c_int64), ("len", _c.c_int64)]


class DsxGroupsDev(_c.Structure):
    _fields_ = [("hyper", DsxAdamwHyper * 16), ("bc_table", _P * 16), ("t_offset", _c.c_int32 * 16),
                ("ngroups", _c.c_int32), ("bc_len", _c.c_int32), ("reserved", _c.c_int64 * 2)]


class DsxFlatPlan(_c.Structure):
    _fields_ = [("master", _P), ("exp_avg", _P), ("exp_avg_sq", _P), ("param16", _P), ("grad", _P),
                ("n", _c.c_int64), ("param_dtype", _c.c_int32), ("grad_dtype", _c.c_int32), ("state", _P),
                ("partials", _P), ("out", _P), ("nparts", _c.c_int32), ("ngroups", _c.c_int32),
                ("scaler", DsxScalerConfig), ("group_end", _c.c_int64 * 16)]


for _s, _n in ((DsxState, 64), (DsxScalerConfig, 32), (DsxAdamwHyper, 56), (DsxStepScalars, 64),
               (DsxTensorRef, 56), (DsxChunk, 24), (DsxGroupsDev, 1112), (DsxFlatPlan, 248)):
    assert _c.sizeof(_s) == _n, (_s.__name__, _c.sizeof(_s))

# name -> (restype, argtypes); every symbol include/dsx.h declares.
SIGNATURES = {
    "dsx_abi_version": (_c.c_int, []),
    "dsx_last_error": (_c.c_char_p, []),
    "dsx_set_tuning_multi": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int]),
    "dsx_set_tuning": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int]),
    "dsx_set_tuning_k2": (_c.c_int, [_c.c_int, _c.c_int]),
    "dsx_set_tuning_k2_chunk": (_c.c_int, [_c.c_int64]),
    "dsx_set_tuning_fold": (_c.c_int, [_c.c_int64]),
    "dsx_copy_unscale_norm": (_c.c_int, [_P, _P, _c.c_int, _c.c_int64, _P, _P, _c.c_int32, _P]),
    "dsx_reduce_segments": (_c.c_int, [_P, _P, _c.c_int32, _P, _P]),
    "dsx_suggest_partials": (_c.c_int32, [_c.c_int64]),
    "dsx_count_chunks": (_c.c_int64, [_P, _c.c_int32, _c.c_int64]),
    "dsx_build_chunks": (_c.c_int64, [_P, _c.c_int32, _c.c_int64, _P, _c.c_int64]),
    "dsx_state_init": (_c.c_int, [_P, _c.c_float, _c.c_int32, _P]),
    "dsx_unscale_norm": (_c.c_int, [_P, _c.c_int, _c.c_int64, _P, _P, _c.c_int32, _P]),
    "dsx_norm_partials": (_c.c_int, [_P, _c.c_int, _c.c_int64, _P, _c.c_double, _P, _c.c_int32, _P]),
    "dsx_norm_partials_multi": (_c.c_int, [_P, _P, _c.c_int64, _c.c_int, _P, _c.c_double, _P, _c.c_int32, _P]),
    "dsx_clip_prepare": (_c.c_int, [_P, _c.c_int32, _c.c_double, _c.c_double, _c.c_double, _P, _P, _P]),
    "dsx_finalize": (_c.c_int, [_P, _c.c_int32, _P, DsxScalerConfig, DsxAdamwHyper, _P, _c.c_int32, _P, _P]),
    "dsx_finalize_groups": (_c.c_int, [_P, _c.c_int32, _P, DsxScalerConfig, _P, _P, _P, _c.c_int32, _c.c_int32,
                                       _P, _P]),
    "dsx_finalize_dev": (_c.c_int, [_P, _c.c_int32, _P, DsxScalerConfig, _P, _c.c_int32, _P, _P]),
    "dsx_groups_upload": (_c.c_int, [_P, _P, _P]),
    "dsx_adamw_flat": (_c.c_int, [_P, _P, _P, _P, _c.c_int, _P, _c.c_int, _c.c_int64, _P, _P]),
    "dsx_traffic_probe_flat": (_c.c_int, [_P, _P, _P, _P, _c.c_int, _P, _c.c_int64, _P]),
    "dsx_zero_step_flat": (_c.c_int, [_P, _P, _P, _P, _c.c_int, _P, _c.c_int, _c.c_int64, _P, DsxScalerConfig,
                                      DsxAdamwHyper, _P, _c.c_int32, _P, _c.c_int32, _P, _P]),
    "dsx_zero_step_plan": (_c.c_int, [_P, _P, _P]),
    "dsx_zero_step_dev": (_c.c_int, [_P, _P, _P]),
    "dsx_zero_step_flat_noalloc": (_c.c_int, [_P, _P, _P, _P, _c.c_int, _P, _c.c_int, _c.c_int64, _P,
                                              DsxScalerConfig, DsxAdamwHyper, _P, _c.c_int32, _c.c_int32, _P, _P]),
    "dsx_unscale_norm_multi": (_c.c_int, [_P, _P, _c.c_int64, _c.c_int, _P, _P, _c.c_int32, _P]),
    "dsx_adamw_multi": (_c.c_int, [_P, _P, _c.c_int64, _c.c_int, _c.c_int, _P, _P]),
    "dsx_zero_step_multi": (_c.c_int, [_P, _P, _c.c_int64, _c.c_int64, _c.c_int, _c.c_int, _P, DsxScalerConfig, _P,
                                       _P, _c.c_int32, _P, _P]),
}

_lib: ctypes.CDLL | None = None


class DsxError(RuntimeError):
    """A libdsx entry point returned a nonzero status."""

    def __init__(self, fn: str, rc: int, msg: str):
        super().__init__(f"{fn} failed (status {rc}): {msg}")
        self.rc = rc


def load(path: str | None = None) -> ctypes.CDLL:
    """Load libdsx.so once; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  -- HIP runtime first (see module docstring)

    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`"
                           " at the repository root (there is no non-HIP fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.dsx_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libdsx ABI {lib.dsx_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().dsx_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> int:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise DsxError(name, rc, last_error())
    return rc
