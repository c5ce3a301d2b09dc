"""The C ABI without a GPU: libdsx.so loads, exports every function
include/dsx.h declares with the layout the Python binding assumes, and its
host-only entry points and argument checks work (no kernel is launched)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsx.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from distributedspeed_amd import _lib
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    from distributedspeed_amd import _lib
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), f"{name} declared in dsx.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_struct_layouts_match_header(lib):
    from distributedspeed_amd import _lib
    text = open(HEADER).read()
    for struct in ("DsxState", "DsxScalerConfig", "DsxAdamwHyper", "DsxStepScalars", "DsxTensorRef", "DsxChunk",
                   "DsxGroupsDev", "DsxFlatPlan"):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = re.findall(r"([A-Za-z_][A-Za-z0-9_\s\*]*?)\s+\*?([a-z0-9_]+)(\[[A-Z0-9_]+\])?\s*;", body)
        cls = getattr(_lib, struct)
        assert [f[1] for f in fields] == [f[0] for f in cls._fields_], struct


def test_abi_version_and_error_string(lib):
    assert lib.dsx_abi_version() == 2
    assert isinstance(lib.dsx_last_error(), bytes)


def test_chunk_table_host_side(lib):
    from distributedspeed_amd import _lib
    sizes = [0, 1, 8, 9, 65536, 65537, 200000]
    arr = (ctypes.c_int64 * len(sizes))(*sizes)
    cnt = lib.dsx_count_chunks(arr, len(sizes), 65536)
    assert cnt == sum(-(-s // 65536) for s in sizes)
    out = (_lib.DsxChunk * cnt)()
    assert lib.dsx_build_chunks(arr, len(sizes), 65536, out, cnt) == cnt
    covered = {}
    for c in out:
        assert 0 < c.len <= 65536 and c.start % 65536 == 0
        covered[c.tensor] = covered.get(c.tensor, 0) + c.len
    assert covered == {i: s for i, s in enumerate(sizes) if s}
    # bad arguments: chunk size not a multiple of 8, too small a buffer
    assert lib.dsx_count_chunks(arr, len(sizes), 100) == -1
    assert lib.dsx_build_chunks(arr, len(sizes), 65536, out, cnt - 1) == -1
    assert b"capacity" in lib.dsx_last_error()


def test_chunk_table_extreme_sizes(lib):
    """Counts and starts near the int64 limit are exact (no intermediate
    overflows), and a total count beyond int64 is refused."""
    from distributedspeed_amd import _lib
    big = 2 ** 63 - 1
    arr = (ctypes.c_int64 * 2)(4096, big)
    ce = 2 ** 63 - 8  # a chunk size whose ceil_div intermediate would overflow
    assert lib.dsx_count_chunks(arr, 2, ce) == 1 + 2
    ce = 2 ** 62
    assert lib.dsx_count_chunks(arr, 2, ce) == 1 + 2
    out = (_lib.DsxChunk * 3)()
    assert lib.dsx_build_chunks(arr, 2, ce, out, 3) == 3
    assert [(c.tensor, c.start, c.len) for c in out] == [(0, 0, 4096), (1, 0, ce), (1, ce, big - ce)]
    many = (ctypes.c_int64 * 8)(*([big] * 8))  # 2^60 chunks each: 7 fit in int64, 8 do not
    assert lib.dsx_count_chunks(many, 7, 8) == 7 * 2 ** 60
    assert lib.dsx_count_chunks(many, 8, 8) == -1
    assert b"overflows" in lib.dsx_last_error()


def test_chunk_table_fuzz(lib):
    """Random and extreme tensor sizes and chunk sizes through
    dsx_count_chunks / dsx_build_chunks (host code only): a table is built
    exactly when it is counted, covers every tensor once in chunks of at most
    chunk_elems, and a buffer one entry short is refused. tests/sanitize runs
    this under ASan/UBSan."""
    import random
    from distributedspeed_amd import _lib
    rnd = random.Random(7)
    I64 = ctypes.c_int64
    for _ in range(3000):
        nt = rnd.choice([0, 1, 2, 5, 17, 100])
        if rnd.random() < 0.8:
            nums = [rnd.choice([0, 1, 7, 8, 4095, 4096, 4097, 65536, rnd.randrange(0, 300000)]) for _ in range(nt)]
        else:
            nums = [rnd.choice([0, -1, 1, 2**40, 2**62, 2**63 - 1, -(2**63)]) for _ in range(nt)]
        ce = rnd.choice([0, 7, 8, 9, 16, 2048, 4096, 65536, 2**40, 2**62, 2**63 - 8])
        arr = (I64 * max(nt, 1))(*nums)
        cnt = lib.dsx_count_chunks(arr, nt, I64(ce))
        bad = ce < 8 or ce % 8 or any(x < 0 for x in nums)
        if bad:
            assert cnt == -1, (nums, ce)
            continue
        assert cnt == sum(-(-x // ce) for x in nums), (nums, ce)
        if cnt > 20000:
            continue
        out = (_lib.DsxChunk * max(cnt + 1, 1))()
        assert lib.dsx_build_chunks(arr, nt, I64(ce), out, I64(cnt + rnd.choice([0, 1]))) == cnt
        tot = [0] * nt
        for k in range(cnt):
            c = out[k]
            assert 0 <= c.tensor < nt and 0 < c.len <= ce and c.start == tot[c.tensor]
            tot[c.tensor] += c.len
        assert tot == nums
        if cnt > 0:
            assert lib.dsx_build_chunks(arr, nt, I64(ce), out, I64(cnt - 1)) == -1


def test_argument_checks_reject_before_launch(lib):
    """Rejected arguments return DSX_EINVAL with a message and never reach a
    HIP call (this runs without a GPU)."""
    from distributedspeed_amd import _lib
    EINVAL = _lib.DSX_EINVAL
    al = 1 << 20  # a 16-byte aligned fake address; never dereferenced on these paths
    sc = _lib.DsxStepScalars()
    # bad grad dtype
    assert lib.dsx_adamw_flat(al, al, al, None, 2, al, 7, 16, ctypes.byref(sc), None) == EINVAL
    assert b"grad dtype" in lib.dsx_last_error()
    # misaligned master
    assert lib.dsx_adamw_flat(al + 4, al, al, None, 2, al, 2, 16, ctypes.byref(sc), None) == EINVAL
    assert b"aligned" in lib.dsx_last_error()
    # negative n
    assert lib.dsx_adamw_flat(al, al, al, None, 2, al, 2, -1, ctypes.byref(sc), None) == EINVAL
    # bad hyper-parameters use torch.optim.Adam's wording
    hp = _lib.DsxAdamwHyper(-1.0, 0.9, 0.999, 1e-8, 0.0, 0.0, 1e-6)
    scfg = _lib.DsxScalerConfig(0, 1000, 1, 0, 1.0, 2.0, 0.5, 0.0)
    assert lib.dsx_finalize(al, 1, al, scfg, hp, al, 1, al, None) == EINVAL
    assert b"Invalid learning rate" in lib.dsx_last_error()
    hp = _lib.DsxAdamwHyper(1e-3, 1.0, 0.999, 1e-8, 0.0, 0.0, 1e-6)
    assert lib.dsx_finalize(al, 1, al, scfg, hp, al, 1, al, None) == EINVAL
    assert b"beta parameter at index 0" in lib.dsx_last_error()
    # bad scaler configuration
    hp = _lib.DsxAdamwHyper(1e-3, 0.9, 0.999, 1e-8, 0.0, 0.0, 1e-6)
    bad = _lib.DsxScalerConfig(2, 0, 1, 0, 1.0, 2.0, 0.5, 0.0)
    assert lib.dsx_finalize(al, 1, al, bad, hp, al, 1, al, None) == EINVAL
    assert b"loss_scale_window" in lib.dsx_last_error()
    # partial count out of range
    assert lib.dsx_unscale_norm(al, 2, 16, al, al, 0, None) == EINVAL
    assert lib.dsx_unscale_norm(al, 2, 16, al, al, _lib.DSX_MAX_PARTIALS + 1, None) == EINVAL
    # the traffic probe: 16-bit grads and params only, param16 required
    assert lib.dsx_traffic_probe_flat(al, al, al, al, 0, al, 16, None) == EINVAL
    assert lib.dsx_traffic_probe_flat(al, al, al, None, 2, al, 16, None) == EINVAL
    assert lib.dsx_traffic_probe_flat(al, al, al, al + 2, 2, al, 16, None) == EINVAL
    assert lib.dsx_traffic_probe_flat(al, al, al, al, 2, al, -1, None) == EINVAL
    # K1 folded into the hand-over copy, and the segment reduce behind it
    assert lib.dsx_copy_unscale_norm(al, al, 7, 16, al, al, 1, None) == EINVAL
    assert lib.dsx_copy_unscale_norm(al, al + 2, 2, 16, al, al, 1, None) == EINVAL
    assert b"aligned" in lib.dsx_last_error()
    assert lib.dsx_copy_unscale_norm(al, al, 2, -1, al, al, 1, None) == EINVAL
    assert lib.dsx_copy_unscale_norm(al, al, 2, 16, None, al, 1, None) == EINVAL
    assert lib.dsx_copy_unscale_norm(al, al, 2, 16, al, al, 0, None) == EINVAL
    assert lib.dsx_reduce_segments(al, al, 0, al, None) == EINVAL
    assert lib.dsx_reduce_segments(al, al, _lib.DSX_MAX_PARTIALS + 1, al, None) == EINVAL
    assert lib.dsx_reduce_segments(None, al, 4, al, None) == EINVAL
    # the graph path's group block: same checks and wording as dsx_finalize_groups
    g = _lib.DsxGroupsDev()
    g.ngroups = 1
    g.bc_len = 4
    g.bc_table[0] = al
    g.hyper[0] = _lib.DsxAdamwHyper(-1.0, 0.9, 0.999, 1e-8, 0.0, 0.0, 1e-6)
    assert lib.dsx_groups_upload(ctypes.byref(g), al, None) == EINVAL
    assert b"Invalid learning rate" in lib.dsx_last_error()
    g.hyper[0].lr = 1e-3
    g.ngroups = 0
    assert lib.dsx_groups_upload(ctypes.byref(g), al, None) == EINVAL
    assert b"ngroups" in lib.dsx_last_error()
    g.ngroups = 1
    g.bc_table[0] = None
    assert lib.dsx_groups_upload(ctypes.byref(g), al, None) == EINVAL
    assert lib.dsx_groups_upload(ctypes.byref(g), al + 4, None) == EINVAL
    # the no-allocation step: partial counts beyond its scratch, negative counts
    hp = _lib.DsxAdamwHyper(1e-3, 0.9, 0.999, 1e-8, 0.0, 0.0, 1e-6)
    assert lib.dsx_zero_step_flat_noalloc(al, al, al, al, 2, al, 2, 16, al, scfg, hp, al, 1,
                                          _lib.DSX_NOALLOC_MAX_PARTIALS + 1, None, None) == EINVAL
    assert b"exceeds the library scratch" in lib.dsx_last_error()
    assert lib.dsx_zero_step_flat_noalloc(al, al, al, al, 2, al, 2, 16, al, scfg, hp, al, 1, -1, None,
                                          None) == EINVAL
    assert lib.dsx_zero_step_flat_noalloc(al + 4, al, al, al, 2, al, 2, 16, al, scfg, hp, al, 1, 0, None,
                                          None) == EINVAL
    assert b"aligned" in lib.dsx_last_error()
    # norms of other types and the one-shot clip: norm_type > 0 (or inf), max_norm >= 0
    for bad in (0.0, -2.0, float("nan"), float("-inf")):
        assert lib.dsx_norm_partials(al, 2, 16, al, bad, al, 1, None) == EINVAL
        assert b"norm_type" in lib.dsx_last_error()
        assert lib.dsx_norm_partials_multi(al, al, 1, 2, al, bad, al, 1, None) == EINVAL
        assert lib.dsx_clip_prepare(al, 1, bad, 1.0, 1e-6, al, al, None) == EINVAL
    assert lib.dsx_norm_partials(al + 2, 2, 16, al, 3.0, al, 1, None) == EINVAL
    assert lib.dsx_norm_partials(al, 2, 16, al, 3.0, al, _lib.DSX_MAX_PARTIALS + 1, None) == EINVAL
    assert lib.dsx_clip_prepare(al, 1, 2.0, -1.0, 1e-6, al, al, None) == EINVAL
    assert b"max_norm" in lib.dsx_last_error()
    assert lib.dsx_clip_prepare(al, 1, 2.0, 1.0, 1e-6, al, None, None) == EINVAL
    # the one-call step: its plan and group block are checked before anything is launched
    plan = _lib.DsxFlatPlan(al, al, al, al, al, 64, 2, 2, al, al, al, 4, 2)
    plan.scaler = scfg
    plan.group_end[0], plan.group_end[1] = 32, 64
    gb = _lib.DsxGroupsDev()
    gb.ngroups, gb.bc_len = 2, 4
    for k in range(2):
        gb.hyper[k] = _lib.DsxAdamwHyper(1e-3, 0.9, 0.999, 1e-8, 0.0, 0.0, 1e-6)
        gb.bc_table[k] = al
    assert lib.dsx_zero_step_plan(None, ctypes.byref(gb), None) == EINVAL
    plan.group_end[0] = 36  # not a multiple of 8
    assert lib.dsx_zero_step_plan(ctypes.byref(plan), ctypes.byref(gb), None) == EINVAL
    assert b"group_end" in lib.dsx_last_error()
    plan.group_end[0], plan.group_end[1] = 32, 60  # the last must end at n
    assert lib.dsx_zero_step_plan(ctypes.byref(plan), ctypes.byref(gb), None) == EINVAL
    plan.group_end[1] = 64
    gb.ngroups = 1
    assert lib.dsx_zero_step_plan(ctypes.byref(plan), ctypes.byref(gb), None) == EINVAL
    assert b"groups" in lib.dsx_last_error()
    gb.ngroups = 2
    gb.hyper[1].lr = -1.0
    assert lib.dsx_zero_step_plan(ctypes.byref(plan), ctypes.byref(gb), None) == EINVAL
    assert b"Invalid learning rate" in lib.dsx_last_error()
    gb.hyper[1].lr = 1e-3
    plan.master = al + 4
    assert lib.dsx_zero_step_plan(ctypes.byref(plan), ctypes.byref(gb), None) == EINVAL
    assert b"aligned" in lib.dsx_last_error()
    # the same plan checks with the group block in device memory
    assert lib.dsx_zero_step_dev(ctypes.byref(plan), al, None) == EINVAL
    assert b"aligned" in lib.dsx_last_error()
    plan.master = al
    assert lib.dsx_zero_step_dev(None, al, None) == EINVAL
    assert lib.dsx_zero_step_dev(ctypes.byref(plan), None, None) == EINVAL
    assert lib.dsx_zero_step_dev(ctypes.byref(plan), al + 4, None) == EINVAL
    plan.group_end[0] = 36
    assert lib.dsx_zero_step_dev(ctypes.byref(plan), al, None) == EINVAL
    assert b"group_end" in lib.dsx_last_error()
    plan.group_end[0] = 32
    # the ragged one-call step
    gb1 = _lib.DsxGroupsDev()
    gb1.ngroups, gb1.bc_len = 1, 4
    gb1.hyper[0] = _lib.DsxAdamwHyper(1e-3, 0.9, 0.999, 1e-8, 0.0, 0.0, 1e-6)
    gb1.bc_table[0] = al
    multi = lambda pdt, gdt, groups, nparts=1: lib.dsx_zero_step_multi(  # noqa: E731
        al, al, 1, 16, pdt, gdt, al, scfg, groups, al, nparts, al, None)
    assert multi(1, 1, None) == EINVAL
    assert multi(0, 1, ctypes.byref(gb1)) == EINVAL and b"param16 dtype" in lib.dsx_last_error()
    assert multi(1, 7, ctypes.byref(gb1)) == EINVAL
    assert multi(1, 1, ctypes.byref(gb1), nparts=0) == EINVAL
    gb1.ngroups = 0
    assert multi(1, 1, ctypes.byref(gb1)) == EINVAL and b"ngroups" in lib.dsx_last_error()
    gb1.ngroups, gb1.hyper[0].eps = 1, -1.0
    assert multi(1, 1, ctypes.byref(gb1)) == EINVAL and b"epsilon" in lib.dsx_last_error()
    # tuning validation
    assert lib.dsx_set_tuning(8, 8, 3, 1) == EINVAL
    assert lib.dsx_set_tuning(0, 8, 4, 1) == EINVAL
    assert lib.dsx_set_tuning(2, -1, 0, 1) == EINVAL and lib.dsx_set_tuning(2, 65, 0, 1) == EINVAL
    assert lib.dsx_set_tuning_k2(-1, 1) == EINVAL and lib.dsx_set_tuning_k2(9, 0) == EINVAL
    assert lib.dsx_set_tuning_k2(0, 2) == EINVAL and lib.dsx_set_tuning_k2(0, -2) == EINVAL
    assert lib.dsx_set_tuning_k2_chunk(-1) == EINVAL and lib.dsx_set_tuning_k2_chunk(1000) == EINVAL
    assert lib.dsx_set_tuning_fold(-1) == EINVAL
    assert lib.dsx_set_tuning_multi(8, 3, 0, 0) == EINVAL
    assert lib.dsx_set_tuning_multi(-1, 1, 0, 0) == EINVAL
    assert lib.dsx_set_tuning_multi(0, 1, 1, 2) == EINVAL


def test_python_layer_mirrors_torch_errors():
    from distributedspeed_amd.flat_step import AdamWHyper, ScalerConfig
    with pytest.raises(ValueError, match="Invalid learning rate"):
        AdamWHyper(lr=-1).validate()
    with pytest.raises(ValueError, match="Invalid beta parameter at index 1"):
        AdamWHyper(beta2=1.0).validate()
    with pytest.raises(ValueError, match="Invalid epsilon"):
        AdamWHyper(eps=-1e-8).validate()
    with pytest.raises(ValueError, match="hysteresis"):
        ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, hysteresis=0).validate()


def test_c_caller_builds_and_checks_its_arguments():
    """The plain C caller of the ABI (tests/c_abi, built by build()) links
    against libdsx.so and the HIP runtime and refuses bad arguments before
    touching a device (its GPU run: tests/test_gpu_c_caller.py)."""
    import subprocess
    exe = os.path.join(ROOT, "tests", "c_abi", "dsx_c_caller")
    assert os.path.exists(exe), "run build(): make -C tests/c_abi"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "usage" in r.stderr
    r = subprocess.run([exe, "0", "1", "4", "/tmp"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "bad arguments" in r.stderr


def test_missing_library_fails_loudly():
    """Without a built libdsx.so the binding raises (there is no CPU or torch
    fallback); run in a fresh process, since a loaded library is cached."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from distributedspeed_amd import _lib\n"
            "try:\n"
            "    _lib.load('/nonexistent/libdsx.so')\n"
            "except RuntimeError as e:\n"
            "    print('raised:', e)\n"
            "    sys.exit(0)\n"
            "sys.exit(1)\n") % ROOT
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "is not built" in r.stdout and "no non-HIP fallback" in r.stdout
