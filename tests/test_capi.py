"""The C-ABI library: it loads, exports every symbol include/elara_amd.h declares, and its host-only entry points
and argument checks behave as documented.  CPU only (no call here reaches the GPU)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from elara_amd import _lib
from oracle import oracle as O

HEADERS = sorted((Path(__file__).resolve().parents[1] / 'include').glob('*.h'))


def declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r'/\*.*?\*/', '', h.read_text(), flags=re.S)
        names |= set(re.findall(r'\b(elr_\w+)\s*\(', text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared()
    assert len(names) >= 7
    for n in names:
        assert hasattr(L, n), n
    assert set(names) <= set(_lib.SIGNATURES), 'binding lacks a signature for a declared entry point'


def test_struct_layouts_match_the_library():
    """Every ctypes mirror of a header struct has the size the library was compiled with (elr_abi_sizes)."""
    out = (ctypes.c_int64 * len(_lib.ABI_STRUCTS))()
    assert _lib.lib().elr_abi_sizes(out, len(out)) == len(out)
    assert list(out) == [ctypes.sizeof(t) for t in _lib.ABI_STRUCTS]


def test_step_exec_checks_and_workspace_size():
    """elr_step_exec_bytes lays out the workspace from the bounds alone; bad bounds and a short workspace are
    rejected on the host."""
    L = _lib.lib()
    a = _lib.ExecArgs()
    a.pv.K, a.upd.D = 3, 64
    assert L.elr_step_exec_bytes(ctypes.byref(a)) > 0                                   # empty step: scratch only
    a.b[1:] = [5, 7, 9, 9, 12, 12, 15, 15, 16, 20]                                      # hits 5, N adm 2, L adm 2, ...
    a.slots.nev = 4
    nb = L.elr_step_exec_bytes(ctypes.byref(a))
    assert nb >= (16 - 5) * 3 * 64 * 4                                                 # the work rows at least
    a.slots.nev = 40
    assert L.elr_step_exec_bytes(ctypes.byref(a)) > nb                                  # more evictions, more bytes
    a.b[3] = 4                                                                           # bounds decrease
    assert L.elr_step_exec_bytes(ctypes.byref(a)) == -1
    o = _lib.ExecOut()
    assert L.elr_step_exec(ctypes.byref(a), ctypes.c_void_p(256), 1 << 30, ctypes.byref(o), None) == -1
    a.b[3] = 9
    assert L.elr_step_exec(ctypes.byref(a), ctypes.c_void_p(256), 10, ctypes.byref(o), None) == -3    # too small
    assert L.elr_step_exec(ctypes.byref(a), ctypes.c_void_p(272), 1 << 30, ctypes.byref(o), None) == -3  # unaligned
    # the device-driven step's optional lookahead mark: its count, last_seen and a 32-bit bit are checked first
    d, do = _lib.StepDevArgs(), _lib.StepDevOut()
    d.mark_rows, d.mark_n, d.mark_nmax, d.mark_bit = 256, None, 10, 1 << 3
    d.plan.last_seen = 256
    assert L.elr_step_dev(ctypes.byref(d), ctypes.c_void_p(256), 1 << 30, ctypes.byref(do), None) == -1  # no count
    d.mark_n, d.mark_bit = 256, 1 << 32
    assert L.elr_step_dev(ctypes.byref(d), ctypes.c_void_p(256), 1 << 30, ctypes.byref(do), None) == -1  # bit > 32b
    d.mark_bit, d.mark_value = 1 << 3, 1 << 31
    assert L.elr_step_dev(ctypes.byref(d), ctypes.c_void_p(256), 1 << 30, ctypes.byref(do), None) == -1  # value
    d.mark_value, d.plan.last_seen = 5, None
    assert L.elr_step_dev(ctypes.byref(d), ctypes.c_void_p(256), 1 << 30, ctypes.byref(do), None) == -1  # last_seen


def test_triton_order_argument_checks():
    """The Triton-order directory calls reject missing release arrays, a short scratch and an unknown step order on
    the host (no call here reaches the GPU: each returns before any launch or has nothing to launch)."""
    L = _lib.lib()
    fake = ctypes.c_void_p(256)          # never dereferenced
    S = _lib.DirState(*([256] * 17), 1)
    P = _lib.DirParams(100, 3, 200, 0, 10, 4, 100, 1)
    sp, pp = ctypes.byref(S), ctypes.byref(P)
    outs = [fake] * 9
    # elr_dir_a_deferred: evictions need rel_cnt
    assert L.elr_dir_a_deferred(sp, pp, None, 0, None, None, 0, fake, 4, 1, *outs, None, fake, 1 << 20, None) == -1
    assert L.elr_dir_evict_deferred(sp, pp, fake, fake, fake, 4, fake, fake, fake, fake, None, fake, 1 << 20,
                                    None) == -1
    assert L.elr_dir_evict_deferred(sp, pp, None, None, None, 0, None, None, None, None, None, None, 0, None) == 0
    # elr_dir_b_release: release items need rows and counts; the scratch covers them
    assert L.elr_dir_b_release(sp, pp, None, None, 0, None, None, 0, 1, None, fake, 5, 1, None, None, fake, 1 << 20,
                               None) == -1
    need = L.elr_dir_scratch_bytes(0, 70_000)
    assert need > L.elr_dir_scratch_bytes(0, 60_000) > 0
    assert L.elr_dir_b_release(sp, pp, None, None, 0, fake, fake, 60_000, 1, fake, fake, 10_000, 1, None, fake,
                               fake, need - 1, None) == -3
    assert L.elr_dir_b_release(sp, pp, None, None, 0, None, None, 0, 1, None, None, 0, 1, None, None, None, 0,
                               None) == 0
    assert L.elr_dir_b_release(sp, pp, None, None, -1, None, None, 0, 1, None, None, 0, 1, None, None, None, 0,
                               None) == -1
    # the step's order flag
    a = _lib.ExecArgs()
    a.pv.K, a.upd.D = 3, 64
    a.b[1:] = [5, 7, 9, 9, 12, 12, 15, 15, 16, 20]
    a.slots.nev = 40
    nb0 = L.elr_step_exec_bytes(ctypes.byref(a))
    a.dir_order = 1
    assert L.elr_step_exec_bytes(ctypes.byref(a)) > nb0          # the deferred release counts
    a.dir_order = 2
    assert L.elr_step_exec_bytes(ctypes.byref(a)) == -1


def test_version_and_errors():
    L = _lib.lib()
    assert L.elr_version() >= 100
    assert b'invalid' in L.elr_error_string(-1)
    with pytest.raises(RuntimeError):
        _lib.check(-1, 'x')


def test_scalars_and_table_match_oracle():
    from elara_amd.ops import adam_scalars
    for hp in [(1e-3, 0.9, 0.999, 1e-8), (5e-2, 0.5, 0.9, 1e-3)]:
        for t in range(0, 3000, 7):
            a = np.array(adam_scalars(*hp, t), np.float32)
            assert np.array_equal(a.view(np.uint32), O.adam_scalars(*hp, t).view(np.uint32))
        tab = np.empty((201, 8), np.float32)
        assert _lib.lib().elr_scalar_table(*hp, 200, tab.ctypes.data_as(ctypes.c_void_p)) == 0
        assert np.array_equal(tab.view(np.uint32), O.scalar_table(*hp, 200).view(np.uint32))


@pytest.mark.parametrize('D,nthreads', [(64, 1), (128, 16), (100, 4), (3, 8)])
def test_cpu_adam_host_entry_point_matches_reference(D, nthreads):
    """elr_cpu_adam (ext().cpu_adam, host memory, no GPU) against the reference's own compiled cpu_adam
    (srm2/csrc/srm2_cpu.cpp:37-56, oracle/_ref) and the oracle, bitwise, over 6 steps with gradients including
    subnormal, huge and signed-zero values; rows outside [0, R) are skipped, and non-contiguous inputs raise as the
    reference's TORCH_CHECK does."""
    import torch
    from elara_amd.ops import ext
    from oracle import ref as REF
    rng = np.random.default_rng(D + nthreads)
    R, n = 3000, 700
    base = rng.standard_normal((R, 3, D)).astype(np.float32) * 0.05
    base[:, 1:] = 0
    ours, orc = torch.from_numpy(base.copy()), base.copy()
    refm = REF.cpu()
    theirs = torch.from_numpy(base.copy())
    HP = (1e-3, 0.9, 0.999, 1e-8)
    for t in range(1, 7):
        rows = rng.choice(R, n, replace=False).astype(np.int64)
        g = (rng.standard_normal((n, D)) * 1e-3).astype(np.float32)
        g[0, :] = 1e-42
        g[1, :] = -0.0
        g[2, :] = 3e30
        rt, gt = torch.from_numpy(rows), torch.from_numpy(g)
        ext().cpu_adam(ours, rt, gt, *HP, t, nthreads)
        O.cpu_adam(orc, rows, g, O.adam_scalars(*HP, t), nthreads)
        if refm is not None:
            refm.cpu_adam(theirs, rt, gt, *HP, t, nthreads)
    assert np.array_equal(ours.numpy().view(np.uint32), orc.view(np.uint32))
    if refm is not None:
        assert torch.equal(ours.view(torch.int32), theirs.view(torch.int32))
    before = ours.clone()
    ext().cpu_adam(ours, torch.tensor([-1, R, R + 5]), torch.ones(3, D), *HP, 7, nthreads)
    assert torch.equal(before, ours)
    with pytest.raises(RuntimeError):
        ext().cpu_adam(ours, torch.arange(4)[::2], torch.ones(2, D), *HP, 7, nthreads)


def test_scalar_recip_is_the_correctly_rounded_double_reciprocal():
    tab = O.scalar_table(1e-3, 0.9, 0.999, 1e-8, 3000)
    r = np.empty((tab.shape[0], 2), np.float64)
    assert _lib.lib().elr_scalar_recip(tab.ctypes.data_as(ctypes.c_void_p), tab.shape[0],
                                       r.ctypes.data_as(ctypes.c_void_p)) == 0
    with np.errstate(divide='ignore'):
        want = 1.0 / tab[:, 5:7].astype(np.float64)
    assert np.array_equal(r, want)
    assert np.isinf(r[0]).all()


def test_host_argument_checks_return_codes():
    L = _lib.lib()
    s = _lib.scalars8([0.0] * 8)
    assert L.elr_adam_rows(None, 0, None, 0, None, -1, 4, s, None) == -1
    assert L.elr_adam_rows(None, 0, None, 0, None, 0, 4, s, None) == 0          # n == 0: no-op
    assert L.elr_adam_rows(None, 0, None, 0, None, 5, 4, s, None) == -1         # null pointers
    assert L.elr_init_rows(None, None, 3, 0, 0, 1.0, None) == -1
    assert L.elr_replay_rows(None, None, None, 0, None, None, None, 1, 4, 9, 0, 1.0, None, None, 0, None) == -2
    assert L.elr_replay_rows(None, None, None, 0, None, None, None, 0, 4, 3, 0, 1.0, None, None, 0, None) == 0


def test_planner_executor_dedup_argument_checks():
    """The entry points of the planner, the fused executor and the dedup plan reject bad arguments on the host,
    before any launch (none of these calls reaches the GPU)."""
    L = _lib.lib()
    fake = ctypes.c_void_p(256)          # never dereferenced: every call below returns before any launch
    assert L.elr_plan_classify(None, None, None, 0, None) == -1
    pin, pout = _lib.PlanIn(), _lib.PlanOut()
    pin.n, pin.nd, pin.nnext, pin.T, pin.K = 0, 0, 0, 1, 3
    pin.toff, pin.kthr, pout.counts = fake.value, fake.value, fake.value
    assert L.elr_plan_classify(ctypes.byref(pin), ctypes.byref(pout), None, 0, None) == -3      # no scratch
    for field, bad in (('n', -1), ('nnext', 5), ('T', 0), ('K', 0)):
        q = _lib.PlanIn.from_buffer_copy(pin)
        setattr(q, field, bad)
        assert L.elr_plan_classify(ctypes.byref(q), ctypes.byref(pout), fake, 1 << 20, None) == -1, field
    q = _lib.PlanIn.from_buffer_copy(pin)
    q.n = 5                                                        # rows but no row pointers
    assert L.elr_plan_classify(ctypes.byref(q), ctypes.byref(pout), fake, 1 << 20, None) == -1
    q = _lib.PlanIn.from_buffer_copy(pin)
    q.next_bits, q.R = fake.value, 0                               # a batch ring needs R
    assert L.elr_plan_classify(ctypes.byref(q), ctypes.byref(pout), fake, 1 << 20, None) == -1
    q.R, q.s, q.next_mask = 100, 33, 0b10                          # the mask holds the step's own bit (33 % 32)
    assert L.elr_plan_classify(ctypes.byref(q), ctypes.byref(pout), fake, 1 << 20, None) == -1
    assert L.elr_plan_scratch_bytes(-1, 0) == -1 and L.elr_plan_scratch_bytes(1000, 10) > 0
    # the classification with the segment sum's partial chunks: either part's bad arguments, before any launch
    assert L.elr_plan_classify_seg(None, None, None, 0, fake, 10, 8, 20, fake, 1 << 20, None) == -1
    assert L.elr_plan_classify_seg(ctypes.byref(pin), ctypes.byref(pout), fake, 1 << 20, fake, 10, 8, 0, fake,
                                   1 << 20, None) == -1                                             # key bits
    assert L.elr_plan_classify_seg(ctypes.byref(pin), ctypes.byref(pout), fake, 1 << 20, fake, 10, 600, 20, fake,
                                   1 << 30, None) == -2                                             # D > 512
    assert L.elr_plan_classify_seg(ctypes.byref(pin), ctypes.byref(pout), fake, 1 << 20, fake, 10, 8, 20, fake, 1,
                                   None) == -3                                                      # plan too small
    assert L.elr_plan_classify_seg(ctypes.byref(pin), ctypes.byref(pout), fake, 1 << 20, None, 10, 8, 20, fake,
                                   1 << 20, None) == -1                                             # no gradients
    adm = [None] * 8
    assert L.elr_plan_admit(None, None, 0, 0, 1, 1, 0, 10, 10, 3, *adm[:7], None) == 0              # nothing to do
    assert L.elr_plan_admit(None, None, 3, 4, 1, 1, 0, 10, 10, 3, *adm[:7], None) == -1             # lazy_n > n
    assert L.elr_plan_admit(None, None, 3, 1, 1, 1, 0, 10, 10, 3, *adm[:7], None) == -1             # null pointers
    sl = _lib.SlotsArgs()
    assert L.elr_plan_admit_slots(None, None, 0, 0, 1, 1, 0, 10, 10, 3, *adm[:7], None) == -1            # no args
    assert L.elr_plan_admit_slots(ctypes.byref(sl), None, 0, 0, 1, 1, 0, 10, 10, 3, *adm[:7], None) == 0  # empty
    sl.n_free, sl.nev = 2, 1
    assert L.elr_plan_admit_slots(ctypes.byref(sl), fake, 4, 0, 1, 1, 0, 10, 10, 3, *adm[:7], None) == -1  # 4 > 3
    assert L.elr_plan_admit_slots(ctypes.byref(sl), fake, 2, 0, 1, 1, 0, 10, 10, 3, *adm[:7], None) == -1  # nulls
    sl.n_free, sl.nev = 8, 4
    assert L.elr_plan_admit_slots(ctypes.byref(sl), None, 0, 0, 1, 1, 0, 10, 10, 3, *adm[:7], None) == -1  # 12 > C
    a = _lib.AssembleArgs()
    a.n, a.D, a.K, a.nseg = 0, 128, 3, 1
    assert L.elr_assemble(None, None) == -1
    assert L.elr_assemble(ctypes.byref(a), None) == 0                                               # n == 0
    a.nseg = 0
    assert L.elr_assemble(ctypes.byref(a), None) == -1
    a.nseg, a.K = 1, 9
    assert L.elr_assemble(ctypes.byref(a), None) == -2                                              # K > 8
    a.K, a.n, a.work, a.rows = 3, 10, fake.value, fake.value
    a.seg_end[0], a.seg_kind[0] = 9, 0
    assert L.elr_assemble(ctypes.byref(a), None) == -1                                              # ends != n
    a.seg_end[0], a.seg_kind[0] = 10, 3
    assert L.elr_assemble(ctypes.byref(a), None) == -1                                              # unknown kind
    a.seg_kind[0] = 1
    assert L.elr_assemble(ctypes.byref(a), None) == -1                                              # replay, no logs
    a.seg_kind[0] = 2
    assert L.elr_assemble(ctypes.byref(a), None) == -1                                              # gather, no MAT
    assert L.elr_dedup_plan_bytes(-1, 1) == -1 and L.elr_dedup_plan_bytes(10, 0) == -1
    assert L.elr_dedup_plan(None, 0, 20, None, None, None, None, 0, 8, None) == 0                   # n == 0
    assert L.elr_dedup_plan(fake, 10, 0, fake, None, fake, fake, 1 << 20, 8, None) == -1            # key bits
    assert L.elr_dedup_plan(fake, 10, 20, fake, None, fake, fake, 1, 8, None) == -3                 # plan too small
    lo = (ctypes.c_int64 * 4)(0, 100, 200, 300)
    F = L.elr_dedup_plan_fields
    assert F(None, 0, 3, lo, 20, None, None, None, None, 0, 8, None) == 0                           # n == 0
    assert F(fake, 2000, 0, lo, 20, fake, None, fake, fake, 1 << 30, 8, None) == -1                 # no fields
    assert F(fake, 2000, 3, None, 20, fake, None, fake, fake, 1 << 30, 8, None) == -1               # no bounds
    assert F(fake, 1 << 30, 3, lo, 20, fake, None, fake, fake, 1 << 30, 8, None) == -1              # n >= 2^31
    assert F(fake, 2000, 3, (ctypes.c_int64 * 4)(0, 100, 50, 300), 20, fake, None, fake, fake, 1 << 30, 8,
             None) == -1                                                                             # descending
    assert F(fake, 2000, 3, (ctypes.c_int64 * 4)(-1, 100, 200, 300), 20, fake, None, fake, fake, 1 << 30, 8,
             None) == -1                                                                             # negative
    assert F(fake, 2000, 3, lo, 20, fake, None, fake, fake, 1, 8, None) == -3                       # plan too small
    assert F(fake, 2000, 3, lo, 20, fake, None, None, fake, 1 << 30, 8, None) == -1                # no count
    assert F(fake, 100, 3, lo, 20, fake, None, fake, fake, 1, 8, None) == -3     # general sort: same checks
    from elara_amd.dedup import field_bounds
    assert field_bounds([0, 5, 5, 9]).dtype == np.int64
    for bad in ([3], [0, 5, 4], [-1, 2], [[0, 1], [2, 3]]):
        with pytest.raises(RuntimeError, match='ascending'):
            field_bounds(bad)
    assert L.elr_segment_sum_plan(fake, 10, 600, 20, fake, 1 << 30, None, fake, 10, None) == -2     # D > 512
    assert L.elr_segment_sum_plan(fake, 10, 8, 20, fake, 1, None, fake, 10, None) == -3             # plan too small
    assert L.elr_segment_sum_plan(fake, 10, 8, 20, fake, 1 << 20, None, fake, -1, None) == -1
    assert L.elr_segment_sum_plan_final(fake, 10, 600, 20, fake, 1 << 30, None, fake, 10, None) == -2
    assert L.elr_segment_sum_plan_final(fake, 10, 8, 20, fake, 1, None, fake, 10, None) == -3
    assert L.elr_segment_sum_plan_final(None, 10, 8, 20, fake, 1 << 20, None, fake, 10, None) == -1
    assert L.elr_mark_rows(None, None, -1, 0, None, 0, None, 0, None) == -1
    assert L.elr_mark_rows(None, None, 0, 0, None, 0, None, 0, None) == 0
    assert L.elr_mark_rows(None, fake, 5, 0, fake, 10, None, 0, None) == -1
    d = ctypes.c_void_p()
    assert L.elr_host_device_ptr(None, ctypes.byref(d)) == -1
    assert L.elr_glog_put(fake, 10, 3, fake, 0, None, fake, 0, 8, None) == 0                       # n == 0
    assert L.elr_glog_put(fake, 10, 0, fake, 0, None, fake, 4, 8, None) == -1                      # K < 1
    assert L.elr_glog_put(fake, 10, 3, None, 0, None, fake, 4, 8, None) == -1                      # no dyn
    assert L.elr_glog_take(fake, 100, fake, fake, 10, 3, fake, 0, 8, None) == 0                    # n == 0
    assert L.elr_glog_take(fake, 100, fake, fake, 0, 3, fake, 4, 8, None) == -1                    # nd < 1
    assert L.elr_glog_take(fake, 100, None, fake, 10, 3, fake, 4, 8, None) == -1                   # no ids
    u = _lib.UpdateArgs()
    u.D, u.K, u.lr, u.b1, u.b2, u.eps, u.step = 128, 3, 1e-3, 0.9, 0.999, 1e-8, 1
    assert L.elr_step_update(None, None) == -1
    assert L.elr_step_update(ctypes.byref(u), None) == 0                                            # empty batch
    q = _lib.UpdateArgs.from_buffer_copy(u)
    q.D = 96                                                                  # any D (the generic kernels), empty
    assert L.elr_step_update(ctypes.byref(q), None) == 0
    for field, bad in (('D', 0), ('K', 0), ('nev', -1), ('lazy_n', 1)):                            # lazy_n > admitted
        q = _lib.UpdateArgs.from_buffer_copy(u)
        setattr(q, field, bad)
        assert L.elr_step_update(ctypes.byref(q), None) == -1, field
    q = _lib.UpdateArgs.from_buffer_copy(u)
    q.b[1:] = [5] + [4] * 9                                                                        # bounds decrease
    assert L.elr_step_update(ctypes.byref(q), None) == -1
    q.b[1:] = [5] * 10                                                                             # 5 hits, no arrays
    assert L.elr_step_update(ctypes.byref(q), None) == -1
    q.grad, q.pool, q.hit_slot = fake.value, fake.value, fake.value
    q.evl = 1                                                                                      # no history record
    assert L.elr_step_update(ctypes.byref(q), None) == -1


def test_ops_raise_without_gpu_tensors():
    import torch
    from elara_amd.ops import gpu_adam
    with pytest.raises(RuntimeError):
        gpu_adam(torch.zeros(4, 3, 8), torch.tensor([0]), torch.zeros(1, 8), 1e-3, 0.9, 0.999, 1e-8, 1)


@pytest.mark.gpu
def test_host_device_ptr_accepts_pinned_and_rejects_pageable(dev):
    """elr_host_device_ptr maps pinned host memory and returns an error (no address) for pageable memory."""
    import torch
    pinned = torch.zeros(1024, pin_memory=True)
    d = ctypes.c_void_p()
    assert _lib.lib().elr_host_device_ptr(ctypes.c_void_p(pinned.data_ptr()), ctypes.byref(d)) == 0 and d.value
    inner = ctypes.c_void_p()
    assert _lib.lib().elr_host_device_ptr(ctypes.c_void_p(pinned[256:].data_ptr()), ctypes.byref(inner)) == 0
    assert inner.value == d.value + 256 * 4
    pageable = torch.zeros(1024)
    bad = ctypes.c_void_p()
    assert _lib.lib().elr_host_device_ptr(ctypes.c_void_p(pageable.data_ptr()), ctypes.byref(bad)) != 0
    assert not bad.value
