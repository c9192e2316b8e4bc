"""One ELARA training step with every arena in HBM (config C5): the caller of the sparse-update path.

Counterpart of srm2/elara.py ELARAPlanner.plan (209-414, the `cpp` directory path) and ELARAExecutor.assemble /
update (471-542) plus the host worker's writes (544-580), for a single GPU that holds everything:
    - the pool of C resident full states (n0 static hot rows pinned, C - n0 dynamic slots with TTL residency);
    - the MAT arena (full states of materialised rows) and the log arena (gradient-log entries), both in HBM, in
      place of the reference's host arenas (srm2/elara.py:40-103);
    - the state directory (elr_dir_a / elr_dir_b) and the resident histories glog.
Per step: plan (classify the batch's unique rows into hit / N / L / F / S classes, directory call A, admissions,
directory call B), assemble (counter-hash init of N rows, replay of L rows from the log arena, gather of F rows
from MAT), then update (Adam on hits, evictions to MAT or back to the log arena, Adam on N/L rows being admitted or
compacted, log appends, transient Adam of M rows).  The dense model is not part of this path: the caller supplies
the per-occurrence gradients, which are reduced per unique row (dedup + segment sum in ATen's order) as the reference's
embedding backward does (srm2/train.py:352, 429).

Layout.  The planner sorts the batch's unique rows by class rank (hits; admitted N, L, F; appended N, L; compacted
N, L; transient F; S), so each group the executor treats alike is one contiguous range: the fused assembly writes
the non-resident rows' full states into one work array in that order, the segment sum writes the per-row gradients
in that order, and the update is a few Adam calls and row copies over contiguous ranges.  The batch is sorted once
(the dedup plan of `unique`), and the segment sum reuses that sort.

Classification, admissions and assembly are HIP kernels; the remaining glue is a few torch ops per step.  The
plan synchronises with the host once (class counts, elara.py:242), plus once more on the rare overflow path.  The
hot-path kernels come from a backend object (HipBackend: this library's HIP kernels), so the same step can be
driven by another implementation of the kernels (the oracle's) for comparison.
"""
import contextlib
import ctypes
import gc
import time

import torch

from . import _lib  # noqa: F401  (the library must be present)
from .assemble import assemble_rows
from .dedup import field_bounds, plan_bytes, segment_sum_plan, unique_plan, unique_plan_async
from .elara_dir import dir_ext
from .gpu_ops import ScalarTable, init_rows, replay_rows
from .ops import adam_rows_dense, gpu_adam
from .planner import (CNT_BAD, CNT_EXP, CNT_LIVE, CNT_LOG_TOP, CNT_MAT_TOP, CNT_PRE, F_ADMIT, F_NEXT, NCOUNTS,
                      classify_from_flags, plan_admit, plan_admit_slots, plan_classify)
from .rows import copy_rows, glog_put, glog_take, mark_rows

I8, I32, I64 = torch.int8, torch.int32, torch.int64
# classes (srm2/elara.py:31-32): hit, N admitted / append / compact, L admitted / append / compact, F admitted /
# not admitted, S
C_HIT, C_NADM, C_NAPP, C_NCMP, C_LADM, C_LAPP, C_LCMP, C_FADM, C_FNADM, C_S = range(10)
# class ranks: the order of the planner's `order` (elr_plan_classify), which makes the admissions (N, L, F), the
# appends (N, L) and the compactions (N, L) contiguous
R_HIT, R_NADM, R_LADM, R_FADM, R_NAPP, R_LAPP, R_NCMP, R_LCMP, R_FN, R_S = range(10)
RANK_CLASSES = (C_HIT, C_NADM, C_LADM, C_FADM, C_NAPP, C_LAPP, C_NCMP, C_LCMP, C_FNADM, C_S)
ASM_INIT, ASM_REPLAY, ASM_GATHER = 0, 1, 2


def rank_order(cls):
    """Positions sorted stably by class rank, and the inverse (the planner's overflow path)."""
    lut = torch.tensor([RANK_CLASSES.index(c) for c in range(10)], dtype=I8, device=cls.device)
    order = torch.argsort(lut[cls.long()], stable=True)
    rank = torch.empty_like(order)
    rank[order] = torch.arange(order.numel(), device=cls.device)
    return order, rank


class HipBackend:
    """The hot-path kernels of this library (HIP, through the C-ABI)."""

    def __init__(self, D, seed, bound, hp, max_step, device):
        self.D, self.seed, self.bound, self.hp = D, seed, bound, hp
        self.table = ScalarTable(*hp, max_step, device)
        self.dx = dir_ext()
        self._arenas = None
        self._exec = None
        self._dev = {}

    def unique(self, ids, bound=None):
        return unique_plan(ids, self.D, bound)

    def unique_async(self, ids, bound=None, nu_out=None, out=None, fields=None):
        return unique_plan_async(ids, self.D, bound, nu_out, out, fields)

    def plan_bytes(self, n):
        return plan_bytes(n, self.D)

    sync_counts = True   # takes counts_out / nu_out: the plan's counts and the deferred counts in one device buffer

    batch_ring = True   # keeps the planner's ring of loaded batches (ElaraStep.next_bits)

    def mark_rows(self, rows, n_dev, value, out, bits=None, bit=0):
        mark_rows(rows, n_dev, value, out, bits, bit)

    def plan_classify(self, *args, **kw):
        return plan_classify(*args, **kw)

    def plan_admit(self, *args):
        plan_admit(*args)

    def plan_admit_slots(self, *args):
        return plan_admit_slots(*args)

    # the planner's first launch also sums the segment sum's partial chunks (plan_classify(seg=...)); segsum then
    # queues the rest (partials_done)
    seg_in_plan = True

    def segsum(self, g_occ, dplan, U, perm=None, partials_done=False):
        return segment_sum_plan(g_occ, dplan, torch.empty(U, self.D, device=g_occ.device), perm, partials_done)

    def assemble(self, rows, segs, L_ids, L_steps, L_cnt, logs, mat, loc, K):
        return assemble_rows(rows, segs, L_ids, L_steps, L_cnt, logs, mat, loc, K, self.D, self.seed, self.bound,
                             self.table)

    def adam_dense(self, state, grad, s):
        adam_rows_dense(state, grad, *self.hp, s)

    def dir_a(self, st, pv, hs, L_row, L_cnt, ev_slot, s, deferred=False):
        return self.dx.elara_dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s, deferred=deferred)

    def dir_b(self, st, pv, a_rows, a_k, c_rows, c_cnt, s, rel=None):
        return self.dx.elara_dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s, rel=rel)

    def init_rows(self, rows):
        return init_rows(rows, self.D, self.seed, self.bound)

    def replay(self, rows, logs, offs, steps, cnt, K):
        return replay_rows(rows, logs, offs, steps, cnt, self.D, K, self.seed, self.bound, self.table)

    def adam(self, state, slots, grad, s):
        gpu_adam(state, slots, grad, *self.hp, s)

    def copy_rows(self, dst, dst_idx, src, src_idx=None):
        copy_rows(dst, dst_idx, src, src_idx)

    def glog_put(self, glog, dyn, j, g, dyn_off=0):
        glog_put(glog, dyn, j, g, dyn_off)

    def glog_take(self, logs, ids, glog, dyn):
        glog_take(logs, ids, glog, dyn)

    def _arena_ptrs(self, es):
        if self._arenas is None or self._arenas[0] is not es:
            self._arenas = (es, _lib.dptr(es.pool).value, _lib.dptr(es.mat).value, _lib.dptr(es.logs).value,
                            _lib.dptr(es.glog).value)
        return self._arenas[1:]

    def step_exec(self, es, p, G, ev_slot, keep_dyn, u_ord, c_ord, sl_ord, loc_ord, link=None):
        """ElaraStep's calls after the class-count synchronisation -- directory call A, the admissions with the slot
        bookkeeping, call B, the assembly and the update -- in one native call (elr_step_exec), in that order on the
        current stream.  link (host arenas): (stream, start event, done event, event to wait on before the assembly
        or None) -- the update's host-arena writes go to that stream.  Returns the workspace and the offsets of the
        arrays written there."""
        from .elara_dir import _state
        S, P, dev, _ = _state(es.state_list(), es.params())
        pool, mat, logs, glog = self._arena_ptrs(es)
        a = _lib.ExecArgs()
        a.dir, a.pv, a.s = S, P, p.s
        a.b[:] = p.b
        n = p.b[-1]
        for name, t, dt in (('u_ord', u_ord, I64), ('c_ord', c_ord, I64), ('sl_ord', sl_ord, I64),
                            ('loc_ord', loc_ord, I64), ('L_row', p.L_row, I64), ('L_cnt', p.L_cnt, I32)):
            if t.dtype != dt or not t.is_contiguous() or t.device != dev:
                raise RuntimeError(f'step_exec: {name} must be a contiguous {dt} tensor on {dev}')
            setattr(a, name, t.data_ptr())
        if G.dtype != torch.float32 or not G.is_contiguous() or G.numel() != n * self.D:
            raise RuntimeError(f'step_exec: the gradients must be a contiguous float32 [{n}, {self.D}] tensor')
        sl = a.slots
        sl.free_stack, sl.n_free = es._free_buf.data_ptr(), es.n_free
        sl.ev_slot, sl.nev = ev_slot.data_ptr(), ev_slot.numel()
        sl.keep, sl.nkeep = keep_dyn.data_ptr(), keep_dyn.numel()
        sl.dyn_out = es._dyn_buf.data_ptr()
        a.seed, a.bound = int(self.seed) & 0xFFFFFFFF, float(self.bound)
        a.table, a.recip, a.table_rows = self.table.t.data_ptr(), self.table.r.data_ptr(), self.table.t.shape[0]
        u = a.upd
        u.D, u.K = self.D, es.K
        u.pool, u.pool_rows, u.mat, u.mat_rows = pool, es.pool.shape[0], mat, es.mat.shape[0]
        u.logs, u.log_rows, u.glog, u.glog_slots = logs, es.logs.shape[0], glog, es.glog.shape[0]
        u.grad = G.data_ptr()
        u.lr, u.b1, u.b2, u.eps = self.hp
        a.dir_order = 1 if es.dir_impl == 'triton' else 0
        if link is not None:
            lk, start, done, wait = link
            a.link_stream, a.link_start, a.link_done = lk.cuda_stream, start.cuda_event, done.cuda_event
            a.link_wait = wait.cuda_event if wait is not None else None
            u.link_blocks = int(es.link_blocks)
        L = _lib.lib()
        nb = int(L.elr_step_exec_bytes(ctypes.byref(a)))
        _lib.check(min(nb, 0), 'elr_step_exec_bytes')
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        off = _lib.ExecOut()
        with _lib.on_device(dev):
            rc = L.elr_step_exec(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), nb, ctypes.byref(off),
                                 ctypes.c_void_p(_lib.raw_stream(dev)))
        _lib.check(rc, 'elr_step_exec')
        return ws, off

    def step_dev(self, es, s, u, n_dev, g_occ, dplan, mark=None):
        """A whole device-driven step in one native call (elr_step_dev): the plan that resolves the step on the GPU,
        the segment sum in its class order and the rest of the step, every count read on the GPU.  The call's
        arguments are built once per ElaraStep and the workspace kept from step to step, so a step costs the host a
        few field updates and one call.  mark: (rows, count on the device, logical step, bit, event or None), the
        lookahead's mark of a batch loaded ahead, done in the step's compaction launch after the stream waits for
        the event.  Returns (workspace, offsets, sequence number)."""
        st = self._dev.get(id(es))
        if st is None or st['es'] is not es:
            st = self._dev[id(es)] = self._dev_setup(es)
        a, dev = st['args'], es.d
        if not (u.dtype == torch.int64 and u.is_contiguous() and u.device == dev and n_dev.dtype == torch.int64
                and n_dev.device == dev and n_dev.numel() == 1):
            raise RuntimeError('step_dev: u must be a contiguous int64 tensor and n_dev an int64 [1] tensor on '
                               f'{dev}')
        n_occ = dplan.n
        if n_occ and not (g_occ.dtype == torch.float32 and g_occ.is_contiguous() and g_occ.device == dev
                          and g_occ.numel() == n_occ * self.D):
            raise RuntimeError(f'step_dev: the gradients must be a contiguous float32 [{n_occ}, {self.D}] tensor')
        a.plan.u, a.plan.n, a.plan.n_dev = u.data_ptr(), u.numel(), n_dev.data_ptr()
        a.plan.s, a.exec.s = s, s
        a.plan.next_mask = sum(1 << ((s + k) % 32) for k in range(1, es.depth)) & 0xFFFFFFFF
        a.grad = g_occ.data_ptr() if n_occ else None
        a.n_occ, a.key_bits = n_occ, dplan.key_bits
        a.dplan, a.dplan_bytes = (dplan.buf.data_ptr(), dplan.nbytes) if n_occ else (None, 0)
        if mark is None:
            a.mark_rows, a.mark_n, a.mark_nmax, a.mark_value, a.mark_bit, a.mark_event = None, None, 0, 0, 0, None
        else:
            mu, mn, mval, mbit, mev = mark
            if not (mu.dtype == torch.int64 and mu.is_contiguous() and mu.device == dev and mn.dtype == torch.int64
                    and mn.device == dev and mn.numel() == 1):
                raise RuntimeError(f'step_dev: the marked rows must be a contiguous int64 tensor with an int64 [1] '
                                   f'count on {dev}')
            a.mark_rows, a.mark_n, a.mark_nmax = mu.data_ptr(), mn.data_ptr(), mu.numel()
            a.mark_value, a.mark_bit = int(mval), int(mbit)
            a.mark_event = mev.cuda_event if mev is not None else None
        L = _lib.lib()
        nb = int(L.elr_step_dev_bytes(ctypes.byref(a)))
        _lib.check(min(nb, 0), 'elr_step_dev_bytes')
        if st['ws'] is None or st['ws'].numel() < nb:
            st['ws'] = torch.empty(nb, dtype=torch.uint8, device=dev)
        ws = st['ws']
        out = _lib.StepDevOut()
        with _lib.on_device(dev):
            rc = L.elr_step_dev(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), nb, ctypes.byref(out),
                                ctypes.c_void_p(_lib.raw_stream(dev)))
        _lib.check(rc, 'elr_step_dev')
        st['seq'] += 1
        return ws, out, st['seq']

    def _dev_setup(self, es):
        """The device-driven step's call arguments that stay fixed for an ElaraStep: the directory, the residency
        state, the arenas and their bounds (elr_step_dev_args)."""
        from .elara_dir import _state
        S, P, dev, _ = _state(es.state_list(), es.params())
        pool, mat, logs, glog = self._arena_ptrs(es)
        a = _lib.StepDevArgs()
        pin = a.plan
        pin.slot_of, pin.last_seen, pin.code = es.slot_of.data_ptr(), es.last_seen.data_ptr(), es.code.data_ptr()
        pin.kthr, pin.toff, pin.T = es.kthr.data_ptr(), es.toff.data_ptr(), es.toff.numel()
        pin.dyn, pin.nd, pin.slot_row = es._dyn_buf.data_ptr(), es._dyn_buf.numel(), es.slot_row.data_ptr()
        pin.mat_top, pin.log_top, pin.live = es.mat_top.data_ptr(), es.log_top.data_ptr(), es.live.data_ptr()
        pin.K, pin.want_t = es.K, int(es.st_mode == 'T')
        pin.loc, pin.R = es.loc.data_ptr(), es.R
        pin.next_bits = es.next_bits.data_ptr()
        pin.carry = int(es.dyn == 'carry')
        pin.nd_dev = es._ctl_state[_lib.S_ND:_lib.S_ND + 1].data_ptr()
        c = a.ctl
        c.state, c.desc = es._ctl_state.data_ptr(), es._desc.data_ptr()
        c.mat_cap, c.log_cap, c.triton = es.mat_cap - 1, es.log_cap, int(es.dir_impl == 'triton')
        e = a.exec
        e.dir, e.pv = S, P
        sl = e.slots
        sl.free_stack, sl.n_free = es._free_buf.data_ptr(), es.C - es.n0
        sl.nev, sl.nkeep = es.Cdyn, es.Cdyn
        sl.dyn_out = es._dyn_buf.data_ptr()
        e.seed, e.bound = int(self.seed) & 0xFFFFFFFF, float(self.bound)
        e.table, e.recip, e.table_rows = self.table.t.data_ptr(), self.table.r.data_ptr(), self.table.t.shape[0]
        up = e.upd
        up.D, up.K = self.D, es.K
        up.pool, up.pool_rows, up.mat, up.mat_rows = pool, es.pool.shape[0], mat, es.mat.shape[0]
        up.logs, up.log_rows, up.glog, up.glog_slots = logs, es.logs.shape[0], glog, es.glog.shape[0]
        up.lr, up.b1, up.b2, up.eps = self.hp
        e.dir_order = 1 if es.dir_impl == 'triton' else 0
        return {'es': es, 'args': a, 'ws': None, 'seq': 0}

    def step_update(self, es, p, G, part=0):
        """ElaraStep.update in one native call (elr_step_update): the same launches in the same order, issued from
        C++ with no per-launch Python work.  part: 0 all, 1 the device part, 2 the link part (ELR_UPDATE_*)."""
        pool, mat, logs, glog = self._arena_ptrs(es)
        b = p.b
        nh, nev = b[R_HIT + 1] - b[R_HIT], p.ev_slot.numel()
        a = _lib.UpdateArgs(
            self.D, es.K, pool, es.pool.shape[0], mat, es.mat.shape[0], logs, es.logs.shape[0], glog,
            es.glog.shape[0], _p64(G, b[-1] * self.D, torch.float32), _p64(p.work, (b[R_S] - b[R_NADM]) * 3 * self.D,
                                                                        torch.float32),
            (_lib.c_i64 * 11)(*b), p.s, *self.hp, int(bool(p.evl)),
            _p64(p.hit_slot, nh), _p64(p.hrec_dyn, nh) if p.evl else 0, _p64(p.hrec_j, nh) if p.evl else 0,
            nev, _p64(p.ev_slot, nev), _p64(p.evf_slots, nev), _p64(p.evl_ids, nev * es.K), _p64(p.ev_dyn, nev),
            _p64(p.adm_slots, b[R_FADM + 1] - b[R_NADM]), p.lazy_n, es.n0,
            _p64(p.c_slots, b[R_LCMP + 1] - b[R_NCMP]), _p64(p.a_ids, b[R_LAPP + 1] - b[R_NAPP]),
            _p64(p.FN_slot, b[R_FN + 1] - b[R_FN]), _p64(p.S_slot, b[R_S + 1] - b[R_S]), int(part),
            int(es.link_blocks) if part == 2 else 0)
        with _lib.on_device(G.device):
            rc = _lib.lib().elr_step_update(ctypes.byref(a), ctypes.c_void_p(_lib.raw_stream(G.device)))
        _lib.check(rc, 'elr_step_update')


def _p64(t, n, dtype=torch.int64):
    """Address of a contiguous tensor of the given dtype on the GPU holding n elements (0 when n == 0)."""
    if n == 0:
        return 0
    if t.dtype != dtype or not t.is_contiguous() or t.numel() != n or not t.is_cuda:
        raise RuntimeError(f'step_update: expected a contiguous cuda {dtype} tensor of {n} elements, got '
                           f'{tuple(t.shape)} {t.dtype} {t.device}')
    return t.data_ptr()


class Plan:
    """One step's plan.  With the native executor (HipBackend.step_exec) the arrays it writes -- the directory calls'
    outputs, the admitted slots, the work rows -- live in its workspace and become tensors on first access."""

    # name: (field of elr_exec_out, dtype, shape keys)
    _VIEWS = {'L_steps': ('L_steps', I32, ('nL', 'K')), 'L_ids': ('L_ids', I32, ('nL', 'K')),
              'hrec_dyn': ('hrec_dyn', I64, ('nh',)), 'hrec_j': ('hrec_j', I64, ('nh',)),
              'ev_row': ('ev_row', I64, ('nev',)), 'ev_rep': ('rep', torch.bool, ('nev',)),
              'evl_ids': ('evl_ids', I64, ('nev', 'K')), 'evf_slots': ('evf_slots', I64, ('nev',)),
              'ev_dyn': ('ev_dyn', I64, ('nev',)), 'adm_slots': ('adm_slots', I64, ('n_adm',)),
              'a_ids': ('a_ids', I64, ('na',)), 'c_slots': ('c_slots', I64, ('nc',)),
              'work': ('work', torch.float32, ('nw', 3, 'D'))}

    def __getattr__(self, name):
        d = self.__dict__
        if '_doff' in d and '_dims' not in d and not name.startswith('__'):
            self._resolve_dev()   # a device-driven step's plan: its counts are read now (a synchronisation)
            return getattr(self, name)
        if '_ws' not in d or name not in Plan._VIEWS and name not in ('FN_slot', 'S_slot', 'adm_rec_slot'):
            raise AttributeError(name)
        if name in ('FN_slot', 'S_slot'):
            b, r = self.b, R_FN if name == 'FN_slot' else R_S
            v = d['_loc_ord'][b[r]:b[r + 1]]
        elif name == 'adm_rec_slot':
            if not (self.lazy_n and self.evl):
                raise AttributeError(name)
            v = self.adm_slots[:self.lazy_n]
        else:
            field, dt, shape = Plan._VIEWS[name]
            dims = [x if isinstance(x, int) else d['_dims'][x] for x in shape]
            n = 1
            for x in dims:
                n *= x
            o = getattr(d['_off'], field)
            v = d['_ws'][o:o + n * _lib.ESIZE[dt]].view(dt).view(*dims)
        setattr(self, name, v)
        return v

    def _resolve_dev(self):
        """The counts and arrays of a device-driven step's plan, from its descriptor and the outputs the step left in
        its workspace: the same attributes a host-planned step has (a host synchronisation)."""
        d = self.__dict__
        es, ws, off = d['_es'], d['_ws'], d['_doff']
        if d['_seq'] != es.be._dev[id(es)]['seq']:
            raise RuntimeError(f'the plan of step {d["s"]} is no longer readable: a later step has reused its '
                               'workspace (read a device-driven plan before the next step)')
        desc = es._desc.tolist()
        b = desc[_lib.D_B:_lib.D_B + 11]
        counts = [0] * 10
        for r, cl in enumerate(RANK_CLASSES):
            counts[cl] = b[r + 1] - b[r]
        nNa, nNp, nNc, nLa, nLp, nLc = counts[1:7]
        nev, n = desc[_lib.D_NEV], desc[_lib.D_NROWS]

        def arr(field, dt, m):
            o = getattr(off, field)
            return ws[o:o + m * _lib.ESIZE[dt]].view(dt)
        self.b, self.counts, self.n = b, counts, n
        self.nL = (nLa, nLp, nLc)
        self.lazy_n = desc[_lib.D_LAZY]
        self.skipped = bool(desc[_lib.D_SKIP])
        self.overflowed = desc[_lib.D_OVERFLOW] > 0
        self.barrier = bool(desc[_lib.D_BARRIER])
        self.preempted = desc[_lib.D_TAKE]
        self.order, self.rank, self.u_ord = arr('order', I64, n), arr('rank', I64, n), arr('u_ord', I64, n)
        self.ev_slot = arr('dyn_out', I64, nev)
        self.hit_slot = arr('sl_ord', I64, b[R_HIT + 1])
        nL = nLa + nLp + nLc
        self.L_row, self.L_cnt = arr('L_row', I64, nL), arr('L_cnt', I32, nL)
        self.G = arr('grad_rows', torch.float32, n * es.D).view(n, es.D)
        d['_loc_ord'] = arr('loc_ord', I64, n)
        eo = off.exec_ws
        d['_off'] = _lib.ExecOut(*[getattr(off.exec, f) + eo for f in _lib.EXEC_OUT_FIELDS])
        d['_dims'] = dict(nL=nL, K=es.K, nh=b[R_HIT + 1], nev=nev, n_adm=desc[_lib.D_NADM], na=nNp + nLp,
                          nc=nNc + nLc, nw=b[R_S] - b[R_NADM], D=es.D)


class HostBudgetExceeded(RuntimeError):
    """The capacity-tier arenas would exceed the enforced host budget (srm2/store.py:26-27): raised by the plan of
    the step whose allocations cross it, after that plan's directory calls and before its update."""


CHUNK = 64 << 20   # fault granularity of the capacity-tier accounting, in bytes (srm2/store.py:23)


class ElaraStep:
    """Planner + executor of ELARA over HBM-resident arenas.

    toff: first row of each table (int64 [T]); R total rows; D width; C pool slots; static_rows: pinned hot rows
    (the `static` base, srm2/train.py:262-270) or None; K = Kmax; kthr: materialisation threshold per table (or one
    int); evl: the residency-aware representation (evicted rows may return to L; srm2/elara.py:110-116): 0 or False
    off, 1 or True on, 2 gated by memory pressure (switched on, once, by the first plan that finds the arenas'
    used bytes (3 mat_top + live) * D * 4 at or above evl_gate_frac of host_budget; never on without a budget);
    dyn: dynamic residency 'ttl' (admitted when the row recurs within the lookahead, kept while it does) or
    'carry' (admitted when it appears in the next depth-1 batches, evicted as soon as it does not;
    srm2/elara.py:221, 231-233); L: TTL lookahead; depth: number of batches u_nexts covers plus one
    (srm2/train.py:366); st_mode 'T' (transient full-state updates on the GPU) or 'S' (materialised cold rows
    updated in the MAT arena); log_cap / mat_cap: arena capacities in rows (row log_cap of the log arena and row
    mat_cap - 1 of the MAT arena are trash rows); host_arenas: keep the MAT and log arenas in pinned host memory
    (the capacity tier, srm2/elara.py:40-103), whose writes go to a link stream unless link_stream is False;
    sync_free: the device-driven step where it applies (no link stream, no host budget, the ring of loaded
    batches); host_budget: bytes the arenas may hold, accounted as the
    reference's ArenaStore does (faulted in chunks of budget_chunk bytes up to each arena's top; 0: no budget),
    HostBudgetExceeded when a step would pass it (srm2/elara.py:63-81); dir_impl: the log-id allocation order of
    the reference directory it stands in for (srm2/elara.py:150-155, srm2/train.py:133): 'cpp' (the default) or
    'ref', equal, or 'triton', which allocates every log id of a step before any release (srm2/elara_kernels.py);
    the other states are the same under all three.  field_layout: every batch that run() loads is laid out by table,
    as the reference's one-hot batches are (srm2/train.py:187-214): (sample, table) order, with table t's column
    holding rows [toff[t], toff[t + 1]) (toff[T] = R); its dedup plan then sorts each table's column on its own
    (dedup.unique_plan_async(fields=...)), the same plan in three launches.  A row outside its table's range is then
    reported as a row outside [0, R).
    """

    def __init__(self, toff, R, D, C, static_rows=None, K=3, kthr=3, evl=True, L=8, depth=3, st_mode='T', seed=42,
                 bound=0.01, hp=(1e-3, 0.9, 0.999, 1e-8), max_step=1000, log_cap=None, mat_cap=None, device='cuda',
                 backend=None, host_arenas=False, dyn='ttl', evl_gate_frac=0.75, host_budget=0, budget_chunk=CHUNK,
                 dir_impl='cpp', sync_free=True, link_stream=None, field_layout=False):
        d = torch.device(device)
        if dir_impl not in ('cpp', 'ref', 'triton'):
            raise ValueError(f"dir_impl must be 'cpp', 'ref' or 'triton' (got {dir_impl!r})")
        self.dir_impl = dir_impl
        self.d, self.R, self.D, self.C, self.K, self.L, self.depth = d, R, D, C, K, L, depth
        self.MAT = K + 1
        self.st_mode = st_mode
        if dyn not in ('ttl', 'carry') or st_mode not in ('S', 'T'):
            raise ValueError(f'dyn must be ttl or carry and st_mode S or T (got {dyn!r}, {st_mode!r})')
        self.dyn = dyn
        self.evl_mode = int(evl)
        if self.evl_mode not in (0, 1, 2):
            raise ValueError(f'evl must be 0, 1 or 2 (got {evl!r})')
        self.evl = self.evl_mode == 1
        self.evl_gate_frac = float(evl_gate_frac)
        self.host_budget = int(host_budget)
        self.budget_chunk = int(budget_chunk)
        self.faulted = {'mat': 0, 'log': 0}   # arena rows the budget accounting holds (ArenaStore.faulted)
        self._observed = 0   # highest logical step whose batch has been observed (the lookahead)
        self.hp = hp
        self.be = backend or HipBackend(D, seed, bound, hp, max_step, d)
        self.toff = torch.as_tensor(toff, dtype=I64).to(d)
        T = self.toff.numel()
        # batches laid out by table ((sample, table) order, table t's column holding its rows): sorted per table
        self.field_bounds = (field_bounds(torch.cat([self.toff.cpu(), torch.tensor([R], dtype=I64)]).numpy())
                             if field_layout else None)
        self.kthr = (torch.full((T,), int(kthr), dtype=I8) if isinstance(kthr, int)
                     else torch.as_tensor(kthr, dtype=I8)).to(d)
        self.log_cap = int(log_cap or 2 * R)
        self.mat_cap = int(mat_cap or R + 1)
        # ---- state directory (srm2/elara.py:117-125) ----
        self.code = torch.zeros(R, dtype=I8, device=d)
        self.loc = torch.full((R + 1,), -1, dtype=I32, device=d)
        self.ent = torch.full(((R + 1) * K,), -1, dtype=I32, device=d)
        self.lstep = torch.zeros(self.log_cap + 1, dtype=I32, device=d)
        self.lfree = torch.zeros(self.log_cap + 1, dtype=I32, device=d)
        self.n_lfree, self.log_top, self.mat_top, self.live = (torch.zeros(1, dtype=I64, device=d) for _ in range(4))
        # ---- residency (srm2/elara.py:128-146) ----
        self.slot_of = torch.full((R,), -1, dtype=I32, device=d)
        self.slot_row = torch.full((C,), -1, dtype=I64, device=d)
        self.pinned = torch.zeros(C, dtype=torch.bool, device=d)
        self.last_seen = torch.full((R,), -1, dtype=I32, device=d)
        # ring of loaded batches for the planner's "appears in the next batches" test (bit t % 32 of next_bits[r]
        # set while the batch of logical step t holds row r): one load per row instead of searches of the next
        # batches' unique rows.  The L + 1 batches loaded ahead and the current one must fit in 32 bits.
        self.next_bits = (torch.zeros(R, dtype=I32, device=d)
                          if getattr(self.be, 'batch_ring', False) and d.type == 'cuda' and L + 2 <= 32 else None)
        n0 = 0
        self.static_rows = None
        if static_rows is not None and len(static_rows):
            sr = torch.as_tensor(static_rows, dtype=I64).to(d)
            n0 = sr.numel()
            assert n0 <= C
            self.slot_of[sr] = torch.arange(n0, dtype=I32, device=d)
            self.slot_row[:n0] = sr
            self.pinned[:n0] = True
            self.static_rows = sr
        self.n0, self.Cdyn = n0, C - n0
        self.free = torch.arange(C - 1, n0 - 1, -1, dtype=I64, device=d)
        self.n_free = C - n0
        self.dyn_slots = torch.empty(0, dtype=I64, device=d)
        # with a backend that keeps the free stack and the dynamic slot list in place (plan_admit_slots), their
        # storage: the stack holds at most C entries, the slot list at most C - n0
        self._slots_in_place = getattr(self.be, 'plan_admit_slots', None) is not None
        if self._slots_in_place:
            self._free_buf = torch.empty(C, dtype=I64, device=d)
            self._free_buf[:C - n0] = self.free
            self.free = self._free_buf[:C - n0]
            self._dyn_buf = torch.empty(max(C - n0, 1), dtype=I64, device=d)
            self.dyn_slots = self._dyn_buf[:0]
        self.adm_c0 = torch.full((C,), -1, dtype=I8, device=d)
        self.rj = torch.zeros(C, dtype=I8, device=d)
        self.rok = torch.zeros(C, dtype=I8, device=d)
        self.pstep = torch.zeros(self.Cdyn + 1, K, dtype=I32, device=d)
        self.mat_trash = R
        # ---- arenas (HBM) ----
        self.pool = torch.zeros(C, 3, D, device=d)
        self.glog = torch.zeros(self.Cdyn + 1, K, D, device=d)
        # the capacity tier: with host_arenas the MAT and log arenas live in pinned host memory, which the kernels
        # read and write directly over the host link (no staging copies, no host-side arithmetic)
        ad = dict(device='cpu', pin_memory=True) if host_arenas and d.type == 'cuda' else dict(device=d)
        self.host_arenas = bool(host_arenas and d.type == 'cuda')
        self.mat = torch.empty(self.mat_cap, 3, D, **ad)
        self.logs = torch.empty(self.log_cap + 1, D, **ad)
        # with host arenas and link_stream, the update's writes into them (compacted and transient rows into MAT,
        # log appends, S rows) run on a second stream of default priority while the next step plans and assembles,
        # so the host link carries both directions at once (update writes, assembly reads).  The next assembly that
        # might read those rows waits for them: the one two steps later, or the next one if the step overflowed (an
        # un-admitted row of batch s can reappear in batch s + 1; otherwise a row of batch s + 1 is a hit or admitted
        # in step s, and the rows the link part writes are neither)
        # (link_stream None: on with host arenas; False: the host-arena step runs as the HBM one does, on one
        # stream -- device-driven when nothing else needs the host)
        if link_stream is None:
            link_stream = self.host_arenas
        self._link = (torch.cuda.Stream(device=d) if link_stream and self.host_arenas
                      and getattr(self.be, 'step_update', None) else None)
        self._link_pending = []
        self._link_start = None
        if self._link is not None:
            self._link_start = torch.cuda.Event()
            self._link_start.record(self._link)   # creates the event the native step records on its stream
        self.link_blocks = 64   # blocks per launch of the link part (measured best of 32-128 at C5 with host arenas)
        self._stats = {k: 0 for k in ('adm', 'ev', 'hits', 'N', 'L', 'F', 'S', 'overflow', 'preempt',
                                     'compactions', 'appends', 'syncs', 'barriers')}
        self.wait_s = 0.0   # host time spent waiting for the GPU at the plans' synchronisations
        self._deferred = []
        self._pin = None
        # one device buffer for everything a plan's synchronisation reads: the class counts in [0, NCOUNTS), the
        # unique counts of batches loaded ahead in a ring after them (each read at the next synchronisation), so
        # the read is a single copy with no gathering kernel
        sync = d.type == 'cuda' and getattr(self.be, 'sync_counts', False)
        self._sync = torch.zeros(64, dtype=I64, device=d) if sync else None
        self._sync_next = NCOUNTS
        self.dedup_ahead = True   # run() sorts the batches loaded ahead on a second stream (dedup_stream)
        self._side = None
        self._plan_pool = None   # run()'s reusable dedup-plan buffers (PlanPool), made on first use
        # run(), device-driven with the dedup on a second stream: each batch loaded ahead is marked (the lookahead) in
        # the launch of the previous step's directory compaction instead of a launch of its own between the steps
        self.fold_mark = True
        self._pending_mark = None
        if self.static_rows is not None:   # srm2/elara.py:434-440 load_static: pinned rows' state lives in the pool
            self.pool[:n0] = self.be.init_rows(self.static_rows)
            self.code[self.static_rows] = self.MAT
        # the device-driven step: the plan's counts stay on the GPU (elr_step_dev: the plan resolves the step there
        # and the executor reads the resolution), so the host never waits for a step.  Taken when the backend has
        # it and nothing needs the host between the plan and the update: no link stream (its ordering is kept by
        # the host), no host budget (its accounting reads the arenas' tops), the ring of loaded batches (the next
        # batches are not needed as lists).  Host arenas are reached by the same kernels in place.
        self.sync_free = bool(sync_free and getattr(self.be, 'step_dev', None) is not None
                              and self._slots_in_place and self._sync is not None and self.next_bits is not None
                              and self._link is None and self.host_budget == 0)
        self._ctl_state = None
        self._err_poll = None
        self._polls = 0
        if self.sync_free:
            self._ctl_state = torch.zeros(_lib.CTL_WORDS, dtype=I64, device=d)
            self._ctl_state[_lib.S_NFREE] = C - n0
            self._desc = torch.zeros(_lib.DESC_WORDS, dtype=I64, device=d)
            self._err_pin = torch.zeros(1, dtype=I64, pin_memory=True)
        if d.type == 'cuda':
            # the end of every run() reads the arenas' tops (check_capacity, through torch's stack kernel); reading
            # them once here loads that kernel, whose first load in a process (10-20 ms) would otherwise fall at
            # the end of the first run's steps
            self._host(self.mat_top, self.log_top)
            self._stats['syncs'] -= 1

    @property
    def stats(self):
        """Per-run counts (srm2/elara.py's planner stats): admitted, evicted, hits, N, L, F, S rows, overflow,
        preempted, compactions, appends, barriers, and 'syncs', the host synchronisations of the plans.  In the
        device-driven step the row counts accumulate on the GPU: reading them is a synchronisation (not counted)."""
        if self._ctl_state is None:
            return self._stats
        out = dict(self._stats)
        vals = self._ctl_state[_lib.S_STATS:_lib.S_STATS + len(_lib.STAT_KEYS)].tolist()
        for k, v in zip(_lib.STAT_KEYS, vals):
            if k in out:
                out[k] = v
        return out

    # ---- helpers ----
    def state_list(self):
        return [self.code, self.loc, self.ent, self.lstep, self.lfree, self.n_lfree, self.log_top, self.mat_top,
                self.live, self.adm_c0, self.rj, self.pstep, self.kthr, self.toff, self.slot_of, self.slot_row,
                self.rok]

    def params(self):
        return [self.R, self.K, self.log_cap, self.n0, self.Cdyn, self.MAT, self.mat_trash, int(self.evl)]

    def check_errors(self):
        """The device-driven step's errors, read from its control state (a host synchronisation): ValueError for a
        batch with rows outside [0, R), RuntimeError for a step that could allocate past an arena.  The step that
        hit the error and every later one did nothing.  Also brings the host's view of the free stack and the
        dynamic slot list up to date."""
        if self._ctl_state is None:
            return
        st = self._ctl_state.tolist()
        nf, nd = st[_lib.S_NFREE], st[_lib.S_ND]
        self.n_free, self.free = nf, self._free_buf[:nf]
        self.dyn_slots = self._dyn_buf[:nd]
        err, s_err = st[_lib.S_ERR], st[_lib.S_ERR_STEP]
        if err & _lib.STEP_ERR_ROWS:
            raise ValueError(f'step {s_err}: {st[_lib.S_ERR_A]} rows of the batch lie outside [0, {self.R})')
        if err & _lib.STEP_ERR_CAPACITY:
            raise RuntimeError(f'arena capacity: step {s_err} may allocate up to MAT row {st[_lib.S_ERR_B]} (capacity '
                               f'{self.mat_cap - 1}) and log entry {st[_lib.S_ERR_C]} (capacity {self.log_cap})')

    POLL_EVERY = 16   # device-driven steps between two looks at the error word

    def _poll_errors(self):
        """Raise a device-driven step's error soon after the host can see it, without waiting: every POLL_EVERY
        steps the error word is copied to pinned memory behind the step's work, and looked at once that copy has
        completed.  (A step with an error and every later one do nothing on the GPU, so raising late changes no
        state; the end of a run reads the word in any case.)"""
        self._polls += 1
        if self._polls % self.POLL_EVERY:
            return
        ev = self._err_poll
        if ev is not None:
            if not ev.query():
                return
            if int(self._err_pin[0]):
                self.check_errors()
        self._err_pin.copy_(self._ctl_state[_lib.S_ERR:_lib.S_ERR + 1], non_blocking=True)
        self._err_poll = torch.cuda.Event()
        self._err_poll.record()

    def check_capacity(self):
        """Raise if an allocation ran past the MAT or log arena (rows beyond capacity are not written)."""
        self.check_errors()
        mt, lt = self._host(self.mat_top, self.log_top)
        if mt > self.mat_cap - 1 or lt > self.log_cap:
            raise RuntimeError(f'arena capacity exceeded (MAT {mt}/{self.mat_cap - 1}, logs {lt}/{self.log_cap})')

    def _wait_link(self, due):
        """Make the current stream wait for the pending link-stream updates (s, event, link_next) for which
        due(s, link_next) holds (link_next: the plan's flag that the next step's rows may be among them)."""
        keep = []
        cur = torch.cuda.current_stream(self.d) if self._link_pending else None
        for s_ev, ev, nxt in self._link_pending:
            if due(s_ev, nxt):
                cur.wait_event(ev)
            else:
                keep.append((s_ev, ev, nxt))
        self._link_pending = keep

    def _link_args(self, p):
        """The link-stream arguments of a native step with host arenas: the done event it records, and the event its
        assembly waits for -- the latest pending link update the assembly may read (the rule of assemble), whose
        predecessors on the link stream are then done too."""
        wait, keep = None, []
        for s_ev, ev, nxt in self._link_pending:
            if s_ev <= p.s - 2 or (s_ev == p.s - 1 and nxt):
                wait = ev
            else:
                keep.append((s_ev, ev, nxt))
        self._link_pending = keep
        done = torch.cuda.Event()
        done.record(self._link)   # creates the event; the step records it again after its link launches
        return self._link, self._link_start, done, wait

    def join_link(self):
        """Make the current stream wait for every pending link-stream update (before reading the arenas)."""
        self._wait_link(lambda s_ev, nxt: True)

    def observe(self, step, u, n_dev=None):
        """Record that rows u appear at logical step `step` (the TTL lookahead, srm2/elara.py:160-161); with n_dev
        (a device count) only the first n_dev rows of u, without a synchronisation."""
        self._observed = max(self._observed, int(step))
        bit = 1 << (step % 32)
        if n_dev is None:
            if u.device.type == 'cpu' and u.numel() and (int(u.min()) < 0 or int(u.max()) >= self.R):
                raise ValueError(f'step {step}: rows of the batch lie outside [0, {self.R})')
            self.last_seen[u] = step
            if self.next_bits is not None:
                self.next_bits[u] = self.next_bits[u] | (bit - (1 << 32) if bit >= 1 << 31 else bit)
        elif self.next_bits is not None:
            self.be.mark_rows(u, n_dev, step, self.last_seen, self.next_bits, bit)
        else:
            self.be.mark_rows(u, n_dev, step, self.last_seen)

    def observe_in_next_step(self, step, u, n_dev, event=None):
        """observe(step, u, n_dev) done by the next device-driven step's native call, in the launch of its directory
        compaction -- after that step's plan has read the lookahead and before the following step's plan -- once the
        stream has waited for `event` (recorded after u's dedup plan on another stream)."""
        if not self.sync_free or self.next_bits is None:
            raise RuntimeError('observe_in_next_step needs the device-driven step')
        if self._pending_mark is not None:
            raise RuntimeError('a batch is already waiting to be marked by the next step')
        self._observed = max(self._observed, int(step))
        self._pending_mark = (u, n_dev, int(step), 1 << (step % 32), event)

    def defer_count(self, t, cb):
        """Read the device int64 scalar t at the next host synchronisation and pass it to cb."""
        self._deferred.append((t, cb))

    def dedup_stream(self):
        """The stream run() queues the dedup of the batches loaded ahead on (a stream of default priority, made on
        first use), or None to keep it on the current stream: with the HIP backend unless dedup_ahead is False."""
        if not (self.dedup_ahead and self.d.type == 'cuda' and getattr(self.be, 'sync_counts', False)):
            return None
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.d)
        return self._side

    def count_slot(self):
        """A device int64 [1] for a count the next synchronisation reads (defer_count), inside the plan's sync buffer;
        None without one.  The ring holds 64 - NCOUNTS slots, far more than the counts deferred between two
        synchronisations."""
        if self._sync is None:
            return None
        i = self._sync_next
        self._sync_next = i + 1 if i + 1 < self._sync.numel() else NCOUNTS
        return self._sync[i:i + 1]

    def flush_deferred(self):
        """One host synchronisation that resolves every deferred count (counted in stats like any other)."""
        self._host_list(torch.zeros(0, dtype=I64, device=self.d))

    def _host(self, *ts):
        self._stats['syncs'] += 1
        return torch.stack([t.reshape(()).to(I64) for t in ts]).tolist()

    def _host_list_async(self, t):
        """Start reading t (a device int64 vector) and the deferred counts to the host; returns a function that waits
        for them and returns t's values.  On the GPU the values go to pinned memory by an asynchronous copy
        followed by an event, so the host waits only for the work queued before that copy: kernels the caller
        queues after this call keep the GPU busy while the host waits and then acts on the values."""
        if not (t.is_cuda and self.d.type == 'cuda'):
            vals = self._host_list(t)
            return lambda: vals
        self._stats['syncs'] += 1
        n = t.numel()
        sb = self._sync
        if sb is not None and t.data_ptr() == sb.data_ptr() and all(
                x.data_ptr() - sb.data_ptr() in range(0, sb.numel() * 8, 8) for x, _ in self._deferred):
            # everything to read lies in the sync buffer: copy it whole, pick the deferred values by offset
            dev = sb
            picks = list(range(n)) + [(x.data_ptr() - sb.data_ptr()) // 8 for x, _ in self._deferred]
        else:
            dev = torch.cat([t.reshape(-1).to(I64)] + [x.reshape(-1) for x, _ in self._deferred])
            picks = None
        m = dev.numel()
        if self._pin is None or self._pin.numel() < m:
            self._pin = torch.empty(max(m, 64), dtype=I64, pin_memory=True)
        host = self._pin[:m]
        host.copy_(dev, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        deferred, self._deferred = self._deferred, []

        def finish():
            t0 = time.perf_counter()
            ev.synchronize()
            self.wait_s += time.perf_counter() - t0
            vals = host.tolist()
            if picks is not None:
                vals = [vals[i] for i in picks]
            for (_, cb), v in zip(deferred, vals[n:]):
                cb(v)
            return vals[:n]
        return finish

    def _host_list(self, t):
        """t.tolist() -- with any deferred device counts read in the same transfer (one synchronisation)."""
        self._stats['syncs'] += 1
        if not self._deferred:
            return t.tolist()
        n = t.numel()
        vals = torch.cat([t.reshape(-1).to(I64)] + [x.reshape(-1) for x, _ in self._deferred]).tolist()
        for (_, cb), v in zip(self._deferred, vals[n:]):
            cb(v)
        self._deferred = []
        return vals[:n]

    # ---- plan (srm2/elara.py:209-414, cpp directory path) ----
    def plan(self, s, u, u_nexts, g_occ=None, dplan=None):
        """The step's plan.  With g_occ and dplan, the batch's per-row gradients (the segment sum in class-rank
        order) are queued right after the classification, before the host waits for the class counts, and kept
        in p.G unless the overflow path reorders the rows.  In the device-driven step u is (rows, count on the
        device) and the whole step is issued here (_plan_dev)."""
        if isinstance(u, tuple):
            if not self.sync_free:
                raise RuntimeError('plan: a device count of rows needs the device-driven step')
            return self._plan_dev(s, u[0], u[1], g_occ, dplan)
        d, K, C = self.d, self.K, self.C
        n = u.numel()
        # classes, class order, expired / preemptible / protected dynamic slots, counts (srm2/elara.py:214-267)
        ring = {}
        if self.next_bits is not None:
            ring = dict(next_bits=self.next_bits,
                        next_mask=sum(1 << ((s + k) % 32) for k in range(1, self.depth)))
        if self._sync is not None:
            ring['counts_out'] = self._sync[:NCOUNTS]
        seg_in_plan = g_occ is not None and getattr(self.be, 'seg_in_plan', False)
        if seg_in_plan:
            g_occ = g_occ.contiguous()
            ring['seg'] = (g_occ, dplan)
        sk = {'partials_done': True} if seg_in_plan else {}
        pc = self.be.plan_classify(u, u_nexts, self.slot_of, self.last_seen, self.code, self.kthr, self.toff,
                                   self.dyn_slots, self.slot_row, self.mat_top, self.log_top, s, K,
                                   self.st_mode == 'T', self.loc, self.R, carry=self.dyn == 'carry', live=self.live,
                                   **ring)
        finish = self._host_list_async(pc.counts)
        G = self.be.segsum(g_occ, dplan, n, pc.rank, **sk) if g_occ is not None else None
        vals = finish()
        counts = vals[:10]
        n_exp, n_pre, mat_top, log_top = vals[CNT_EXP], vals[CNT_PRE], vals[CNT_MAT_TOP], vals[CNT_LOG_TOP]
        live = vals[CNT_LIVE]
        if vals[CNT_BAD]:
            raise ValueError(f'step {s}: {vals[CNT_BAD]} rows of the batch lie outside [0, {self.R})')
        # memory-pressure gate of the residency-aware representation (srm2/elara.py:212-213, 423-425): the arenas'
        # used bytes as the previous step left them against the budget; sticky once on
        if (self.evl_mode == 2 and not self.evl and self.host_budget > 0
                and (mat_top * 3 + live) * self.D * 4 >= self.evl_gate_frac * self.host_budget):
            self.evl = True
            self._stats['evl_on_step'] = s
        sl, c, order = pc.sl, pc.c, pc.order
        n_adm = counts[C_NADM] + counts[C_LADM] + counts[C_FADM]
        nd = self.dyn_slots.numel()
        need = n_adm - (self.n_free + n_exp)
        take = min(need, n_pre) if need > 0 and nd > n_exp else 0
        if take:   # preempt residents not needed within the pipeline window
            ev_slot, keep_dyn = pc.dyn_out[:n_exp + take], pc.dyn_out[n_exp + take:nd]
            n_exp += take
            need -= take
            self._stats['preempt'] += take
        else:
            ev_slot, keep_dyn = pc.dyn_out[:n_exp], pc.dyn_out[nd + n_exp:]
        rank = pc.rank
        u_ord, c_ord, sl_ord, L_row, L_cnt, loc_ord = pc.u_ord, pc.c_ord, pc.sl_ord, pc.L_row, pc.L_cnt, pc.loc_ord
        overflowed = need > 0
        barrier = False
        if overflowed:   # overflow: un-admit (non-carry first) and recount
            admit = (pc.flags & F_ADMIT) != 0
            in_next = (pc.flags & F_NEXT) != 0
            pri = (~admit).to(I32) * 4 + admit.to(I32) * (2 - 2 * in_next.to(I32))
            oo = torch.argsort(pri, stable=True)
            drop = oo[n_adm - need:n_adm]
            admit[drop] = False
            self._stats['overflow'] += need
            n_adm -= need
            cls = classify_from_flags(pc.flags, admit, self.st_mode == 'T')
            # with the class counts: how many of the dropped rows recur in the next batches (carry rows) -- the
            # reference's exactness barrier (srm2/elara.py:252-257)
            *counts, n_carry_drop = self._host(*torch.bincount(cls.long(), minlength=10), in_next[drop].sum())
            barrier = n_carry_drop > 0
            order, rank = rank_order(cls)
            u_ord, c_ord, sl_ord, L_row = u[order], c[order].long(), sl[order].long(), None
            G = None   # the rows' order changed: the segment sum is redone in the new order
            loc_ord = self.loc[u_ord].long()
        # class-rank bounds: positions b[r] .. b[r+1] of `order` hold the rows of rank r
        b = [0]
        for cl in RANK_CLASSES:
            b.append(b[-1] + counts[cl])
        nNa, nNp, nNc, nLa, nLp, nLc, nFa, nFn = counts[1:9]
        p = Plan()
        p.s, p.u, p.n, p.b, p.order, p.rank = s, u, n, b, order, rank
        p.G = G
        p.overflowed = overflowed
        p.barrier = barrier
        # the next step's assembly waits for this step's writes into host arenas when a row of the next batch may be
        # among them: after an overflow (an un-admitted row), or when the next batch was not observed before this
        # plan (its rows were then not admitted for it)
        p.link_next = overflowed or self._observed <= s
        p.evl = self.evl
        p.counts = counts
        p.u_ord = u_ord
        p.hit_slot = sl_ord[b[R_HIT]:b[R_HIT + 1]]
        rs = lambda r0, r1: slice(b[r0], b[r1 + 1])  # noqa: E731
        # L rows in the reference's order (admitted, append, compact) for the directory's replay inputs
        if L_row is None:
            Ls = (rs(R_LADM, R_LADM), rs(R_LAPP, R_LAPP), rs(R_LCMP, R_LCMP))
            p.L_row = torch.cat([u_ord[x] for x in Ls])
            p.L_cnt = torch.cat([c_ord[x] for x in Ls]).to(I32)
        else:
            p.L_row, p.L_cnt = L_row[:nLa + nLp + nLc], L_cnt[:nLa + nLp + nLc]
        p.nL = (nLa, nLp, nLc)
        nev = ev_slot.numel()
        # the step's allocations at most: a MAT slot per eviction and compaction, a log entry per append and K per
        # eviction, the latter from the free stack first (n_lfree = log_top - live).  Raised here, before any
        # directory call, when that could pass an arena's capacity; with a host budget, the exact tops are read
        # after the directory calls whenever the bound could fault a new chunk (budget_account).
        mt_hi = mat_top + nev + nNc + nLc
        lt_hi = log_top + max(0, nev * K + nNp + nLp - (log_top - live))
        if mt_hi > self.mat_cap - 1 or lt_hi > self.log_cap:
            raise RuntimeError(f'arena capacity: step {s} may allocate up to MAT row {mt_hi} (capacity '
                               f'{self.mat_cap - 1}) and log entry {lt_hi} (capacity {self.log_cap})')
        p.ev_slot = ev_slot
        lazy_n = nNa + nLa
        p.lazy_n = lazy_n
        nf = self.n_free + nev
        # the native executor takes the rest of the step in one call, unless the host must look at the arenas'
        # tops between the directory calls and the update (a host budget this step could reach) or the update's
        # host-arena writes go to the link stream
        native = (getattr(self.be, 'step_exec', None) is not None and self._slots_in_place
                  and g_occ is not None and not (self.host_budget and (mt_hi > self.faulted['mat']
                                                                       or lt_hi > self.faulted['log'])))
        if native:
            if G is None:
                G = self.be.segsum(g_occ, dplan, n, rank, **sk)
            link = self._link_args(p) if self._link is not None else None
            p._ws, p._off = self.be.step_exec(self, p, G, ev_slot, keep_dyn, u_ord, c_ord, sl_ord, loc_ord,
                                              link=link)
            if link is not None:   # kept until the link stream has read them
                for t in (p._ws, G, loc_ord):
                    t.record_stream(self._link)
                self._link_pending.append((p.s, link[2], p.link_next))
            p._dims = dict(nL=nLa + nLp + nLc, K=K, nh=counts[C_HIT], nev=nev, n_adm=n_adm, na=nNp + nLp,
                           nc=nNc + nLc, nw=b[R_S] - b[R_NADM], D=self.D)
            p._loc_ord = loc_ord
            p.G = None
            p.done = True
            self.free = self._free_buf[:nf - n_adm]
            self.dyn_slots = self._dyn_buf[:keep_dyn.numel() + n_adm]
            self.n_free = nf - n_adm
            self._plan_stats(p, n_adm, nev, barrier)
            return p
        st, pv = self.state_list(), self.params()
        triton = self.dir_impl == 'triton'
        outs = self.be.dir_a(st, pv, p.hit_slot, p.L_row, p.L_cnt, ev_slot, s, deferred=triton)
        (p.L_steps, p.L_ids, p.hrec_dyn, p.hrec_j, p.ev_row, p.ev_rep, p.evl_ids, p.evf_slots, p.ev_dyn) = outs[:9]
        # admissions (srm2/elara.py:345-367): admitted N, L, F rows take slots from the free stack's top
        if self._slots_in_place:   # the stack push, the admissions and the new slot list in one launch
            adm_slots = self.be.plan_admit_slots(self._free_buf, self.n_free, ev_slot, keep_dyn,
                                                 u_ord[rs(R_NADM, R_FADM)], lazy_n, self.evl, s, self.n0, self.C,
                                                 self.R, K, self.code, self.slot_of, self.slot_row, self.adm_c0,
                                                 self.rj, self.rok, self.pstep, self._dyn_buf)
            self.free = self._free_buf[:nf - n_adm]
            self.dyn_slots = self._dyn_buf[:keep_dyn.numel() + n_adm]
        else:
            pool_free = torch.cat([self.free, ev_slot])
            adm_slots = pool_free[nf - n_adm:]
            self.free = pool_free[:nf - n_adm]
            self.be.plan_admit(u_ord[rs(R_NADM, R_FADM)], adm_slots, lazy_n, self.evl, s, self.n0, self.C, self.R,
                               K, self.code, self.slot_of, self.slot_row, self.adm_c0, self.rj, self.rok, self.pstep)
            self.dyn_slots = torch.cat([keep_dyn, adm_slots])
        self.n_free = nf - n_adm
        p.adm_slots = adm_slots
        if lazy_n and self.evl:
            p.adm_rec_slot = adm_slots[:lazy_n]   # their resident histories start at entry 0 of slot - n0
        # non-resident lazy rows: append (stay L, entry index = current count) or compact (to M)
        # (the Triton path's order: the evictions' deferred releases go first, after the appends' pops)
        p.a_ids, p.c_slots = self.be.dir_b(st, pv, u_ord[rs(R_NAPP, R_LAPP)], c_ord[rs(R_NAPP, R_LAPP)],
                                           u_ord[rs(R_NCMP, R_LCMP)], c_ord[rs(R_NCMP, R_LCMP)], s,
                                           rel=(p.ev_row, outs[9]) if triton else None)
        # MAT slots of the transient F and the S rows (adjacent ranks; the directory calls above move no F/S row)
        fs = loc_ord[rs(R_FN, R_S)]
        p.FN_slot, p.S_slot = fs[:nFn], fs[nFn:]
        self._plan_stats(p, n_adm, nev, barrier)
        if self.host_budget and (mt_hi > self.faulted['mat'] or lt_hi > self.faulted['log']):
            self.budget_account(*self._host(self.mat_top, self.log_top))
        return p

    def _plan_dev(self, s, u, n_dev, g_occ, dplan):
        """The device-driven step (srm2/elara.py:209-414 and 471-580 with no host read): one native call
        (elr_step_dev) issues the classification whose scan launch resolves the step on the GPU, the segment sum in
        the resolved class order and the rest of the step, every launch sized from upper bounds -- the batch's
        occurrence count for its unique rows, the dynamic pool for evictions and admissions.  Returns a Plan whose
        counts and arrays are read from the GPU only when something asks for them, which must happen before the
        next step is issued (the next step reuses the workspace)."""
        if g_occ is None or dplan is None:
            raise RuntimeError('the device-driven step takes the batch\'s occurrence gradients and dedup plan')
        self._poll_errors()
        p = Plan()
        p.s, p.u, p.evl, p._es = s, u, self.evl, self
        mark, self._pending_mark = self._pending_mark, None
        p._ws, p._doff, p._seq = self.be.step_dev(self, s, u, n_dev, g_occ.contiguous(), dplan, mark)
        p.done = True
        return p

    def _plan_stats(self, p, n_adm, nev, barrier):
        counts = p.counts
        nNa, nNp, nNc, nLa, nLp, nLc, nFa, nFn = counts[1:9]
        st_ = self._stats
        st_['adm'] += n_adm
        st_['ev'] += nev
        st_['hits'] += counts[C_HIT]
        st_['N'] += nNa + nNp + nNc
        st_['L'] += nLa + nLp + nLc
        st_['F'] += nFa + nFn
        st_['S'] += counts[C_S]
        st_['compactions'] += nNc + nLc
        st_['appends'] += nNp + nLp
        st_['barriers'] += int(barrier)

    def budget_account(self, mat_top, log_top):
        """Fault the arenas' accounting up to the tops a step left (ArenaStore.fault, srm2/elara.py:63-81, as the
        update worker calls it, srm2/elara.py:555-557): each arena is held in steps of budget_chunk bytes (a fault
        takes at least one step, at most the arena's capacity), MAT records 12 * D bytes, log entries 4 * D.
        HostBudgetExceeded if the held bytes would pass host_budget."""
        for which, top in (('mat', mat_top), ('log', log_top)):
            rec = (3 if which == 'mat' else 1) * self.D * 4
            step = max(1, self.budget_chunk // rec)
            cap = self.mat_cap - 1 if which == 'mat' else self.log_cap
            cur = self.faulted[which]
            if top <= cur:
                continue
            new = min(cap, max(top, cur + step))
            if self.host_budget and self.resident_bytes() + (new - cur) * rec > self.host_budget:
                raise HostBudgetExceeded(f'arena store would exceed host budget {self.host_budget / 2**30:.3f} GiB '
                                         f'(mat rows {mat_top}, log entries {log_top})')
            self.faulted[which] = new

    def resident_bytes(self):
        """Bytes the budget accounting holds (ArenaStore.resident_bytes, srm2/elara.py:60-61)."""
        return self.faulted['mat'] * 12 * self.D + self.faulted['log'] * 4 * self.D

    def dir_check(self):
        """The directory's consistency check that the reference records at the end of every ELARA run
        (srm2/train.py:474-477): the live log entries equal the valid entry ids, and live entries plus the free
        stack's depth equal the log arena's top.  One host synchronisation (not counted in stats['syncs'])."""
        self.join_link()
        valid = (self.ent[:self.R * self.K] >= 0).sum()
        live, nf, top, mt, ev = torch.stack([t.reshape(()).to(I64) for t in (
            self.live, self.n_lfree, self.log_top, self.mat_top, valid)]).tolist()
        return {'live': live, 'ent_valid': ev, 'n_free': nf, 'log_top': top, 'mat_top': mt,
                'ok': live == ev and live + nf == top}

    def footprint(self):
        """The arenas' footprint as the reference reports it (ArenaStore.footprint, srm2/elara.py:95-103); one
        host synchronisation."""
        mt, lt, live = self._host(self.mat_top, self.log_top, self.live)
        D = self.D
        return {'store': 'elara_arena', 'mat_rows': mt, 'live_log_entries': live, 'log_arena_entries': lt,
                'store_bytes': mt * 3 * D * 4 + live * D * 4, 'mat_bytes': mt * 3 * D * 4, 'log_bytes': live * D * 4,
                'index_bytes': 0, 'resident_bytes': self.resident_bytes()}

    # ---- assemble (srm2/elara.py:471-489): full states of the non-resident rows, one fused launch ----
    def assemble(self, p):
        """Work array [b[R_S] - b[R_NADM], 3, D] in class-rank order: admitted N / L / F, appended N / L, compacted
        N / L and transient F rows -- N rows by counter-hash init, L rows by replay of their log entries, F rows
        from the MAT arena."""
        self._wait_link(lambda s_ev, nxt: s_ev <= p.s - 2 or (s_ev == p.s - 1 and nxt))
        b = p.b
        w0 = b[R_NADM]
        nLa, nLp, _ = p.nL
        segs = [(b[r + 1] - w0, kind, aux) for r, kind, aux in (
            (R_NADM, ASM_INIT, 0), (R_LADM, ASM_REPLAY, 0), (R_FADM, ASM_GATHER, 0), (R_NAPP, ASM_INIT, 0),
            (R_LAPP, ASM_REPLAY, nLa), (R_NCMP, ASM_INIT, 0), (R_LCMP, ASM_REPLAY, nLa + nLp),
            (R_FN, ASM_GATHER, 0))]
        p.work = self.be.assemble(p.u_ord[w0:b[R_S]], segs, p.L_ids, p.L_steps, p.L_cnt, self.logs, self.mat,
                                  self.loc, self.K)

    # ---- update (srm2/elara.py:491-542 and the host worker's writes 544-580, all in HBM) ----
    def update(self, p, G):
        """G [n, D]: the batch's per-row gradients in class-rank order (p.order).  A backend with step_update
        (the HIP one: elr_step_update) issues the whole update natively, in the order below."""
        if getattr(self.be, 'step_update', None) is not None:
            if self._link is None:
                self.be.step_update(self, p, G)
                return
            self.be.step_update(self, p, G, part=1)
            self._link.wait_stream(torch.cuda.current_stream(self.d))
            with torch.cuda.stream(self._link):
                self.be.step_update(self, p, G, part=2)
                ev = torch.cuda.Event()
                ev.record()
            for t in (p.work, G, p.c_slots, p.a_ids, p.FN_slot, p.S_slot):   # kept until the link stream is done
                if t is not None and t.numel():
                    t.record_stream(self._link)
            self._link_pending.append((p.s, ev, p.link_next))
            return
        be, s, b = self.be, p.s, p.b
        W, w0 = p.work, b[R_NADM]
        rg = lambda r0, r1: G[b[r0]:b[r1 + 1]]  # noqa: E731
        rw = lambda r0, r1: W[b[r0] - w0:b[r1 + 1] - w0]  # noqa: E731
        if b[R_HIT + 1] > b[R_HIT]:
            gh = rg(R_HIT, R_HIT)
            if p.evl:
                be.glog_put(self.glog, p.hrec_dyn, p.hrec_j, gh)
            be.adam(self.pool, p.hit_slot, gh, s)
        if p.ev_slot.numel():
            # evicted slots are read before admissions reuse them: full states of rows going to M into their MAT
            # slots (rows going back to L carry the trash slot), history entries of rows going back to L into
            # their new log ids (-1 for none)
            be.copy_rows(self.mat, p.evf_slots, self.pool, p.ev_slot)
            be.glog_take(self.logs, p.evl_ids, self.glog, p.ev_dyn)
        # Adam on the admitted, compacted and transient work rows (appended rows only log their gradient)
        if b[R_FADM + 1] > b[R_NADM]:
            be.adam_dense(rw(R_NADM, R_FADM), rg(R_NADM, R_FADM), s)
        if b[R_FN + 1] > b[R_NCMP]:
            be.adam_dense(rw(R_NCMP, R_FN), rg(R_NCMP, R_FN), s)
        if p.adm_slots.numel():
            be.copy_rows(self.pool, p.adm_slots, rw(R_NADM, R_FADM))
        if p.lazy_n and p.evl:   # admission gradient = resident history entry 0 of admitted N / L rows
            be.glog_put(self.glog, p.adm_rec_slot, None, rg(R_NADM, R_LADM), self.n0)
        if p.c_slots.numel():
            be.copy_rows(self.mat, p.c_slots, rw(R_NCMP, R_LCMP))
        if p.a_ids.numel():
            be.copy_rows(self.logs, p.a_ids, rg(R_NAPP, R_LAPP))
        if p.FN_slot.numel():
            be.copy_rows(self.mat, p.FN_slot, rw(R_FN, R_FN))
        if p.S_slot.numel():
            be.adam(self.mat, p.S_slot, rg(R_S, R_S), s)

    # ---- one step from a batch's occurrence ids and gradients ----
    def step(self, s, ids, g_occ, u, dplan, u_nexts):
        """Logical step s (1-based): ids int64 [O] (occurrences), g_occ [O, D] their gradients, u the batch's
        unique rows and dplan its dedup plan (from be.unique), u_nexts the unique rows of the next depth-1
        batches.  The lookahead is the caller's: batches s+1 .. s+L are observed (observe) before this call, as
        run() does (srm2/train.py:359-366); if batch s+1 was not, the next step waits for this step's writes into
        host arenas before it assembles."""
        p = self.plan(s, u, u_nexts, g_occ, dplan)
        if p.__dict__.get('done', False):   # the native executor has issued the assembly and the update
            return p
        self.assemble(p)
        G = p.G if p.G is not None else self.be.segsum(g_occ, dplan, u.numel(), p.rank)
        p.G = None
        self.update(p, G)
        return p

    # ---- eval-style materialisation (srm2/elara.py:582-604) ----
    def eval_weights(self, rows, full=False):
        """Current (w) -- or (w, m, v) with full=True -- of `rows`: resident rows from the pool, materialised rows
        from the MAT arena, logged and implicit rows by replay from the log arena."""
        K, D = self.K, self.D
        self.join_link()
        out = torch.empty(rows.numel(), 3, D, device=self.d)
        sl = self.slot_of[rows]
        res = sl >= 0
        ri = res.nonzero().flatten()
        if ri.numel():
            self.be.copy_rows(out, ri, self.pool, sl[ri].long())
        nr = (~res).nonzero().flatten()
        r = rows[nr]
        c = self.code[r]
        mat = c == self.MAT
        mi = mat.nonzero().flatten()
        if mi.numel():
            self.be.copy_rows(out, nr[mi], self.mat, self.loc[r[mi]].long())
        li = (~mat).nonzero().flatten()
        if li.numel():
            rl = r[li]
            cnt = c[li].to(I32)
            kk = torch.arange(K, device=self.d)
            e = self.ent[rl[:, None] * K + kk[None, :]]
            ids = torch.where(kk[None, :] < cnt[:, None], e, torch.full_like(e, -1))
            steps = torch.where(e >= 0, self.lstep[e.clamp(min=0).long()], torch.zeros_like(e))
            off = torch.cumsum(cnt.long(), 0) - cnt.long()
            valid = kk[None, :] < cnt.long()[:, None]
            dst = torch.where(valid, off[:, None] + kk[None, :], torch.full_like(off[:, None], -1))
            lg = torch.empty(rl.numel() * K, D, device=self.d)
            self.be.copy_rows(lg, dst.reshape(-1), self.logs, ids.reshape(-1).to(I64))
            fl = self.be.replay(rl, lg, off, steps, cnt, K)
            self.be.copy_rows(out, nr[li], fl)
        return out if full else out[:, 0]


def run(step, batches, grads, steps=None, on_step=None, freeze_gc=True):
    """Drive `step` over a sequence of batches as srm2/train.py:344-444 does: the batch of logical step j+1 is
    deduplicated and observed L+1 steps ahead (TTL lookahead), plan(s) sees the next depth-1 batches, then the step
    assembles and updates.  batches[j]: int64 occurrence ids; grads(j) or grads[j]: [O_j, D] occurrence gradients.
    on_step(s, plan) is called after each step.

    freeze_gc: for the duration of the loop, the objects that exist when it starts are moved out of the Python
    collector's generations (gc.freeze; gc.unfreeze afterwards).  A step allocates a few thousand short-lived
    objects, and each full collection they trigger would otherwise walk every long-lived object of the process --
    on average about 0.17 ms of host time per step at config C5, where the host is the bottleneck."""
    if not freeze_gc:
        return _run(step, batches, grads, steps, on_step)
    gc.collect()
    gc.freeze()
    try:
        return _run(step, batches, grads, steps, on_step)
    finally:
        gc.unfreeze()


class PlanPool:
    """Reusable dedup-plan buffers for run(): one entry (plan buffer, unique-id array, unique count, and the events
    that order its reuse) per batch between its dedup and its step.  Without it each batch's plan would be new
    allocations handed between streams with record_stream: the device-driven step's host, which runs steps ahead of
    the GPU, would then find no freed block of that size and allocate anew on every batch (tens of microseconds of
    host time per allocation, the host being the step's bottleneck).

    An entry is taken for a batch's sort and given back once the batch's step has been issued; a reused entry's sort
    first waits, on the GPU, for the event recorded on the main stream after that step (on one stream, stream order
    alone suffices).  Entries are reused only while at least `spare` are free, so a sort waits for the step before
    the one just issued and not for the last one."""

    def __init__(self, dev, spare=2):
        self.dev, self.spare = dev, spare
        self.free = []   # entries given back, oldest first
        self.made = 0

    def take(self, n, nbytes, side):
        if len(self.free) >= self.spare:
            e = self.free.pop(0)
            if side is not None:   # the main stream's work on its last batch comes first
                if e['rel_set']:
                    side.wait_event(e['rel'])
                else:   # given back without an event (by a run on one stream): wait for all the main stream's work
                    side.wait_stream(torch.cuda.current_stream(self.dev))
            if e['buf'].numel() >= nbytes and e['u'].numel() >= n:
                return e
            # too small for this batch: new buffers; the old ones go back to the allocator only after the main
            # stream's work on them (they were made on the sort's stream)
            if side is not None:
                main = torch.cuda.current_stream(self.dev)
                e['buf'].record_stream(main)
                e['u'].record_stream(main)
                e['nu'].record_stream(main)
        else:
            e = {'rel': torch.cuda.Event(), 'sorted': torch.cuda.Event(), 'rel_set': False}
            self.made += 1
        ctx = torch.cuda.stream(side) if side is not None else contextlib.nullcontext()
        with ctx:   # made on the stream that writes them first
            e['buf'] = torch.empty(nbytes, dtype=torch.uint8, device=self.dev)
            e['u'] = torch.empty(max(n, 1), dtype=I64, device=self.dev)
            e['nu'] = torch.empty(1, dtype=I64, device=self.dev)
        return e

    def give(self, e, side):
        if side is not None:
            e['rel'].record(torch.cuda.current_stream(self.dev))
            e['rel_set'] = True
        self.free.append(e)


def _run(step, batches, grads, steps, on_step):
    S = len(batches) if steps is None else steps
    U, PLANS, AHEAD, ENTRY = {}, {}, {}, {}
    dev = step.d
    side = step.dedup_stream()
    pool = None
    if dev.type == 'cuda' and getattr(step.be, 'plan_bytes', None) is not None:
        if step._plan_pool is None:
            step._plan_pool = PlanPool(dev)
        pool = step._plan_pool

    def dedup(j):
        """Batch j's dedup plan.  With a side stream it is queued there one step before the batch is observed, so
        that its sort runs beside the next step's kernels.  Its buffers come from the plan pool (given back after
        batch j's step); without a pool, the tensors it makes are used on the main stream later (record_stream keeps
        the allocator from reusing them before that work is done)."""
        src = batches[j]
        ids = src.to(dev)
        # the host-planned step reads the unique count at its next synchronisation, from a slot of its sync buffer;
        # the device-driven step never reads it, and the host runs steps ahead of the GPU, so each batch has a count
        # tensor of its own (its pool entry's, or one kept by the allocator until the main stream's work on it is
        # done) rather than a slot the host could hand to a later batch before this one's plan has run
        slot = None if step.sync_free else step.count_slot()
        kw = {} if slot is None else {'nu_out': slot}
        n = ids.numel()
        if pool is not None and step.field_bounds is not None:
            kw['fields'] = step.field_bounds
        e = pool.take(n, step.be.plan_bytes(n), side) if pool is not None and n else None
        if e is not None:
            ENTRY[j] = e
            kw['out'] = (e['buf'], e['u'], e['nu'])
        if side is None:
            AHEAD[j] = (*step.be.unique_async(ids, step.R, **kw), None)
            return
        main = torch.cuda.current_stream(dev)
        copied = src.device != ids.device or src.data_ptr() != ids.data_ptr()
        if copied:
            side.wait_stream(main)   # the copy that made ids
        with torch.cuda.stream(side):
            u, dplan, nu = step.be.unique_async(ids, step.R, **kw)
            ev = e['sorted'] if e is not None else torch.cuda.Event()
            ev.record()
        if copied:
            ids.record_stream(side)
        if e is None:
            for t in (u, dplan.buf, nu if slot is None else None):
                if t is not None:
                    t.record_stream(main)
        AHEAD[j] = (u, dplan, nu, ev)

    def observe(j, in_next_step=False):
        """Mark batch j's rows (the lookahead) on the main stream, its unique count read at the next host
        synchronisation (the plan's).  in_next_step (device-driven, sorted on the side stream): marked by the next
        step's native call instead, which waits for the sort there."""
        u, dplan, nu, ev = AHEAD.pop(j)
        if ev is not None and not in_next_step:
            torch.cuda.current_stream(dev).wait_event(ev)
        PLANS[j] = dplan
        if step.sync_free:   # the device-driven step takes the rows with their count on the device, never read here
            if nu is None:   # an empty batch
                u, nu = torch.zeros(1, dtype=torch.int64, device=dev), torch.zeros(1, dtype=torch.int64, device=dev)
            U[j] = (u, nu)
            if in_next_step:
                step.observe_in_next_step(j + 1, u, nu, ev)
            else:
                step.observe(j + 1, u, nu)
            return
        if nu is None:
            U[j] = u
            step.observe(j + 1, u)
            return

        def resolve(v, j=j, u=u, dplan=dplan):
            U[j] = u[:v]
            dplan.U = v
        step.observe(j + 1, u, nu)
        step.defer_count(nu, resolve)

    # device-driven with the sorts on the side stream: batch s + L + 2, sorted just before step s is issued, is marked
    # by step s itself (after its plan, as observe() before step s + 1 would)
    fold = bool(step.sync_free and side is not None and getattr(step, 'fold_mark', False))
    if fold:
        step._pending_mark = None
    try:
        for j in range(min(S, step.L + 1)):
            dedup(j)
            observe(j)
        if step.L + 1 < S:
            dedup(step.L + 1)
            if fold:
                observe(step.L + 1)
        if not step.sync_free:
            step.flush_deferred()
        for s in range(S):
            if s + step.L + 1 < S and not fold:
                observe(s + step.L + 1)
            if s + step.L + 2 < S:
                dedup(s + step.L + 2)
                if fold:
                    observe(s + step.L + 2, in_next_step=True)
            u_nexts = [] if step.sync_free else [U[s + k] for k in range(1, step.depth) if s + k < S]
            g = grads(s) if callable(grads) else grads[s]
            p = step.step(s + 1, batches[s].to(dev), g.to(dev), U.pop(s), PLANS.pop(s), u_nexts)
            if on_step is not None:
                on_step(s + 1, p)
            e = ENTRY.pop(s, None)
            if e is not None:   # batch s's last use: its step (and the unique rows of the depth-1 plans before it)
                pool.give(e, side)
        step.join_link()
        step.check_capacity()
    finally:
        # entries still out (a step raised): back to the pool behind the main stream's work queued so far, so that
        # no later sort writes into a plan that queued work may still read
        for e in ENTRY.values():
            pool.give(e, side)
        ENTRY.clear()
