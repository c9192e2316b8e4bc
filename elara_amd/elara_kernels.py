"""The directory's second front end -- drop-in for srm2/elara_kernels.py (the `--elara-dir-impl triton` path).

    hits(pl, hs, s) -> (out_dyn, out_j)                 elara_kernels.py:16-40
    lsteps(pl, rows, cnt) -> (steps [n,K] int32, ids [n,K] int64)          elara_kernels.py:43-60
    Directory(pl).evict(ev_slot, ev_row, thr) -> (rep, evl_ids, evf_slots, release part)   elara_kernels.py:152-171
    Directory(pl).appends(rows, ks, s) -> ids           elara_kernels.py:173-186
    Directory(pl).compact(rows, cnt) -> slots           elara_kernels.py:188-197
    Directory(pl).release(parts)                        elara_kernels.py:199-209

`pl` is the planner: any object carrying the 17 directory tensors under the reference's names (code, loc, ent,
lstep, lfree, n_lfree, log_top, mat_top, live, adm_c0, rj, pstep, kthr, toff, slot_of, slot_row, rok) and R, Kmax
(or K), log_cap, n0, Cdyn, MAT, mat_trash, evict_logs (or evl) -- srm2/elara.py ELARAPlanner, or elara_amd.step
.ElaraStep.  The calls run the HIP directory kernels of elr_dir_a / elr_dir_evict / elr_dir_b.

Allocation order: the Triton path's own (srm2/elara_kernels.py:5-7).  Every log id of a step is allocated before any
of its releases: evict() releases nothing and returns the host logs of rows going to M as its release part,
appends() pops after the evictions' allocations, compact() assigns MAT slots only, and release(parts) pushes the
parts' entries in the order given (elr_dir_evict_deferred, elr_dir_b_release).  The reference's default (`cpp`)
directory releases at once instead (srm2/elara_dir.cpp:80-94, 102-108), so its log ids differ; every other state
and every weight is the same under both orders.
"""
import ctypes

import torch

from . import _lib
from .elara_dir import I32, I64, _idx, _scratch

ST_NAMES = ('code', 'loc', 'ent', 'lstep', 'lfree', 'n_lfree', 'log_top', 'mat_top', 'live', 'adm_c0', 'rj', 'pstep',
            'kthr', 'toff', 'slot_of', 'slot_row', 'rok')


def _K(pl):
    return int(getattr(pl, 'Kmax', None) or pl.K)


def _state(pl):
    from .elara_dir import _state as st_of
    evl = getattr(pl, 'evict_logs', None)
    if evl is None:
        evl = pl.evl
    pv = [pl.R, _K(pl), pl.log_cap, pl.n0, pl.Cdyn, pl.MAT, pl.mat_trash, int(bool(evl))]
    S, P, dev, K = st_of([getattr(pl, n) for n in ST_NAMES], pv)
    return S, P, dev, K, pl.code


def hits(pl, hs, s):
    """Resident-history recording of the hit slots hs at logical step s (srm2/elara_kernels.py:16-40)."""
    S, P, dev, K, anchor = _state(pl)
    hs = _idx(hs, dev)
    n = hs.numel()
    out_dyn = torch.empty(n, dtype=I64, device=dev)
    out_j = torch.empty(n, dtype=I64, device=dev)
    if n:
        p = _lib.ptr
        with _lib.on_device(dev):
            rc = _lib.lib().elr_dir_a(ctypes.byref(S), ctypes.byref(P), p(hs), n, None, None, 0, None, 0, int(s),
                                      None, None, p(out_dyn), p(out_j), None, None, None, None, None, None, 0,
                                      _lib.stream_of(anchor))
        _lib.check(rc, 'elr_dir_a')
    return out_dyn, out_j


def lsteps(pl, rows, cnt):
    """Replay inputs of the logged rows: steps [n,K] int32 (0 where no entry) and entry ids [n,K] int64 (-1 for
    k >= cnt) (srm2/elara_kernels.py:43-60)."""
    S, P, dev, K, anchor = _state(pl)
    rows, cnt = _idx(rows, dev), _idx(cnt, dev, I32)
    n = rows.numel()
    steps = torch.empty(n, K, dtype=I32, device=dev)
    ids = torch.empty(n, K, dtype=I32, device=dev)
    if n:
        p = _lib.ptr
        with _lib.on_device(dev):
            rc = _lib.lib().elr_dir_a(ctypes.byref(S), ctypes.byref(P), None, 0, p(rows), p(cnt), n, None, 0, 0,
                                      p(steps), p(ids), None, None, None, None, None, None, None, None, 0,
                                      _lib.stream_of(anchor))
        _lib.check(rc, 'elr_dir_a')
    return steps, ids.to(I64)


class Directory:
    """Directory operations of one plan step, bound to a planner (srm2/elara_kernels.py:145-209)."""

    def __init__(self, pl):
        self.pl = pl

    def evict(self, ev_slot, ev_row, thr):
        """Eviction representation of slots already unmapped by the caller: back to L if the full history fits
        thr, else to M.  Returns (rep int64 [n], evl_ids int64 [n,K], evf_slots int64 [n] (trash for rows going
        back to L), release part (ev_row, counts): the host-log entries of rows going to M, for release())."""
        pl = self.pl
        S, P, dev, K, anchor = _state(pl)
        ev_slot, ev_row = _idx(ev_slot, dev), _idx(ev_row, dev)
        thr = torch.as_tensor(thr, device=dev).to(torch.int8).contiguous().reshape(-1)
        n = ev_slot.numel()
        if ev_row.numel() != n or thr.numel() != n:
            raise RuntimeError('ev_slot, ev_row and thr must have the same length')
        rep = torch.empty(n, dtype=torch.uint8, device=dev)
        evl_ids = torch.empty(n, K, dtype=I64, device=dev)
        evf = torch.empty(n, dtype=I64, device=dev)
        ev_dyn = torch.empty(n, dtype=I64, device=dev)
        rel_cnt = torch.empty(n, dtype=I64, device=dev)
        if n:
            scratch, nbytes = _scratch(dev, n, 0)
            p = _lib.ptr
            with _lib.on_device(dev):
                rc = _lib.lib().elr_dir_evict_deferred(ctypes.byref(S), ctypes.byref(P), p(ev_slot), p(ev_row),
                                                       p(thr), n, p(rep), p(evl_ids), p(evf), p(ev_dyn),
                                                       p(rel_cnt), p(scratch), nbytes, _lib.stream_of(anchor))
            _lib.check(rc, 'elr_dir_evict_deferred')
        return rep.to(I64), evl_ids, evf, (ev_row, rel_cnt)

    def appends(self, rows, ks, s):
        """One new log entry per row at entry index ks (the row stays L): returns the log ids int64 [n]."""
        return self._dir_b(rows, ks, None, None, s)[0]

    def compact(self, rows, cnt):
        """MAT slots for rows going to M (code = MAT); their cnt logged entries are released by release()."""
        return self._dir_b(None, None, rows, cnt, 0, c_release=False)[1]

    def release(self, parts):
        """parts: list of (rows, counts): push the first counts[i] logged entries of each row onto the free stack,
        in the order of the parts and rows, after this step's allocations."""
        parts = [(r, c) for r, c in parts if r.numel()]
        if not parts:
            return
        rows = torch.cat([r.to(I64) for r, _ in parts])
        cnt = torch.cat([c.to(I64) for _, c in parts])
        self._dir_b(None, None, None, None, 0, rel=(rows, cnt))

    def _dir_b(self, a_rows, a_k, c_rows, c_cnt, s, rel=None, c_release=True):
        pl = self.pl
        dev = pl.code.device
        z = torch.empty(0, dtype=I64, device=dev)
        a_rows = z if a_rows is None else a_rows
        a_k = z if a_k is None else a_k
        c_rows = z if c_rows is None else c_rows
        c_cnt = z if c_cnt is None else c_cnt
        from .elara_dir import elara_dir_b
        evl = getattr(pl, 'evict_logs', None)
        if evl is None:
            evl = pl.evl
        pv = [pl.R, _K(pl), pl.log_cap, pl.n0, pl.Cdyn, pl.MAT, pl.mat_trash, int(bool(evl))]
        return elara_dir_b([getattr(pl, n) for n in ST_NAMES], pv, a_rows, a_k, c_rows, c_cnt, s, rel=rel,
                           c_release=c_release)
