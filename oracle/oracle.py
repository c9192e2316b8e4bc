"""numpy wrappers of liboracle.so (the plain-C restatement in elara_oracle.c).  Test infrastructure only."""
import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / 'liboracle.so'

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} missing: run `make -C oracle`')
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.orc_fmix32.restype = ctypes.c_uint32
        _lib.orc_fmix32.argtypes = [ctypes.c_uint32]
        _lib.orc_segment_sum.restype = ctypes.c_int64
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else ctypes.c_void_p(0)


def _need(a, dtype, name):
    if not (isinstance(a, np.ndarray) and a.dtype == dtype and a.flags.c_contiguous):
        raise TypeError(f'{name} must be a contiguous {np.dtype(dtype).name} array')
    return a


def nthreads_default():
    return max(1, min(16, os.cpu_count() or 1))


def adam_scalars(lr, b1, b2, eps, step):
    out = np.zeros(8, dtype=np.float32)
    lib().orc_adam_scalars(ctypes.c_double(lr), ctypes.c_double(b1), ctypes.c_double(b2), ctypes.c_double(eps),
                           ctypes.c_int64(step), _p(out))
    return out


def scalar_table(lr, b1, b2, eps, max_step):
    t = np.zeros((max_step + 1, 8), dtype=np.float32)
    for s in range(1, max_step + 1):
        t[s] = adam_scalars(lr, b1, b2, eps, s)
    return t


def cpu_adam(state, rows, grad, sc, nthreads=1):
    """In place on state [R,3,D] float32; rows int64 [n]; grad [n,D]; sc = 8 scalars."""
    _need(state, np.float32, 'state'); _need(rows, np.int64, 'rows'); _need(grad, np.float32, 'grad')
    sc = np.ascontiguousarray(sc, dtype=np.float32)
    D = state.shape[2]
    assert grad.shape == (rows.size, D)
    rc = lib().orc_cpu_adam(_p(state), _p(rows), _p(grad), ctypes.c_int64(rows.size), ctypes.c_int64(D), _p(sc),
                            ctypes.c_int(nthreads))
    assert rc == 0


def fmix32(x):
    return int(lib().orc_fmix32(ctypes.c_uint32(x & 0xFFFFFFFF)))


def init_rows(rows, D, seed, bound):
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((rows.size, 3, D), dtype=np.float32)
    lib().orc_init_rows(_p(out), _p(rows), ctypes.c_int64(rows.size), ctypes.c_int64(D),
                        ctypes.c_uint32(int(seed) & 0xFFFFFFFF), ctypes.c_float(bound))
    return out


def replay_rows(rows, logs, offs, steps, cnt, D, K, seed, bound, table, nthreads=1):
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    logs = np.ascontiguousarray(logs, dtype=np.float32).reshape(-1, D)
    offs = np.ascontiguousarray(offs, dtype=np.int64)
    steps = np.ascontiguousarray(steps, dtype=np.int32)
    cnt = np.ascontiguousarray(cnt, dtype=np.int32)
    table = np.ascontiguousarray(table, dtype=np.float32)
    out = np.empty((rows.size, 3, D), dtype=np.float32)
    rc = lib().orc_replay_rows(_p(out), _p(rows), _p(logs), ctypes.c_int64(logs.shape[0]), _p(offs), _p(steps),
                               _p(cnt), ctypes.c_int64(rows.size), ctypes.c_int64(D), ctypes.c_int(K),
                               ctypes.c_uint32(int(seed) & 0xFFFFFFFF), ctypes.c_float(bound), _p(table),
                               ctypes.c_int64(table.shape[0]), ctypes.c_int(nthreads))
    if rc != 0:
        raise ValueError('replay input out of range')
    return out


def segment_sum(ids, grad):
    """-> (unique ids ascending int64 [U], summed grads [U,D], inverse int64 [O])."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    O, D = grad.shape
    uniq = np.empty(max(O, 1), dtype=np.int64)
    gsum = np.empty((max(O, 1), D), dtype=np.float32)
    inv = np.empty(max(O, 1), dtype=np.int64)
    U = lib().orc_segment_sum(_p(ids), _p(grad), ctypes.c_int64(O), ctypes.c_int64(D), _p(uniq), _p(gsum), _p(inv))
    return uniq[:U].copy(), gsum[:U].copy(), inv[:O].copy()


# ------------------------------------------------------------------------------------------------------------
# directory
class _Dir(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ('code', 'loc', 'ent', 'lstep', 'lfree', 'n_lfree', 'log_top',
                                               'mat_top', 'live', 'adm_c0', 'rj', 'pstep', 'kthr', 'toff',
                                               'slot_of', 'slot_row', 'rok')] + [('T', ctypes.c_int64)]


class _Params(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ('R', 'K', 'Lcap', 'n0', 'Cdyn', 'MAT', 'trash', 'evl')]


DIR_FIELDS = ('code', 'loc', 'ent', 'lstep', 'lfree', 'n_lfree', 'log_top', 'mat_top', 'live', 'adm_c0', 'rj',
              'pstep', 'kthr', 'toff', 'slot_of', 'slot_row', 'rok')
DIR_DTYPES = dict(code=np.int8, loc=np.int32, ent=np.int32, lstep=np.int32, lfree=np.int32, n_lfree=np.int64,
                  log_top=np.int64, mat_top=np.int64, live=np.int64, adm_c0=np.int8, rj=np.int8, pstep=np.int32,
                  kthr=np.int8, toff=np.int64, slot_of=np.int32, slot_row=np.int64, rok=np.int8)


class DirState:
    """The 17 directory arrays of srm2/csrc/elara_dir.cpp:8-10 as numpy arrays (initial values as
    srm2/elara.py:117-148 sets them)."""

    def __init__(self, R, C, K, n0, toff, kthr, log_cap=None):
        self.R, self.C, self.K, self.n0 = R, C, K, n0
        self.Cdyn = C - n0
        self.Lcap = log_cap or 2 * R
        self.MAT = K + 1
        self.code = np.zeros(R, np.int8)
        self.loc = np.full(R + 1, -1, np.int32)
        self.ent = np.full((R + 1) * K, -1, np.int32)
        self.lstep = np.zeros(self.Lcap + 1, np.int32)
        self.lfree = np.zeros(self.Lcap + 1, np.int32)
        self.n_lfree = np.zeros(1, np.int64)
        self.log_top = np.zeros(1, np.int64)
        self.mat_top = np.zeros(1, np.int64)
        self.live = np.zeros(1, np.int64)
        self.adm_c0 = np.full(C, -1, np.int8)
        self.rj = np.zeros(C, np.int8)
        self.pstep = np.zeros((self.Cdyn + 1) * K, np.int32)
        self.kthr = np.ascontiguousarray(kthr, np.int8)
        self.toff = np.ascontiguousarray(toff, np.int64)
        self.slot_of = np.full(R, -1, np.int32)
        self.slot_row = np.full(C, -1, np.int64)
        self.rok = np.zeros(C, np.int8)

    def params(self, evl):
        return (self.R, self.K, self.Lcap, self.n0, self.Cdyn, self.MAT, self.R, int(bool(evl)))

    def arrays(self):
        return [getattr(self, f) for f in DIR_FIELDS]

    def copy(self):
        c = object.__new__(DirState)
        c.__dict__.update({k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in self.__dict__.items()})
        return c

    def _c(self):
        return _Dir(*[_p(getattr(self, f)) for f in DIR_FIELDS], self.kthr.size)


def dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s, deferred=False):
    """Oracle of elara_dir_a (srm2/csrc/elara_dir.cpp:50-96); mutates st.  Returns the 9 outputs as numpy.
    deferred: the Triton path's order (srm2/elara_kernels.py:152-171): the host logs of rows going to M are not
    released, and a 10th output holds their release counts (for dir_b's `rel`)."""
    K = st.K
    hs = np.ascontiguousarray(hs, np.int64); L_row = np.ascontiguousarray(L_row, np.int64)
    L_cnt = np.ascontiguousarray(L_cnt, np.int32); ev_slot = np.ascontiguousarray(ev_slot, np.int64)
    nh, nL, nev = hs.size, L_row.size, ev_slot.size
    L_steps = np.empty((nL, K), np.int32); L_ids = np.empty((nL, K), np.int32)
    hrec_dyn = np.empty(nh, np.int64); hrec_j = np.empty(nh, np.int64)
    ev_row = np.empty(nev, np.int64); rep = np.empty(nev, np.uint8); evl_ids = np.empty((nev, K), np.int64)
    evf = np.empty(nev, np.int64); ev_dyn = np.empty(nev, np.int64)
    rel_cnt = np.zeros(nev, np.int64) if deferred else None
    d = st._c(); p = _Params(*pv)
    lib().orc_dir_a(ctypes.byref(d), ctypes.byref(p), _p(hs), ctypes.c_int64(nh), _p(L_row), _p(L_cnt),
                    ctypes.c_int64(nL), _p(ev_slot), ctypes.c_int64(nev), ctypes.c_int64(s), _p(L_steps), _p(L_ids),
                    _p(hrec_dyn), _p(hrec_j), _p(ev_row), _p(rep), _p(evl_ids), _p(evf), _p(ev_dyn),
                    _p(rel_cnt) if deferred else None)
    out = [L_steps, L_ids, hrec_dyn, hrec_j, ev_row, rep.astype(bool), evl_ids, evf, ev_dyn]
    return out + [rel_cnt] if deferred else out


def _check_counted_entries(st, pv, rows, cnt):
    """The Triton path's release (srm2/elara_kernels.py:104-116, 199-209) reserves stack positions from the
    requested counts and adds their total to n_lfree, skipping entries that are -1; this build (the HIP kernels and
    orc_dir_b) pushes the live entries packed and counts those.  The two agree exactly when every counted entry
    exists (the reference's comment at elara_kernels.py:208 states it holds by construction): asserted here for
    every release of the Triton order, so that a break shows as a failure instead of silently different ids."""
    R, K = int(pv[0]), int(pv[1])
    rows = np.asarray(rows, np.int64)
    cnt = np.minimum(np.maximum(np.asarray(cnt, np.int64), 0), K)
    ok = (rows >= 0) & (rows < R)
    rows, cnt = rows[ok], cnt[ok]
    if not rows.size:
        return
    kk = np.arange(K, dtype=np.int64)
    e = st.ent[rows[:, None] * K + kk[None, :]]
    missing = (kk[None, :] < cnt[:, None]) & (e < 0)
    if missing.any():
        i = int(np.flatnonzero(missing.any(axis=1))[0])
        raise AssertionError(f'Triton-order release of row {int(rows[i])}: {int(cnt[i])} entries counted, '
                             f'{int((e[i] >= 0).sum())} live')


def dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s, rel=None, c_release=True):
    """Oracle of elara_dir_b (srm2/csrc/elara_dir.cpp:98-110); mutates st.  Returns (a_ids, c_slots).
    rel = (rows, counts): releases pushed after the appends, ahead of the compacted rows' (which are released only
    when c_release) -- the Triton path's Directory.compact / .release (srm2/elara_kernels.py:188-209)."""
    a_rows = np.ascontiguousarray(a_rows, np.int64); a_k = np.ascontiguousarray(a_k, np.int64)
    c_rows = np.ascontiguousarray(c_rows, np.int64); c_cnt = np.ascontiguousarray(c_cnt, np.int64)
    a_ids = np.empty(a_rows.size, np.int64); c_slots = np.empty(c_rows.size, np.int64)
    r_rows, r_cnt = (np.zeros(0, np.int64),) * 2 if rel is None else \
        (np.ascontiguousarray(rel[0], np.int64), np.ascontiguousarray(rel[1], np.int64))
    if r_rows.size != r_cnt.size:
        raise ValueError('rel rows and counts must have the same length')
    if rel is not None:
        _check_counted_entries(st, pv, np.concatenate([r_rows, c_rows]), np.concatenate([r_cnt, c_cnt]))
    d = st._c(); p = _Params(*pv)
    lib().orc_dir_b(ctypes.byref(d), ctypes.byref(p), _p(a_rows), _p(a_k), ctypes.c_int64(a_rows.size), _p(c_rows),
                    _p(c_cnt), ctypes.c_int64(c_rows.size), ctypes.c_int64(s), _p(a_ids), _p(c_slots),
                    ctypes.c_int(int(bool(c_release))), _p(r_rows), _p(r_cnt), ctypes.c_int64(r_rows.size))
    return [a_ids, c_slots]
