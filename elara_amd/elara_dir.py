"""GPU state directory -- drop-in for the reference's directory extension (srm2/ops.py:32-39 dir_ext(),
srm2/csrc/elara_dir.cpp).

    dir_ext().elara_dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s)
        -> [L_steps, L_ids, hrec_dyn, hrec_j, ev_row, rep, evl_ids, evf_slots, ev_dyn]      elara_dir.cpp:50-96
    dir_ext().elara_dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s) -> [a_ids, c_slots]       elara_dir.cpp:98-110

st is the list of the 17 directory tensors in the reference's order (elara_dir.cpp:8-10; built at
srm2/elara.py:275-277), updated in place; pv = (R, K, Lcap, n0, Cdyn, MAT, trash, evl).  Outputs have the
reference's dtypes and shapes.  Both calls run as HIP kernels (elara_amd/csrc/directory.hip) on torch's current
stream, with no host synchronisation: the allocator counters stay in device memory.
"""
import ctypes

import torch

from . import _lib

I8, I32, I64 = torch.int8, torch.int32, torch.int64
ST_DTYPES = (I8, I32, I32, I32, I32, I64, I64, I64, I64, I8, I8, I32, I8, I64, I32, I64, I8)


_STATE_CACHE = {}


def _state(st, pv):
    """The validated DirState / DirParams of (st, pv).  A directory is called once or twice per step with the same
    17 tensors, so the structures are kept per (tensor addresses and sizes, pv) and validated once."""
    if len(st) != 17 or len(pv) != 8:
        raise RuntimeError('st must hold the 17 directory tensors and pv the 8 parameters')
    key = (tuple((t.data_ptr(), t.numel(), t.dtype, t.device, t.is_contiguous()) for t in st),
           tuple(int(x) for x in pv))
    hit = _STATE_CACHE.get(key)
    if hit is not None:
        return hit
    res = _state_checked(st, pv)
    if len(_STATE_CACHE) >= 16:
        _STATE_CACHE.clear()
    _STATE_CACHE[key] = res
    return res


def _state_checked(st, pv):
    R, K, Lcap, n0, Cdyn = (int(x) for x in pv[:5])
    C = n0 + Cdyn
    dev = st[0].device
    sizes = (R, R + 1, (R + 1) * K, Lcap + 1, Lcap + 1, 1, 1, 1, 1, C, C, (Cdyn + 1) * K, None, None, R, C, C)
    for idx, (t, dt, n) in enumerate(zip(st, ST_DTYPES, sizes)):
        if not (t.is_cuda and t.device == dev and t.dtype == dt and t.is_contiguous()):
            raise RuntimeError(f'st[{idx}] ({_lib.DIR_FIELDS[idx]}) must be a contiguous cuda {dt} tensor on {dev}')
        if n is not None and t.numel() != n:
            raise RuntimeError(f'st[{idx}] ({_lib.DIR_FIELDS[idx]}) must have {n} elements, has {t.numel()}')
    if st[12].numel() != st[13].numel() or st[13].numel() < 1:
        raise RuntimeError('kthr and toff must have the same nonzero length (one entry per table)')
    S = _lib.DirState(*[t.data_ptr() for t in st], st[13].numel())
    P = _lib.DirParams(*(int(x) for x in pv))
    return S, P, dev, K


def _idx(t, dev, dtype=I64):
    t = torch.as_tensor(t, device=dev)
    if t.device != dev:
        raise RuntimeError(f'index tensors must be on {dev}')
    return t.to(dtype).contiguous().reshape(-1)


def _scratch(dev, nev, nc):
    n = int(_lib.lib().elr_dir_scratch_bytes(nev, nc))
    if n < 0:
        _lib.check(n, 'elr_dir_scratch_bytes')
    return torch.empty(max(n, 1), dtype=torch.uint8, device=dev), n


def elara_dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s):
    S, P, dev, K = _state(st, pv)
    hs, L_row, ev_slot = _idx(hs, dev), _idx(L_row, dev), _idx(ev_slot, dev)
    L_cnt = _idx(L_cnt, dev, I32)
    nh, nL, nev = hs.numel(), L_row.numel(), ev_slot.numel()
    if L_cnt.numel() != nL:
        raise RuntimeError('L_cnt must have one count per L row')
    e = lambda *shape, dt=I64: torch.empty(*shape, dtype=dt, device=dev)  # noqa: E731
    out = [e(nL, K, dt=I32), e(nL, K, dt=I32), e(nh), e(nh), e(nev), e(nev, dt=torch.bool), e(nev, K), e(nev), e(nev)]
    scratch, nbytes = _scratch(dev, nev, 0)
    p = _lib.ptr
    with _lib.on_device(dev):
        rc = _lib.lib().elr_dir_a(ctypes.byref(S), ctypes.byref(P), p(hs), nh, p(L_row), p(L_cnt), nL,
                                  p(ev_slot), nev, int(s), *[p(o) for o in out], p(scratch), nbytes,
                                  _lib.stream_of(st[0]))
    _lib.check(rc, 'elr_dir_a')
    return out


def elara_dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s):
    S, P, dev, K = _state(st, pv)
    a_rows, a_k, c_rows, c_cnt = (_idx(x, dev) for x in (a_rows, a_k, c_rows, c_cnt))
    na, nc = a_rows.numel(), c_rows.numel()
    if a_k.numel() != na or c_cnt.numel() != nc:
        raise RuntimeError('a_k must match a_rows and c_cnt must match c_rows')
    a_ids = torch.empty(na, dtype=I64, device=dev)
    c_slots = torch.empty(nc, dtype=I64, device=dev)
    if na or nc:
        scratch, nbytes = _scratch(dev, 0, nc)
        p = _lib.ptr
        with _lib.on_device(dev):
            rc = _lib.lib().elr_dir_b(ctypes.byref(S), ctypes.byref(P), p(a_rows), p(a_k), na, p(c_rows),
                                      p(c_cnt), nc, int(s), p(a_ids), p(c_slots), p(scratch), nbytes,
                                      _lib.stream_of(st[0]))
        _lib.check(rc, 'elr_dir_b')
    return [a_ids, c_slots]


class _DirExt:
    """Mirror of the reference's dir_ext() module."""

    elara_dir_a = staticmethod(elara_dir_a)
    elara_dir_b = staticmethod(elara_dir_b)


_dir = _DirExt()


def dir_ext():
    """Counterpart of srm2/ops.py:32-39 dir_ext(): the directory operations elara_dir_a / elara_dir_b."""
    _lib.lib()
    return _dir
