"""GPU state directory -- drop-in for the reference's directory extension (srm2/ops.py:32-39 dir_ext(),
srm2/csrc/elara_dir.cpp).

    dir_ext().elara_dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s)
        -> [L_steps, L_ids, hrec_dyn, hrec_j, ev_row, rep, evl_ids, evf_slots, ev_dyn]      elara_dir.cpp:50-96
    dir_ext().elara_dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s) -> [a_ids, c_slots]       elara_dir.cpp:98-110

st is the list of the 17 directory tensors in the reference's order (elara_dir.cpp:8-10; built at
srm2/elara.py:275-277), updated in place; pv = (R, K, Lcap, n0, Cdyn, MAT, trash, evl).  Outputs have the
reference's dtypes and shapes.  Both calls run as HIP kernels (elara_amd/csrc/directory.hip) on torch's current
stream, with no host synchronisation: the allocator counters stay in device memory.

The planner's Triton directory path allocates its log ids in another order (srm2/elara_kernels.py: every allocation
of a step before any release).  elara_dir_a(..., deferred=True) and elara_dir_b(..., rel=(ev_row, rel_cnt)) give that
order: call A leaves the host logs of rows going to M in place and returns their release counts as a 10th
output, which call B releases after its appends and ahead of the compacted rows' logs.
"""
import ctypes
import weakref

import torch

from . import _lib

I8, I32, I64 = torch.int8, torch.int32, torch.int64
ST_DTYPES = (I8, I32, I32, I32, I32, I64, I64, I64, I64, I8, I8, I32, I8, I64, I32, I64, I8)


_STATE_CACHE = {}


def _state(st, pv):
    """The validated DirState / DirParams of (st, pv).  A directory is called once or twice per step with the same
    17 tensor objects, so the structures are kept per (tensor identities, pv) and validated once.  The entry holds
    weak references to the tensors and is used only while each one is still the very object it was made from
    (a tensor's storage cannot change address without a new tensor object, except by in-place resizing, which the
    directory's fixed-size arrays never see)."""
    if len(st) != 17 or len(pv) != 8:
        raise RuntimeError('st must hold the 17 directory tensors and pv the 8 parameters')
    key = (tuple(map(id, st)), tuple(int(x) for x in pv))
    hit = _STATE_CACHE.get(key)
    if hit is not None and all(r() is t for r, t in zip(hit[0], st)):
        return hit[1]
    res = _state_checked(st, pv)
    if len(_STATE_CACHE) >= 16:
        _STATE_CACHE.clear()
    _STATE_CACHE[key] = (tuple(weakref.ref(t) for t in st), res)
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
    if isinstance(t, torch.Tensor) and t.dtype == dtype and t.device == dev and t.dim() == 1 and t.is_contiguous():
        return t
    t = torch.as_tensor(t, device=dev)
    if t.device != dev:
        raise RuntimeError(f'index tensors must be on {dev}')
    return t.to(dtype).contiguous().reshape(-1)


def _scratch(dev, nev, nc):
    n = int(_lib.lib().elr_dir_scratch_bytes(nev, nc))
    if n < 0:
        _lib.check(n, 'elr_dir_scratch_bytes')
    return torch.empty(max(n, 1), dtype=torch.uint8, device=dev), n


def elara_dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s, deferred=False):
    S, P, dev, K = _state(st, pv)
    hs, L_row, ev_slot = _idx(hs, dev), _idx(L_row, dev), _idx(ev_slot, dev)
    L_cnt = _idx(L_cnt, dev, I32)
    nh, nL, nev = hs.numel(), L_row.numel(), ev_slot.numel()
    if L_cnt.numel() != nL:
        raise RuntimeError('L_cnt must have one count per L row')
    nbytes = int(_lib.lib().elr_dir_scratch_bytes(nev, 0))
    if nbytes < 0:
        _lib.check(nbytes, 'elr_dir_scratch_bytes')
    i32 = _lib.split_empty(dev, I32, (nL * K, nL * K))
    h, hj, er, evl, evf, evd = _lib.split_empty(dev, I64, (nh, nh, nev, nev * K, nev, nev))
    out = [i32[0].view(nL, K), i32[1].view(nL, K), h, hj, er, torch.empty(nev, dtype=torch.bool, device=dev),
           evl.view(nev, K), evf, evd]
    scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    p = _lib.ptr
    if deferred:
        rel_cnt = torch.empty(nev, dtype=I64, device=dev)
        with _lib.on_device(dev):
            rc = _lib.lib().elr_dir_a_deferred(ctypes.byref(S), ctypes.byref(P), p(hs), nh, p(L_row), p(L_cnt), nL,
                                               p(ev_slot), nev, int(s), *[p(o) for o in out], p(rel_cnt),
                                               p(scratch), nbytes, _lib.stream_of(st[0]))
        _lib.check(rc, 'elr_dir_a_deferred')
        return out + [rel_cnt]
    with _lib.on_device(dev):
        rc = _lib.lib().elr_dir_a(ctypes.byref(S), ctypes.byref(P), p(hs), nh, p(L_row), p(L_cnt), nL,
                                  p(ev_slot), nev, int(s), *[p(o) for o in out], p(scratch), nbytes,
                                  _lib.stream_of(st[0]))
    _lib.check(rc, 'elr_dir_a')
    return out


def elara_dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s, rel=None, c_release=True):
    """Call B; rel = (rows, counts): releases pushed after the appends and ahead of the compacted rows' (which are
    released only when c_release), as elr_dir_b_release."""
    S, P, dev, K = _state(st, pv)
    a_rows, a_k, c_rows, c_cnt = (_idx(x, dev) for x in (a_rows, a_k, c_rows, c_cnt))
    r_rows, r_cnt = (None, None) if rel is None else (_idx(rel[0], dev), _idx(rel[1], dev))
    na, nc, nr = a_rows.numel(), c_rows.numel(), 0 if rel is None else r_rows.numel()
    if a_k.numel() != na or c_cnt.numel() != nc or (rel is not None and r_cnt.numel() != nr):
        raise RuntimeError('a_k must match a_rows, c_cnt c_rows and the release counts their rows')
    nbytes = int(_lib.lib().elr_dir_scratch_bytes(0, nc + nr)) if na or nc or nr else 0
    if nbytes < 0:
        _lib.check(nbytes, 'elr_dir_scratch_bytes')
    a_ids, c_slots = _lib.split_empty(dev, I64, (na, nc))
    if na or nc or nr:
        scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        p = _lib.ptr
        with _lib.on_device(dev):
            if rel is None and c_release:
                rc = _lib.lib().elr_dir_b(ctypes.byref(S), ctypes.byref(P), p(a_rows), p(a_k), na, p(c_rows),
                                          p(c_cnt), nc, int(s), p(a_ids), p(c_slots), p(scratch), nbytes,
                                          _lib.stream_of(st[0]))
            else:
                rc = _lib.lib().elr_dir_b_release(ctypes.byref(S), ctypes.byref(P), p(a_rows), p(a_k), na,
                                                  p(c_rows), p(c_cnt), nc, int(bool(c_release)),
                                                  p(r_rows) if nr else None, p(r_cnt) if nr else None, nr, int(s),
                                                  p(a_ids), p(c_slots), p(scratch), nbytes, _lib.stream_of(st[0]))
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
