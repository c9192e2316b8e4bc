"""Planner classification of one ELARA step on the GPU (elr_plan_classify): srm2/elara.py:214-267.

plan_classify(...) returns the per-position class, flags, slot and code of the batch's unique rows, their positions
sorted stably by class, the dynamic pool slots partitioned into expired / preemptible / protected, and a device
block of counts for the host (one small read, the plan's only synchronisation in the common case).
"""
import ctypes
import weakref
from collections import namedtuple

import torch

from . import _lib

I8, I32, I64 = torch.int8, torch.int32, torch.int64
# classes (srm2/elara.py:31-32)
C_HIT, C_NADM, C_NAPP, C_NCMP, C_LADM, C_LAPP, C_LCMP, C_FADM, C_FNADM, C_S = range(10)
F_HIT, F_N, F_L, F_APP, F_ADMIT, F_NEXT = 1, 2, 4, 8, 16, 32
# counts[16]: 10 class counts, then these
CNT_EXP, CNT_PRE, CNT_PROT, CNT_MAT_TOP, CNT_LOG_TOP, CNT_LIVE, CNT_BAD, NCOUNTS = 10, 11, 12, 13, 14, 15, 16, 17

PlanClass = namedtuple('PlanClass', 'cls flags sl c order rank dyn_out counts u_ord c_ord sl_ord L_row L_cnt loc_ord')


def _dev_i64(t, dev):
    if t.dtype == I64 and t.device == dev and t.is_contiguous():
        return t
    return t.to(device=dev, dtype=I64).contiguous()


_CHECKED = {}


def _check_state(dev, named):
    """dtype / device / contiguity of the planner's state tensors, checked once per set of tensor objects (a step
    passes the same directory tensors to every plan); weak references make sure the entry is used only while each
    tensor is still the very object that was checked."""
    key = tuple(id(t) for t, _, _ in named)
    hit = _CHECKED.get(key)
    if hit is not None and all(r() is t for r, (t, _, _) in zip(hit, named)):
        return
    for t, dt, name in named:
        if t.dtype != dt or t.device != dev or not t.is_contiguous():
            raise RuntimeError(f'plan_classify: {name} must be a contiguous {dt} tensor on {dev}')
    if len(_CHECKED) >= 16:
        _CHECKED.clear()
    _CHECKED[key] = tuple(weakref.ref(t) for t, _, _ in named)


def plan_classify(u, u_nexts, slot_of, last_seen, code, kthr, toff, dyn, slot_row, mat_top, log_top, s, K, want_t,
                  loc=None, R=0, next_bits=None, next_mask=0, carry=False, live=None, counts_out=None, seg=None,
                  n_dev=None, nd_dev=None, ctl=None):
    """Classify the unique rows u (int64, ascending) of logical step s and split the occupied dynamic slots dyn.

    u_nexts: up to 4 ascending int64 tensors (unique rows of the next batches).  State tensors as ElaraStep keeps
    them: slot_of int32 [R], last_seen int32 [R], code int8 [R], kthr int8 [T], toff int64 [T], slot_row int64 [C],
    mat_top / log_top int64 [1].  Returns PlanClass(cls int8 [n], flags uint8 [n], sl int32 [n], c int8 [n],
    order int64 [n] (positions by class rank), rank int64 [n] (its inverse), dyn_out int64 [2 nd], counts int64 [17]
    on the device, and in class-rank order u_ord, c_ord, sl_ord int64 [n] (u, c, sl at `order`); L_row int64 [n] and
    L_cnt int32 [n]: the L rows and their codes as admitted, append, compact, valid up to their count; loc_ord int64
    [n]: loc (int32 [R + 1], when given) of the rows in class-rank order, else None).  With R > 0 a row of u outside
    [0, R) is classified S with no slot and no MAT slot (skipped by every later copy and update), and counted in
    counts[16].

    next_bits (int32 [R], with R > 0) and next_mask: the caller's ring of loaded batches (bit t % 32 of
    next_bits[r] set while the batch of step t holds row r; see rows.mark_rows).  Membership in the next batches is
    then one load per row instead of searches of u_nexts, and bit s % 32 of u's rows is cleared.

    carry: the 'carry' residency (srm2/elara.py:221, 231-233): a missing row is admitted when it appears in the next
    batches, and every unprotected dynamic slot is expired; otherwise 'ttl'.  live (int64 [1], optional): the live
    log-entry counter, copied into counts[15] for the host.  counts_out (int64 [17] on the device, optional): where
    the counts go (e.g. a buffer the caller reads together with other values), else a new tensor.

    seg=(grad, dplan): also the partial chunks of the segment sum of grad [n_occ, D] over the batch's dedup plan
    (dedup.unique_plan), in the classification's first launch (elr_plan_classify_seg); complete the sum with
    dedup.segment_sum_plan(grad, dplan, ..., partials_done=True).

    The device-driven step (elr_plan_step): n_dev / nd_dev (int64 [1] on the device) hold the row and dynamic slot
    counts, u.numel() and dyn.numel() then bound them; ctl = (state, desc, mat_cap, log_cap, triton) with state
    (int64 [CTL_WORDS]) the step's control state and desc (int64 [DESC_WORDS]) where the scan launch writes the
    resolved step (preemption, overflow, class bounds, capacity check; see include/elara_amd.h)."""
    dev = u.device
    if dev.type != 'cuda':
        raise RuntimeError('plan_classify: tensors must be on a GPU')
    u = _dev_i64(u, dev)
    nexts = [_dev_i64(x, dev) for x in u_nexts if x.numel()]
    if len(nexts) > 4:
        raise RuntimeError('plan_classify: at most 4 next batches')
    _check_state(dev, ((slot_of, I32, 'slot_of'), (last_seen, I32, 'last_seen'), (code, I8, 'code'),
                       (kthr, I8, 'kthr'), (toff, I64, 'toff'), (slot_row, I64, 'slot_row'),
                       (mat_top, I64, 'mat_top'), (log_top, I64, 'log_top'))
                 + (((live, I64, 'live'),) if live is not None else ()) + (((loc, I32, 'loc'),) if loc is not None
                                                                           else ()))
    if counts_out is not None and not (counts_out.dtype == I64 and counts_out.device == dev
                                       and counts_out.is_contiguous() and counts_out.numel() == NCOUNTS):
        raise RuntimeError(f'plan_classify: counts_out must be a contiguous {I64} tensor of {NCOUNTS} on {dev}')
    dyn = _dev_i64(dyn, dev)
    n, nd = u.numel(), dyn.numel()
    nbytes = int(_lib.lib().elr_plan_step_scratch_bytes(n, nd) if ctl is not None
                 else _lib.lib().elr_plan_scratch_bytes(n, nd))
    if nbytes < 0:
        _lib.check(nbytes, 'elr_plan_scratch_bytes')
    o64 = _lib.split_empty(dev, I64, (n, n, 2 * nd, 0 if counts_out is not None else NCOUNTS, n, n, n, n,
                                      n if loc is not None else 0))
    o32 = _lib.split_empty(dev, I32, (n, n))
    o8 = _lib.split_empty(dev, I8, (n, n))
    flags = torch.empty(n, dtype=torch.uint8, device=dev)
    scratch = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=dev)
    parts = [o8[0], flags, o32[0], o8[1], o64[0], o64[1], o64[2], counts_out if counts_out is not None else o64[3],
             o64[4], o64[5], o64[6], o64[7], o32[1], o64[8] if loc is not None else None]
    out = PlanClass(*parts)
    p = _lib.ptr
    pin = _lib.PlanIn()
    pin.u, pin.n = u.data_ptr(), n
    for k, x in enumerate(nexts):
        pin.next[k] = x.data_ptr()
        pin.n_next[k] = x.numel()
    pin.nnext = len(nexts)
    pin.slot_of, pin.last_seen, pin.code = slot_of.data_ptr(), last_seen.data_ptr(), code.data_ptr()
    pin.kthr, pin.toff, pin.T = kthr.data_ptr(), toff.data_ptr(), toff.numel()
    pin.dyn, pin.nd, pin.slot_row = dyn.data_ptr(), nd, slot_row.data_ptr()
    pin.mat_top, pin.log_top = mat_top.data_ptr(), log_top.data_ptr()
    pin.s, pin.K, pin.want_t = int(s), int(K), int(bool(want_t))
    pin.loc = loc.data_ptr() if loc is not None else None
    pin.R = int(R)
    pin.carry = int(bool(carry))
    pin.live = live.data_ptr() if live is not None else None
    if next_bits is not None:
        if not (next_bits.dtype == I32 and next_bits.device == dev and next_bits.is_contiguous()
                and next_bits.numel() >= R > 0):
            raise RuntimeError(f'plan_classify: next_bits must be a contiguous {I32} tensor of R rows on {dev}')
        pin.next_bits, pin.next_mask = next_bits.data_ptr(), int(next_mask) & 0xFFFFFFFF
    for t, name in ((n_dev, 'n_dev'), (nd_dev, 'nd_dev')):
        if t is not None and not (t.dtype == I64 and t.device == dev and t.numel() == 1):
            raise RuntimeError(f'plan_classify: {name} must be an int64 tensor of one element on {dev}')
    pin.n_dev = n_dev.data_ptr() if n_dev is not None else None
    pin.nd_dev = nd_dev.data_ptr() if nd_dev is not None else None
    pout = _lib.PlanOut(*[t.data_ptr() if t is not None else None for t in out])
    if ctl is not None:
        state, desc, mat_cap, log_cap, triton = ctl
        for t, m, name in ((state, _lib.CTL_WORDS, 'state'), (desc, _lib.DESC_WORDS, 'desc')):
            if not (t.dtype == I64 and t.device == dev and t.is_contiguous() and t.numel() == m):
                raise RuntimeError(f'plan_classify: ctl {name} must be a contiguous int64 tensor of {m} on {dev}')
        if live is None or nd_dev is None:
            raise RuntimeError('plan_classify: the device-driven step needs live and nd_dev')
        c = _lib.PlanCtl(state.data_ptr(), desc.data_ptr(), int(mat_cap), int(log_cap), int(bool(triton)))
        grad, dplan = seg if seg is not None else (None, None)
        if grad is not None and not (grad.is_cuda and grad.device == dev and grad.dtype == torch.float32
                                     and grad.is_contiguous() and grad.numel() == dplan.n * dplan.D):
            raise RuntimeError(f'plan_classify: seg grad must be a contiguous float32 tensor of {dplan.n}x{dplan.D} '
                               f'on {dev}')
        with _lib.on_device(dev):
            rc = _lib.lib().elr_plan_step(ctypes.byref(pin), ctypes.byref(pout), ctypes.byref(c), p(scratch), nbytes,
                                          p(grad), dplan.n if grad is not None else 0,
                                          dplan.D if grad is not None else 0, dplan.key_bits if grad is not None else 0,
                                          p(dplan.buf) if grad is not None else None,
                                          dplan.nbytes if grad is not None else 0, _lib.stream_of(u))
        _lib.check(rc, 'elr_plan_step')
        return out
    with _lib.on_device(dev):
        if seg is None:
            rc = _lib.lib().elr_plan_classify(ctypes.byref(pin), ctypes.byref(pout), p(scratch), nbytes,
                                              _lib.stream_of(u))
        else:
            grad, dplan = seg
            n_occ, D = dplan.n, dplan.D
            if not (grad.is_cuda and grad.device == dev and grad.dtype == torch.float32 and grad.is_contiguous()
                    and grad.numel() == n_occ * D):
                raise RuntimeError(f'plan_classify: seg grad must be a contiguous float32 tensor of {n_occ}x{D} on '
                                   f'{dev}')
            rc = _lib.lib().elr_plan_classify_seg(ctypes.byref(pin), ctypes.byref(pout), p(scratch), nbytes,
                                                  grad.data_ptr(), n_occ, D, dplan.key_bits, p(dplan.buf),
                                                  dplan.nbytes, _lib.stream_of(u))
    _lib.check(rc, 'elr_plan_classify' if seg is None else 'elr_plan_classify_seg')
    return out


def classify_from_flags(flags, admit, want_t):
    """Classes from the flags of plan_classify with a changed admission mask (the planner's overflow path,
    srm2/elara.py:244-258 applied to the un-admitted rows)."""
    dev = flags.device
    f = flags.to(torch.int32)
    hit, isN, isL, app = (f & F_HIT) != 0, (f & F_N) != 0, (f & F_L) != 0, (f & F_APP) != 0
    t8 = lambda v: torch.tensor(v, dtype=I8, device=dev)  # noqa: E731
    cls = torch.full(flags.shape, C_S, dtype=I8, device=dev)
    wantT = torch.full(flags.shape, bool(want_t), dtype=torch.bool, device=dev)
    cls = torch.where(~isN & ~isL & (admit | wantT), torch.where(admit, t8(C_FADM), t8(C_FNADM)), cls)
    cls = torch.where(isL, torch.where(admit, t8(C_LADM), torch.where(app, t8(C_LAPP), t8(C_LCMP))), cls)
    cls = torch.where(isN, torch.where(admit, t8(C_NADM), torch.where(app, t8(C_NAPP), t8(C_NCMP))), cls)
    return torch.where(hit, t8(C_HIT), cls)


def plan_admit(adm_rows, adm_slots, lazy_n, evl, s, n0, C, R, K, code, slot_of, slot_row, adm_c0, rj, rok, pstep):
    """Admissions of one step (elr_plan_admit, srm2/elara.py:352-367): row adm_rows[i] takes pool slot
    adm_slots[i]; the first lazy_n rows are N/L rows."""
    n = adm_rows.numel()
    if adm_slots.numel() != n:
        raise RuntimeError('plan_admit: one slot per admitted row')
    if n == 0:
        return
    dev = code.device
    rows = _dev_i64(adm_rows, dev)
    slots = _dev_i64(adm_slots, dev)
    for t, dt, name in ((code, I8, 'code'), (slot_of, I32, 'slot_of'), (slot_row, I64, 'slot_row'),
                        (adm_c0, I8, 'adm_c0'), (rj, I8, 'rj'), (rok, I8, 'rok'), (pstep, I32, 'pstep')):
        if t.dtype != dt or t.device != dev or not t.is_contiguous():
            raise RuntimeError(f'plan_admit: {name} must be a contiguous {dt} tensor on {dev}')
    p = _lib.ptr
    with _lib.on_device(dev):
        rc = _lib.lib().elr_plan_admit(p(rows), p(slots), n, int(lazy_n), int(bool(evl)), int(s), int(n0), int(C),
                                       int(R), int(K), p(code), p(slot_of), p(slot_row), p(adm_c0), p(rj), p(rok),
                                       p(pstep), _lib.stream_of(code))
    _lib.check(rc, 'elr_plan_admit')


def plan_admit_slots(free_stack, n_free, ev_slot, keep, adm_rows, lazy_n, evl, s, n0, C, R, K, code, slot_of, slot_row,
                     adm_c0, rj, rok, pstep, dyn_out):
    """plan_admit with the pool-slot bookkeeping before it, in one launch (elr_plan_admit_slots, srm2/elara.py:345-347,
    352-368): the evicted slots ev_slot are pushed on the free stack free_stack[:n_free] (updated in place; new depth
    n_free + nev - n_adm), its top n_adm entries go to the rows adm_rows, and dyn_out[:nkeep + n_adm] receives keep
    followed by those slots.  Returns the admitted slots (int64 [n_adm])."""
    dev = code.device
    n_adm, nev, nkeep = adm_rows.numel(), ev_slot.numel(), keep.numel()
    for t, name in ((free_stack, 'free_stack'), (dyn_out, 'dyn_out'), (ev_slot, 'ev_slot'), (keep, 'keep'),
                    (adm_rows, 'adm_rows')):
        if t.dtype != I64 or t.device != dev or not t.is_contiguous():
            raise RuntimeError(f'plan_admit_slots: {name} must be a contiguous {I64} tensor on {dev}')
    if free_stack.numel() < n_free + nev or dyn_out.numel() < nkeep + n_adm or n_adm > n_free + nev:
        raise RuntimeError('plan_admit_slots: stack or output too small, or more admissions than free slots')
    _check_state(dev, ((code, I8, 'code'), (slot_of, I32, 'slot_of'), (slot_row, I64, 'slot_row'),
                       (adm_c0, I8, 'adm_c0'), (rj, I8, 'rj'), (rok, I8, 'rok'), (pstep, I32, 'pstep')))
    adm_slots = torch.empty(n_adm, dtype=I64, device=dev)
    a = _lib.SlotsArgs(free_stack.data_ptr(), int(n_free), ev_slot.data_ptr(), nev, keep.data_ptr(), nkeep,
                       adm_slots.data_ptr(), dyn_out.data_ptr())
    p = _lib.ptr
    with _lib.on_device(dev):
        rc = _lib.lib().elr_plan_admit_slots(ctypes.byref(a), p(adm_rows), n_adm, int(lazy_n), int(bool(evl)), int(s),
                                             int(n0), int(C), int(R), int(K), p(code), p(slot_of), p(slot_row),
                                             p(adm_c0), p(rj), p(rok), p(pstep), _lib.stream_of(code))
    _lib.check(rc, 'elr_plan_admit_slots')
    return adm_slots
