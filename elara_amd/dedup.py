"""Batch dedup and duplicate-id gradient reduction on the GPU -- the step before Adam on every batch.

    unique(ids) -> (u, inv)                       torch.unique(ids, return_inverse=True), srm2/train.py:352
    unique_plan(ids, D) -> (u, plan); segment_sum_plan(grad, plan, out, perm)
                                                  the same dedup sorted once per batch: the segment sum of the
                                                  backward reuses the sort of the unique
    embedding_dense_backward(grad, inv, num_weights, padding_idx=-1, scale_grad_by_freq=False) -> [num_weights, D]
                                                  aten.embedding_dense_backward as srm2/train.py:429 calls it
    adam_dedup(pool, ids, grad, lr, b1, b2, eps, step)
                                                  dedup + segment sum in ATen's order + row-sparse Adam on pool[id]
                                                  (config C3: one Adam step per unique id of a batch)

Summation order of duplicate ids: ATen's embedding_dense_backward as it runs on this GPU (third-party code the
reference calls; aten/src/ATen/native/cuda/Embedding.cu, EmbeddingBackwardKernel.cu).  Up to 3072 indices, per
window of 16 consecutive indices an id's gradients are summed left to right and the window sums are added into a
zeroed row; above 3072, an id's occurrences in ascending index are cut into runs of 10, each run summed from zero,
and the run sums added from zero.  Equal bits to torch.ops.aten.embedding_dense_backward on the same inputs.  All
of it runs as HIP kernels (elara_amd/csrc/dedup.hip) on torch's current stream.
"""
import torch

from . import _lib
from .ops import _check_state, _scalars8, check_rows

I64 = torch.int64


def _scratch(dev, n, D):
    nbytes = int(_lib.lib().elr_dedup_scratch_bytes(int(n), int(D)))
    if nbytes < 0:
        _lib.check(nbytes, 'elr_dedup_scratch_bytes')
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev), nbytes


def _ids(ids, name='ids'):
    if not ids.is_cuda:
        raise RuntimeError(f'{name} must be a cuda tensor')
    if ids.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(f'{name} must be int32 or int64')
    return ids.reshape(-1).to(I64).contiguous()


def _bits(bound):
    b = 1
    while b < 63 and (1 << b) < bound:
        b += 1
    return b


def _key_bits(flat, bound):
    if bound is not None:
        return _bits(int(bound))
    lo, hi = torch.aminmax(flat)
    lo, hi = int(lo), int(hi)
    if lo < 0:
        raise RuntimeError('unique: ids must be non-negative')
    return _bits(hi + 1)


def unique(ids, bound=None):
    """Sorted unique values of `ids` (int32/int64, >= 0) and the inverse, as torch.unique(ids, sorted=True,
    return_inverse=True) returns them (int64).  Synchronises once to size the output, as torch.unique does.  With
    `bound` (every id < bound, the caller's guarantee) the key width comes from it instead of a min/max pass and
    its synchronisation."""
    flat = _ids(ids)
    n = flat.numel()
    dev = flat.device
    inv = torch.empty(ids.shape, dtype=I64, device=dev)
    if n == 0:
        return torch.empty(0, dtype=I64, device=dev), inv
    kb = _key_bits(flat, bound)
    u = torch.empty(n, dtype=I64, device=dev)
    nu = torch.empty(1, dtype=I64, device=dev)
    scratch, nbytes = _scratch(dev, n, 1)
    with _lib.on_device(dev):
        rc = _lib.lib().elr_unique(_lib.ptr(flat), n, kb, _lib.ptr(u), _lib.ptr(inv), _lib.ptr(nu),
                                   _lib.ptr(scratch), nbytes, _lib.stream_of(flat))
    _lib.check(rc, 'elr_unique')
    return u[:int(nu)], inv


class DedupPlan:
    """One batch's sort and segment layout (elr_dedup_plan), kept for elr_segment_sum_plan."""
    __slots__ = ('buf', 'nbytes', 'n', 'D', 'key_bits', 'U')


def field_bounds(lo):
    """Host int64 array of a batch's field bounds for unique_plan(fields=...): nfields + 1 ascending values, field
    c's ids in [lo[c], lo[c + 1])."""
    import numpy as np
    a = np.ascontiguousarray(np.asarray(lo, dtype=np.int64))
    if a.ndim != 1 or a.size < 2 or a[0] < 0 or bool((a[1:] < a[:-1]).any()):
        raise RuntimeError('field bounds must be at least two ascending non-negative values')
    return a


def unique_plan(ids, D, bound=None, fields=None):
    """unique(ids) without the inverse, keeping the sort as a plan for segment_sum_plan over gradients of width D:
    returns (u, plan).  fields: see unique_plan_async."""
    u, plan, nu = unique_plan_async(ids, D, bound, fields=fields)
    if nu is not None:
        plan.U = int(nu)
        u = u[:plan.U]
    return u, plan


def plan_bytes(n, D):
    """Bytes of the plan buffer of a batch of n ids for gradients of width D (elr_dedup_plan_bytes)."""
    nbytes = int(_lib.lib().elr_dedup_plan_bytes(int(n), int(D)))
    if nbytes < 0:
        _lib.check(nbytes, 'elr_dedup_plan_bytes')
    return nbytes


def unique_plan_async(ids, D, bound=None, nu_out=None, out=None, fields=None):
    """unique_plan without reading the unique count: returns (u_full, plan, nu) with u_full [n] whose first nu
    entries are the unique ids, nu the count on the device (None when n == 0).  Set plan.U once nu is known.
    nu_out (int64 [1] on the device, optional): where the count goes, else a new tensor.
    out (optional): (buf, u, nu) to write into instead of new tensors -- uint8 buf of at least plan_bytes(n, D)
    bytes, int64 u of at least n elements, int64 nu [1] (nu_out, if given, takes its place); the caller keeps them
    from being reused before the GPU's work on the plan is done.
    fields (optional, field_bounds(...)): the batch is laid out by field -- (sample, field) order, field c's ids in
    [fields[c], fields[c + 1]) -- and is sorted per field (elr_dedup_plan_fields): the same plan, in three launches.
    An id outside its field's rows comes out as -1 in u.  Batches whose size is not a multiple of the field count
    take the general sort."""
    flat = _ids(ids)
    n = flat.numel()
    dev = flat.device
    plan = DedupPlan()
    plan.n, plan.D, plan.U = n, int(D), 0
    plan.buf, plan.nbytes, plan.key_bits = None, 0, 1
    if n == 0:
        return torch.empty(0, dtype=I64, device=dev), plan, None
    plan.key_bits = _key_bits(flat, bound)
    nbytes = plan_bytes(n, D)
    if out is not None:
        buf, u, nu0 = out
        if not (buf.dtype == torch.uint8 and buf.device == dev and buf.numel() >= nbytes and buf.is_contiguous()
                and u.dtype == I64 and u.device == dev and u.numel() >= n and u.is_contiguous()):
            raise RuntimeError(f'out must hold a uint8 buffer of {nbytes} bytes and an int64 tensor of {n} '
                               f'elements on {dev}')
        plan.buf, plan.nbytes = buf, nbytes
        u = u[:n]
        if nu_out is None:
            nu_out = nu0
    else:
        plan.buf, plan.nbytes = torch.empty(nbytes, dtype=torch.uint8, device=dev), nbytes
        u = torch.empty(n, dtype=I64, device=dev)
    if nu_out is not None and not (nu_out.dtype == I64 and nu_out.device == dev and nu_out.numel() == 1):
        raise RuntimeError(f'nu_out must be an int64 tensor of one element on {dev}')
    nu = nu_out if nu_out is not None else torch.empty(1, dtype=I64, device=dev)
    nf = 0 if fields is None else fields.size - 1
    with _lib.on_device(dev):
        if nf > 0 and n % nf == 0:
            rc = _lib.lib().elr_dedup_plan_fields(_lib.ptr(flat), n // nf, nf, fields.ctypes.data, plan.key_bits,
                                                  _lib.ptr(u), None, _lib.ptr(nu), _lib.ptr(plan.buf), nbytes, int(D),
                                                  _lib.stream_of(flat))
            _lib.check(rc, 'elr_dedup_plan_fields')
            return u, plan, nu
        rc = _lib.lib().elr_dedup_plan(_lib.ptr(flat), n, plan.key_bits, _lib.ptr(u), None, _lib.ptr(nu),
                                       _lib.ptr(plan.buf), nbytes, int(D), _lib.stream_of(flat))
    _lib.check(rc, 'elr_dedup_plan')
    return u, plan, nu


def segment_sum_plan(grad, plan, out=None, perm=None, partials_done=False):
    """Per-segment sums of grad [n, D] over a unique_plan: segment u into row perm[u] (or u) of out [rows, D]
    (allocated [U, D] when None), in embedding_dense_backward's summation order for n = plan.n indices.
    partials_done: the partial chunks of these gradients over this plan were computed already (planner.plan_classify
    with seg=(grad, plan)); only the rest of the sum is queued (elr_segment_sum_plan_final)."""
    n, D = plan.n, plan.D
    if not (grad.is_cuda and grad.dtype == torch.float32 and grad.numel() == n * D):
        raise RuntimeError(f'grad must be a cuda float32 tensor with {n}x{D} elements')
    dev = grad.device
    if out is None:
        out = torch.empty(plan.U, D, dtype=torch.float32, device=dev)
    if not (out.is_cuda and out.dtype == torch.float32 and out.is_contiguous() and out.dim() == 2
            and out.shape[1] == D):
        raise RuntimeError(f'out must be a contiguous cuda float32 tensor [rows, {D}]')
    if perm is not None:
        if perm.dtype != I64 or not perm.is_cuda or perm.numel() < plan.U:
            raise RuntimeError('perm must be a cuda int64 tensor with one row per segment')
        perm = perm.contiguous()
    if n == 0:
        return out
    g = grad.reshape(n, D).contiguous()
    with _lib.on_device(dev):
        fn = _lib.lib().elr_segment_sum_plan_final if partials_done else _lib.lib().elr_segment_sum_plan
        rc = fn(_lib.ptr(g), n, D, plan.key_bits, _lib.ptr(plan.buf), plan.nbytes, _lib.ptr(perm), _lib.ptr(out),
                out.shape[0], _lib.stream_of(g))
    _lib.check(rc, 'elr_segment_sum_plan_final' if partials_done else 'elr_segment_sum_plan')
    return out


def embedding_dense_backward(grad_output, indices, num_weights, padding_idx=-1, scale_grad_by_freq=False):
    """[num_weights, D] per-row sums of grad_output [n, D] over indices [n] (rows without an index are zero), in
    ATen's summation order.  Supports the reference's call (padding_idx=-1, no frequency scaling)."""
    if padding_idx != -1 or scale_grad_by_freq:
        raise RuntimeError('embedding_dense_backward: only padding_idx=-1 and scale_grad_by_freq=False are supported')
    idx = _ids(indices, 'indices')
    n = idx.numel()
    D = grad_output.shape[-1]
    if not (grad_output.is_cuda and grad_output.dtype == torch.float32 and grad_output.numel() == n * D):
        raise RuntimeError(f'grad_output must be a cuda float32 tensor with {n}x{D} elements')
    dev = idx.device
    out = torch.zeros(int(num_weights), D, dtype=torch.float32, device=dev)
    if n == 0:
        return out
    g = grad_output.reshape(n, D).contiguous()
    scratch, nbytes = _scratch(dev, n, D)
    with _lib.on_device(dev):
        rc = _lib.lib().elr_segment_sum(_lib.ptr(g), _lib.ptr(idx), n, D, int(num_weights), _lib.ptr(out),
                                        _lib.ptr(scratch), nbytes, _lib.stream_of(g))
    _lib.check(rc, 'elr_segment_sum')
    return out


def adam_dedup_plan(pool, u, grad, plan, lr, b1, b2, eps, step):
    """adam_dedup over a dedup plan made earlier for the same ids (unique_plan / unique_plan_async, for instance
    queued on another stream a step ahead): u is that call's unique ids (u_full of unique_plan_async: its first
    U entries, U read on the device), grad [n, D] the occurrence gradients in the ids' order."""
    n, D = plan.n, plan.D
    if n == 0:
        return
    _check_state(pool)
    if pool.shape[2] != D:
        raise RuntimeError(f'adam_dedup_plan: pool rows of width {pool.shape[2]}, plan of width {D}')
    if not (grad.is_cuda and grad.dtype == torch.float32 and grad.numel() == n * D):
        raise RuntimeError(f'grad must be a cuda float32 tensor with {n}x{D} elements')
    if not (u.is_cuda and u.dtype == I64 and u.is_contiguous() and u.numel() >= plan.U):
        raise RuntimeError('adam_dedup_plan: u must be the plan\'s contiguous int64 unique ids')
    g = grad.reshape(n, D).contiguous()
    dev = pool.device
    s = _scalars8(lr, b1, b2, eps, step)
    with _lib.on_device(dev):
        rc = _lib.lib().elr_adam_dedup_plan(_lib.ptr(pool), pool.shape[0], _lib.ptr(u), _lib.ptr(g), n, D,
                                            plan.key_bits, _lib.ptr(plan.buf), plan.nbytes, s, _lib.stream_of(pool))
    _lib.check(rc, 'elr_adam_dedup_plan')


def adam_dedup(pool, ids, grad, lr, b1, b2, eps, step, check=False):
    """pool [C,3,D] cuda float32 (updated in place); ids int32/int64 [n] rows of pool, repeats allowed; grad [n,D]
    (row i belongs to ids[i]).  Each unique id gets one Adam step with the sum of its gradients.  An id outside
    [0, C) is skipped; check=True raises IndexError for it first (one host synchronisation)."""
    idx = _ids(ids)
    n = idx.numel()
    if n == 0:
        return
    if check:
        check_rows(idx, pool.shape[0], 'ids')
    _check_state(pool)
    D = pool.shape[2]
    if not (grad.is_cuda and grad.dtype == torch.float32 and grad.numel() == n * D):
        raise RuntimeError(f'grad must be a cuda float32 tensor with {n}x{D} elements')
    g = grad.reshape(n, D).contiguous()
    dev = pool.device
    scratch, nbytes = _scratch(dev, n, D)
    s = _scalars8(lr, b1, b2, eps, step)
    with _lib.on_device(dev):
        rc = _lib.lib().elr_adam_dedup(_lib.ptr(pool), pool.shape[0], _lib.ptr(idx), _lib.ptr(g), n, D, s,
                                       _lib.ptr(scratch), nbytes, _lib.stream_of(pool))
    _lib.check(rc, 'elr_adam_dedup')
