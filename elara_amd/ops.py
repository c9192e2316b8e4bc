"""Row-sparse Adam on HBM-resident (w, m, v) records -- drop-in for srm2/ops.py (gpu_adam, ext().adam_scalars).

    gpu_adam(pool, slots, grad, lr, b1, b2, eps, step)       srm2/ops.py:59-67
    ext().adam_scalars(lr, b1, b2, eps, step) -> [8 floats]  srm2/csrc/srm2_cpu.cpp:255-257
    ext().cpu_adam(state, rows, grad, lr, b1, b2, eps, step, nthreads)
                                                             srm2/csrc/srm2_cpu.cpp:37-56 (host tensors)
    dir_ext().elara_dir_a / elara_dir_b                      srm2/ops.py:32-39 (defined in elara_amd.elara_dir)

The update runs in the HIP kernel behind elr_adam_rows (elara_amd/csrc/adam.hip) on torch's current stream;
there is no other implementation in the product path.
"""
import torch

from . import _lib
from .elara_dir import dir_ext  # noqa: F401  (the reference exposes dir_ext from ops)


def adam_scalars(lr, b1, b2, eps, step):
    """The 8 fp32 Adam scalars of logical step `step` (fp64 arithmetic rounded to fp32), as a list of floats."""
    return list(_scalars8(lr, b1, b2, eps, step))


_SC_CACHE = {}


def _scalars8(lr, b1, b2, eps, step):
    """The same as a ctypes float[8] for the C-ABI, cached per (lr, b1, b2, eps, step): the callers pass it read-only,
    and a training loop asks for the same few steps over and over."""
    key = (float(lr), float(b1), float(b2), float(eps), int(step))
    out = _SC_CACHE.get(key)
    if out is None:
        out = (_lib.c_f32 * 8)()
        _lib.lib().elr_adam_scalars(*key, out)
        if len(_SC_CACHE) > 4096:
            _SC_CACHE.clear()
        _SC_CACHE[key] = out
    return out


def cpu_adam(state, rows, grad, lr, b1, b2, eps, step, nthreads=1):
    """Row-sparse Adam on host tensors (srm2/csrc/srm2_cpu.cpp:37-56, ext().cpu_adam): state [R,3,D] float32 CPU
    (updated in place), rows int64 [n], grad float32 [n,D], on nthreads host threads (elr_cpu_adam).  Non-contiguous
    or non-CPU inputs raise RuntimeError, as the reference's TORCH_CHECK does."""
    if not (state.device.type == 'cpu' and rows.device.type == 'cpu' and grad.device.type == 'cpu'):
        raise RuntimeError('cpu_adam: state, rows and grad must be CPU tensors')
    if not (state.is_contiguous() and grad.is_contiguous() and rows.is_contiguous()):
        raise RuntimeError('cpu_adam: state, rows and grad must be contiguous')
    if state.dtype != torch.float32 or grad.dtype != torch.float32 or rows.dtype != torch.int64 or state.dim() != 3:
        raise RuntimeError('cpu_adam: expected float32 state [R,3,D], int64 rows and float32 grad')
    n, D = rows.numel(), state.shape[2]
    if grad.numel() != n * D:
        raise RuntimeError(f'cpu_adam: grad must hold {n}x{D} elements')
    rc = _lib.lib().elr_cpu_adam(_lib.ptr(state), state.shape[0], _lib.ptr(rows), _lib.ptr(grad), n, D,
                                 _scalars8(lr, b1, b2, eps, step), int(nthreads))
    _lib.check(rc, 'elr_cpu_adam')


class _Ext:
    """Mirror of the reference's `ext()` module for the functions on this path."""

    adam_scalars = staticmethod(adam_scalars)
    cpu_adam = staticmethod(cpu_adam)


_ext = _Ext()


def ext():
    """Counterpart of srm2/ops.py:19-26 ext(): the native helpers (here: adam_scalars and cpu_adam)."""
    _lib.lib()
    return _ext


def _check_state(pool, name='pool'):
    if not (pool.is_cuda and pool.dtype == torch.float32 and pool.dim() == 3 and pool.shape[1] == 3
            and pool.is_contiguous()):
        raise RuntimeError(f'{name} must be a contiguous cuda float32 tensor of shape [C,3,D], got '
                           f'{tuple(pool.shape)} {pool.dtype} {pool.device}')


def check_rows(idx, rows, what='slots'):
    """IndexError unless every entry of idx lies in [0, rows) (one min/max reduction and one host read)."""
    if idx.numel():
        lo, hi = (int(x) for x in torch.aminmax(idx))
        if lo < 0 or hi >= rows:
            raise IndexError(f'{what} out of range: [{lo}, {hi}] not within [0, {rows})')


def gpu_adam(pool, slots, grad, lr, b1, b2, eps, step, events=None, check=False):
    """pool [C,3,D] cuda float32 (updated in place); slots int32/int64 [n] (unique rows of pool); grad [n,D]
    (row i -> slots[i]).  srm2/ops.py:59-67.  pool may also be a pinned host arena (the capacity tier): the kernel
    then updates it over the host link.  events: optional (start, stop) hipEvent_t handles (integers) that the launch
    itself records at the kernel's start and end (elr_adam_rows_timed); not recorded when n == 0.  A slot outside
    [0, C) is skipped by the kernel (the reference leaves it undefined); check=True raises IndexError for it first,
    at the cost of a host synchronisation."""
    n = slots.numel()
    if n == 0:
        return
    if check:
        check_rows(slots, pool.shape[0])
    if pool.is_cuda:
        _check_state(pool)
    elif not (_lib.is_arena(pool) and pool.dim() == 3 and pool.shape[1] == 3):
        raise RuntimeError('pool must be a contiguous float32 [C,3,D] tensor on the GPU or in pinned host memory')
    D = pool.shape[2]
    dev = slots.device
    if slots.dtype not in (torch.int32, torch.int64) or not slots.is_cuda or (pool.is_cuda and dev != pool.device):
        raise RuntimeError(f'slots must be a cuda int32/int64 tensor on {pool.device}')
    if not (grad.is_cuda and grad.dtype == torch.float32 and grad.device == dev and grad.numel() == n * D):
        raise RuntimeError(f'grad must be a cuda float32 tensor with {n}x{D} elements on {dev}')
    slots = slots.contiguous()
    grad = grad.contiguous()
    s = _scalars8(lr, b1, b2, eps, step)
    L = _lib.lib()
    e0, e1 = events if events is not None else (None, None)
    with _lib.on_device(dev):
        rc = L.elr_adam_rows_timed(_lib.dptr(pool), pool.shape[0], _lib.ptr(slots), int(slots.dtype == torch.int64),
                                   _lib.ptr(grad), n, D, s, e0, e1, _lib.stream_of(grad))
    _lib.check(rc, 'elr_adam_rows')


def adam_rows_dense(state, grad, lr, b1, b2, eps, step):
    """state [n,3,D] cuda float32 (contiguous; updated in place) with grad [n,D], row i by row i (elr_adam_rows with
    no slot list: the executor's contiguous work arrays)."""
    n = state.shape[0]
    if n == 0:
        return
    _check_state(state, 'state')
    D = state.shape[2]
    if not (grad.is_cuda and grad.dtype == torch.float32 and grad.device == state.device and grad.numel() == n * D):
        raise RuntimeError(f'grad must be a cuda float32 tensor with {n}x{D} elements on {state.device}')
    grad = grad.contiguous()
    s = _scalars8(lr, b1, b2, eps, step)
    with _lib.on_device(state.device):
        rc = _lib.lib().elr_adam_rows(_lib.ptr(state), n, None, 1, _lib.ptr(grad), n, D, s, _lib.stream_of(state))
    _lib.check(rc, 'elr_adam_rows')
