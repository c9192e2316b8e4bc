"""Counter-hash row initialisation and exact replay -- drop-in for srm2/gpu_ops.py.

    init_rows(rows, D, seed, bound, out=None) -> [n,3,D]                                  gpu_ops.py:41-48
    ScalarTable(lr, b1, b2, eps, max_step, device).t                                      gpu_ops.py:82-88
    replay_rows(rows, logs, offs, steps, cnt, D, K, seed, bound, table, out=None) -> [n,3,D]  gpu_ops.py:91-99

init: w0[row, j] = (u(row, j) * 2 - 1) * bound with u from a MurmurHash3-fmix32 counter hash of (seed, row, j);
m = v = 0.  replay: init, then for k < cnt the Adam step of logical step steps[k] with gradient logs[offs+k],
bitwise equal to eager gpu_adam at those steps.  Both run as HIP kernels (elara_amd/csrc/init_replay.hip).
"""
import torch

from . import _lib


def _seed32(seed):
    return int(seed) & 0xFFFFFFFF


def init_rows(rows, D, seed, bound, out=None):
    """rows: cuda int64 [n] -> out [n,3,D] (w0, 0, 0).  Allocates `out` when None."""
    n = rows.numel()
    if out is None:
        out = torch.empty(n, 3, D, device=rows.device)
    if n:
        if not rows.is_cuda:
            raise RuntimeError('rows must be a cuda tensor')
        if not (out.is_cuda and out.dtype == torch.float32 and out.is_contiguous() and out.numel() >= n * 3 * D):
            raise RuntimeError(f'out must be a contiguous cuda float32 tensor with at least {n}x3x{D} elements')
        rows = rows.to(torch.int64).contiguous()
        with _lib.on_device(rows.device):
            rc = _lib.lib().elr_init_rows(_lib.ptr(out), _lib.ptr(rows), n, int(D), _seed32(seed), float(bound),
                                         _lib.stream_of(rows))
        _lib.check(rc, 'elr_init_rows')
    return out


def _recip_host(t_host):
    r = torch.empty(t_host.shape[0], 2, dtype=torch.float64)
    _lib.check(_lib.lib().elr_scalar_recip(_lib.ptr(t_host), t_host.shape[0], _lib.ptr(r)), 'elr_scalar_recip')
    return r


class ScalarTable:
    """Per-logical-step Adam scalars [max_step+1, 8] fp32 in HBM; row 0 is zeros, row t = adam_scalars(t).
    Also holds r [max_step+1, 2] fp64 = (1/bc1, 1/bc2) per row, correctly rounded, for the replay kernel."""

    def __init__(self, lr, b1, b2, eps, max_step, device):
        host = torch.empty(int(max_step) + 1, 8, dtype=torch.float32)
        _lib.check(_lib.lib().elr_scalar_table(float(lr), float(b1), float(b2), float(eps), int(max_step),
                                               _lib.ptr(host)), 'elr_scalar_table')
        self.t = host.to(device)
        self.r = _recip_host(host).to(device)


def replay_rows(rows, logs, offs, steps, cnt, D, K, seed, bound, table, out=None, events=None):
    """rows int64 [n]; logs [sum(cnt), D] with row i's entries at offs[i]; steps int32 [n,K]; cnt int32 [n];
    table: ScalarTable (or its [S,8] tensor) -> out [n,3,D].  Allocates `out` when None.  events: optional
    (start, stop) hipEvent_t handles (integers) that the launch itself records at the kernel's start and end
    (elr_replay_rows_timed); not recorded when n == 0."""
    n = rows.numel()
    if out is None:
        out = torch.empty(n, 3, D, device=rows.device)
    if n:
        t = table if isinstance(table, torch.Tensor) else table.t
        r = None if isinstance(table, torch.Tensor) else getattr(table, 'r', None)
        dev = rows.device
        if not (out.is_cuda and out.dtype == torch.float32 and out.is_contiguous() and out.numel() >= n * 3 * D):
            raise RuntimeError(f'out must be a contiguous cuda float32 tensor with at least {n}x3x{D} elements')
        if not (t.is_cuda and t.dtype == torch.float32 and t.dim() == 2 and t.shape[1] == 8):
            raise RuntimeError('table must be a cuda float32 [S,8] tensor')
        if steps.numel() != n * K or cnt.numel() != n or offs.numel() != n:
            raise RuntimeError(f'steps must have {n}x{K} elements and offs/cnt {n}')
        logs = logs.to(torch.float32).contiguous()
        if logs.numel() % D:
            raise RuntimeError(f'logs must be [L,{D}]')
        rows = rows.to(torch.int64).contiguous()
        offs = offs.to(torch.int64).contiguous()
        steps = steps.to(torch.int32).contiguous()
        cnt = cnt.to(torch.int32).contiguous()
        t = t.contiguous()
        if r is None or r.shape != (t.shape[0], 2) or r.device != t.device:
            r = _recip_host(t.cpu().contiguous()).to(dev)   # a bare [S, 8] table: reciprocals computed here
        e0, e1 = events if events is not None else (None, None)
        with _lib.on_device(dev):
            rc = _lib.lib().elr_replay_rows_timed(_lib.ptr(out), _lib.ptr(rows), _lib.ptr(logs), logs.numel() // D,
                                                  _lib.ptr(offs), _lib.ptr(steps), _lib.ptr(cnt), n, int(D), int(K),
                                                  _seed32(seed), float(bound), _lib.ptr(t), _lib.ptr(r), t.shape[0],
                                                  e0, e1, _lib.stream_of(rows))
        _lib.check(rc, 'elr_replay_rows')
    return out
