"""Row copies in HBM (or between HBM and pinned host arenas): gradient-log appends and the executor's row gathers
and scatters.

    log_append(logs, ids, g)            logs[ids] = g          srm2/elara.py:569-570 (host cpu_scatter into the log
                                                               arena; the arena is in HBM here), and the
                                                               resident-history record glog.index_put_((dyn, j), g)
                                                               (srm2/elara.py:501, 524) with ids = dyn * K + j
    copy_rows(dst, dst_idx, src, src_idx)
                                        dst[dst_idx] = src[src_idx] (None = all rows in order)

Both run the HIP kernel behind elr_copy_rows (elara_amd/csrc/rows.hip) on torch's current stream.  Rows are the
trailing dimensions flattened (a [C,3,D] state has rows of 3*D floats).
"""
import ctypes

import torch

from . import _lib


def _rows2d(t, name):
    if not (_lib.is_arena(t) and t.dim() >= 1):
        raise RuntimeError(f'{name} must be a contiguous float32 tensor on the GPU or in pinned host memory')
    n = t.shape[0]
    return n, (t.numel() // n if n else 0)


def _device(*ts):
    for t in ts:
        if t is not None and t.is_cuda:
            return t.device
    raise RuntimeError('copy_rows: at least one of dst, src and the indices must be on the GPU')


def _index(idx, dev, name):
    if idx is None:
        return None
    if not (idx.is_cuda and idx.device == dev and idx.dtype in (torch.int32, torch.int64)):
        raise RuntimeError(f'{name} must be a cuda int32/int64 tensor on {dev}')
    return idx.reshape(-1).to(torch.int64).contiguous()


def copy_rows(dst, dst_idx, src, src_idx=None):
    """dst[dst_idx[i]] = src[src_idx[i]] for every i (rows of the same width); indices out of range are skipped."""
    nd, wd = _rows2d(dst, 'dst')
    ns, ws = _rows2d(src, 'src')
    dev = _device(dst, src, dst_idx, src_idx)
    di, si = _index(dst_idx, dev, 'dst_idx'), _index(src_idx, dev, 'src_idx')
    n = di.numel() if di is not None else (si.numel() if si is not None else ns)
    if si is not None and di is not None and si.numel() != n:
        raise RuntimeError('dst_idx and src_idx must have the same length')
    if si is None and n > ns:
        raise RuntimeError(f'src has {ns} rows, {n} needed')
    if n == 0:
        return dst
    if wd != ws:
        raise RuntimeError(f'row widths differ: {wd} vs {ws}')
    with _lib.on_device(dev):
        rc = _lib.lib().elr_copy_rows(_lib.dptr(dst), nd, _lib.ptr(di), _lib.dptr(src), ns, _lib.ptr(si), n, wd,
                                      ctypes.c_void_p(_lib.raw_stream(dev)))
    _lib.check(rc, 'elr_copy_rows')
    return dst


def log_append(logs, ids, g):
    """logs[ids[i]] = g[i]: append gradient rows to the log arena at their allocated log ids."""
    return copy_rows(logs, ids, g, None)


def _i64(t, dev, name):
    if not (t.is_cuda and t.device == dev and t.dtype == torch.int64):
        raise RuntimeError(f'{name} must be a cuda int64 tensor on {dev}')
    return t.reshape(-1).contiguous()


def glog_put(glog, dyn, j, g, dyn_off=0):
    """glog.index_put_((dyn - dyn_off, j), g) (srm2/elara.py:501, 524): glog [nd, K, W] cuda float32, dyn / j int64
    [n] (j None: entry 0), g [n, W].  Items whose slot or entry is out of range are skipped."""
    if not (glog.is_cuda and glog.dtype == torch.float32 and glog.is_contiguous() and glog.dim() == 3):
        raise RuntimeError('glog must be a contiguous cuda float32 [nd, K, W] tensor')
    dev = glog.device
    nd, K, W = glog.shape
    dyn = _i64(dyn, dev, 'dyn')
    n = dyn.numel()
    if j is not None:
        j = _i64(j, dev, 'j')
        if j.numel() != n:
            raise RuntimeError('j must match dyn')
    if not (g.is_cuda and g.device == dev and g.dtype == torch.float32 and g.is_contiguous() and g.numel() == n * W):
        raise RuntimeError(f'g must be a contiguous cuda float32 tensor with {n}x{W} elements')
    if n == 0:
        return glog
    with _lib.on_device(dev):
        rc = _lib.lib().elr_glog_put(_lib.ptr(glog), nd, K, _lib.ptr(dyn), int(dyn_off), _lib.ptr(j), _lib.ptr(g), n,
                                     W, ctypes.c_void_p(_lib.raw_stream(dev)))
    _lib.check(rc, 'elr_glog_put')
    return glog


def glog_take(logs, ids, glog, dyn):
    """logs[ids[r*K + k]] = glog[clamp(dyn[r], 0, nd-1), k] for every row r and entry k (ids < 0: none): the
    history entries of evicted rows going back to L, moved into the log arena (srm2/elara.py:396, 507, 569-570).
    logs [nlogs, W] (GPU or pinned host arena), ids int64 [n*K], glog [nd, K, W], dyn int64 [n]."""
    if not (glog.is_cuda and glog.dtype == torch.float32 and glog.is_contiguous() and glog.dim() == 3):
        raise RuntimeError('glog must be a contiguous cuda float32 [nd, K, W] tensor')
    dev = glog.device
    nd, K, W = glog.shape
    nl, wl = _rows2d(logs, 'logs')
    if wl != W:
        raise RuntimeError(f'row widths differ: {wl} vs {W}')
    dyn, ids = _i64(dyn, dev, 'dyn'), _i64(ids, dev, 'ids')
    n = dyn.numel()
    if ids.numel() != n * K:
        raise RuntimeError('ids must hold K entries per row of dyn')
    if n == 0:
        return logs
    with _lib.on_device(dev):
        rc = _lib.lib().elr_glog_take(_lib.dptr(logs), nl, _lib.ptr(ids), _lib.ptr(glog), nd, K, _lib.ptr(dyn), n, W,
                                      ctypes.c_void_p(_lib.raw_stream(dev)))
    _lib.check(rc, 'elr_glog_take')
    return logs


def mark_rows(rows, n_dev, value, out, bits=None, bit=0):
    """out[rows[i]] = value for i < n_dev (a device int64 count; rows beyond it are ignored), with no
    synchronisation: rows int64 [n_max] cuda (distinct), out int32 [R] cuda.  With bits (int32 [R] cuda, the
    planner's ring of loaded batches), also bits[rows[i]] |= bit."""
    if not (rows.is_cuda and rows.dtype == torch.int64 and out.is_cuda and out.dtype == torch.int32
            and n_dev.is_cuda and n_dev.dtype == torch.int64 and out.is_contiguous()):
        raise RuntimeError('mark_rows: rows int64, n_dev int64 and out int32 cuda tensors')
    if bits is not None and not (bits.is_cuda and bits.dtype == torch.int32 and bits.is_contiguous()
                                 and bits.numel() >= out.numel()):
        raise RuntimeError('mark_rows: bits must be a contiguous cuda int32 tensor covering out')
    rows = rows.contiguous()
    with _lib.on_device(out.device):
        rc = _lib.lib().elr_mark_rows(_lib.ptr(rows), _lib.ptr(n_dev), rows.numel(), int(value), _lib.ptr(out),
                                      out.numel(), _lib.ptr(bits), int(bit) & 0xFFFFFFFF,
                                      ctypes.c_void_p(_lib.raw_stream(out.device)))
    _lib.check(rc, 'elr_mark_rows')
