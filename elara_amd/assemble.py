"""Fused weight assembly of one ELARA step on the GPU (elr_assemble): srm2/elara.py:471-489.

assemble_rows(rows, segs, ...) returns the full states [n, 3, D] of the step's non-resident rows in one launch:
each segment of work positions is of one kind -- counter-hash init (N rows), init plus exact replay of the row's
log entries read by entry id (L rows), or a copy from the MAT arena at loc[row] (F rows).
"""
import ctypes

import torch

from . import _lib

I32, I64 = torch.int32, torch.int64
KINDS = (0, 1, 2)   # ELR_ASM_INIT, ELR_ASM_REPLAY, ELR_ASM_GATHER
MAX_SEG = 16


def assemble_rows(rows, segs, L_ids, L_steps, L_cnt, logs, mat, loc, K, D, seed, bound, table):
    """rows int64 [n] (work order); segs: list of (end, kind, aux) with ascending ends, the last equal to n (aux:
    the first L row of a replay segment in L_ids / L_steps / L_cnt, elr_dir_a's int32 [nL, K] replay inputs);
    logs [nlogs, D], mat [M, 3, D] float32 (on the GPU or pinned host arenas), loc int32 [R + 1]; table: a
    gpu_ops.ScalarTable.  Returns the work array [n, 3, D]."""
    dev = rows.device
    n = rows.numel()
    work = torch.empty(n, 3, D, dtype=torch.float32, device=dev)
    if n == 0:
        return work
    if not 1 <= len(segs) <= MAX_SEG:
        raise RuntimeError(f'assemble_rows: 1..{MAX_SEG} segments')
    rows = rows.to(I64).contiguous()
    L_ids, L_steps, L_cnt = (t.to(device=dev, dtype=I32).contiguous() for t in (L_ids, L_steps, L_cnt))
    for t, name in ((logs, 'logs'), (mat, 'mat')):
        if not (_lib.is_arena(t) and t.shape[-1] == D):
            raise RuntimeError(f'assemble_rows: {name} must be a contiguous float32 tensor of width {D} on the GPU '
                               f'or in pinned host memory')
    if loc.dtype != I32 or not loc.is_contiguous():
        raise RuntimeError('assemble_rows: loc must be a contiguous int32 tensor')
    a = _lib.AssembleArgs()
    a.work, a.rows, a.n, a.D, a.K = work.data_ptr(), rows.data_ptr(), n, int(D), int(K)
    a.nseg = len(segs)
    for g, (end, kind, aux) in enumerate(segs):
        if kind not in KINDS:
            raise RuntimeError(f'assemble_rows: unknown segment kind {kind}')
        a.seg_end[g], a.seg_kind[g], a.seg_aux[g] = int(end), int(kind), int(aux)
    a.seed, a.bound = int(seed) & 0xFFFFFFFF, float(bound)
    a.L_ids, a.L_steps, a.L_cnt, a.nL = L_ids.data_ptr(), L_steps.data_ptr(), L_cnt.data_ptr(), L_cnt.numel()
    a.logs, a.nlogs = _lib.dptr(logs).value, logs.shape[0]
    a.table, a.recip, a.table_rows = table.t.data_ptr(), table.r.data_ptr(), table.t.shape[0]
    a.mat, a.mat_rows = _lib.dptr(mat).value, mat.shape[0]
    a.loc, a.R = loc.data_ptr(), loc.numel() - 1
    with _lib.on_device(dev):
        rc = _lib.lib().elr_assemble(ctypes.byref(a), _lib.stream_of(work))
    _lib.check(rc, 'elr_assemble')
    return work
