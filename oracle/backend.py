"""The hot-path kernels of elara_amd.step.ElaraStep implemented by the CPU oracle -- TEST INFRASTRUCTURE ONLY (used
by tests/ and __graft_entry__.smoke()): the same step, on CPU tensors, with every kernel replaced by its oracle
restatement (oracle/elara_oracle.c)."""
import numpy as np
import torch

from . import oracle as O

DT = dict(code=np.int8, loc=np.int32, ent=np.int32, lstep=np.int32, lfree=np.int32)


class OracleBackend:
    def __init__(self, D, seed, bound, hp, max_step, nthreads=8):
        self.D, self.seed, self.bound, self.hp, self.nthreads = D, seed, bound, hp, nthreads
        self.table = O.scalar_table(*hp, max_step)

    def unique(self, ids):
        return torch.unique(ids, return_inverse=True)

    def segsum(self, g_occ, inv, U):
        out = np.zeros((U, self.D), np.float32)
        if inv.numel():
            u, s, _ = O.segment_sum(inv.numpy().astype(np.int64), np.ascontiguousarray(g_occ.numpy()))
            out[u] = s
        return torch.from_numpy(out)

    def _view(self, st, pv):
        v = object.__new__(O.DirState)
        for f, t in zip(O.DIR_FIELDS, st):
            setattr(v, f, t.numpy().reshape(-1))
        v.K = int(pv[1])
        return v

    def dir_a(self, st, pv, hs, L_row, L_cnt, ev_slot, s):
        out = O.dir_a(self._view(st, pv), pv, hs.numpy(), L_row.numpy(), L_cnt.numpy(), ev_slot.numpy(), s)
        return [torch.from_numpy(np.ascontiguousarray(o)) for o in out]

    def dir_b(self, st, pv, a_rows, a_k, c_rows, c_cnt, s):
        out = O.dir_b(self._view(st, pv), pv, a_rows.numpy(), a_k.numpy(), c_rows.numpy(), c_cnt.numpy(), s)
        return [torch.from_numpy(o) for o in out]

    def init_rows(self, rows):
        return torch.from_numpy(O.init_rows(rows.numpy(), self.D, self.seed, self.bound))

    def replay(self, rows, logs, offs, steps, cnt, K):
        n = rows.numel()
        if n == 0:
            return torch.empty(0, 3, self.D)
        out = O.replay_rows(rows.numpy(), logs.numpy(), offs.numpy(), steps.numpy(), cnt.numpy(), self.D, K,
                            self.seed, self.bound, self.table, nthreads=self.nthreads)
        return torch.from_numpy(out)

    def adam(self, state, slots, grad, s):
        assert state.is_contiguous()
        O.cpu_adam(state.numpy(), slots.numpy().astype(np.int64), np.ascontiguousarray(grad.numpy()),
                   O.adam_scalars(*self.hp, s), self.nthreads)

    def copy_rows(self, dst, dst_idx, src, src_idx=None):
        nd, ns = dst.shape[0], src.shape[0]
        D2 = dst.reshape(nd, -1).numpy()
        S2 = src.reshape(ns, -1).numpy()
        n = dst_idx.numel() if dst_idx is not None else (src_idx.numel() if src_idx is not None else ns)
        d = dst_idx.numpy().astype(np.int64) if dst_idx is not None else np.arange(n)
        s_ = src_idx.numpy().astype(np.int64) if src_idx is not None else np.arange(n)
        ok = (d >= 0) & (d < nd) & (s_ >= 0) & (s_ < ns)
        D2[d[ok]] = S2[s_[ok]]
