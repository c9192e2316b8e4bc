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

    def plan_classify(self, u, u_nexts, slot_of, last_seen, code, kthr, toff, dyn, slot_row, mat_top, log_top, s,
                      K, want_t):
        """Restatement of the planner's classification (srm2/elara.py:214-267) with torch ops on CPU tensors:
        slot lookup and hits (:219-220), next-batch membership (:223-226), admission by TTL (:221), protection of
        the slots the next batches need through a scatter of their slots (:227-229), expiry of unprotected
        dynamic slots (:231-233), class per row (:244-258) and the stable class orders (:242, 260-267).  Returns
        what elara_amd.planner.plan_classify returns."""
        from elara_amd.planner import PlanClass
        n = u.numel()
        sl = slot_of[u]
        hit = sl >= 0
        in_next = torch.zeros(n, dtype=torch.bool)
        for un in u_nexts:
            if un.numel():
                j = torch.searchsorted(un, u).clamp(max=un.numel() - 1)
                in_next |= un[j] == u
        admit = ~hit & (last_seen[u].long() > s)
        C = slot_row.numel()
        prot = torch.zeros(C + 1, dtype=torch.bool)
        for un in u_nexts:
            sn = slot_of[un].long()
            prot[torch.where(sn >= 0, sn, torch.full_like(sn, C))] = True
        dyn = dyn.long()
        unprot = ~prot[dyn]
        exp = unprot & (last_seen[slot_row[dyn]].long() <= s)
        pre = unprot & ~exp
        c = code[u]
        thr = kthr[torch.searchsorted(toff, u, right=True) - 1]
        isN = c == 0
        isL = (c >= 1) & (c <= K)
        app = c < thr
        t8 = lambda v: torch.tensor(v, dtype=torch.int8)  # noqa: E731
        cls = torch.full((n,), 9, dtype=torch.int8)
        wantT = torch.full((n,), bool(want_t), dtype=torch.bool)
        cls = torch.where(~isN & ~isL & (admit | wantT), torch.where(admit, t8(7), t8(8)), cls)
        cls = torch.where(isL, torch.where(admit, t8(4), torch.where(app, t8(5), t8(6))), cls)
        cls = torch.where(isN, torch.where(admit, t8(1), torch.where(app, t8(2), t8(3))), cls)
        cls = torch.where(hit, t8(0), cls)
        flags = (hit.to(torch.uint8) | (isN.to(torch.uint8) << 1) | (isL.to(torch.uint8) << 2) |
                 (app.to(torch.uint8) << 3) | (admit.to(torch.uint8) << 4) | (in_next.to(torch.uint8) << 5))
        order = torch.argsort(cls, stable=True)
        dcls = torch.where(exp, 0, torch.where(pre, 1, 2)).to(torch.int8)
        dyn_out = torch.cat([dyn[torch.argsort(dcls, stable=True)], dyn[torch.argsort((~exp).to(torch.int8),
                                                                                      stable=True)]])
        counts = torch.cat([torch.bincount(cls.long(), minlength=10),
                            torch.stack([exp.sum(), pre.sum(), (dcls == 2).sum()]),
                            mat_top.reshape(1), log_top.reshape(1), torch.zeros(1, dtype=torch.int64)])
        return PlanClass(cls, flags, sl, c, order, dyn_out, counts)

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
