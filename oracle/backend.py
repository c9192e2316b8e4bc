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

    def unique(self, ids, bound=None):
        """(u, plan): the plan of the oracle's dedup is the inverse (torch.unique, srm2/train.py:352)."""
        return torch.unique(ids, return_inverse=True)

    def unique_async(self, ids, bound=None):
        """(u, plan, None): the oracle's count is known at once."""
        u, inv = torch.unique(ids, return_inverse=True)
        return u, inv, None

    def plan_classify(self, u, u_nexts, slot_of, last_seen, code, kthr, toff, dyn, slot_row, mat_top, log_top, s,
                      K, want_t, loc=None, R=0, carry=False, live=None):
        """Restatement of the planner's classification (srm2/elara.py:214-267) with torch ops on CPU tensors:
        slot lookup and hits (:219-220), next-batch membership (:223-226), admission by TTL or, with carry, by
        next-batch membership (:221), protection of the slots the next batches need through a scatter of their
        slots (:227-229), expiry of unprotected dynamic slots (:231-233; with carry every unprotected slot), class
        per row (:244-258) and the stable class orders (:242, 260-267).  Returns what
        elara_amd.planner.plan_classify returns."""
        from elara_amd.planner import PlanClass
        n = u.numel()
        sl = slot_of[u]
        hit = sl >= 0
        in_next = torch.zeros(n, dtype=torch.bool)
        for un in u_nexts:
            if un.numel():
                j = torch.searchsorted(un, u).clamp(max=un.numel() - 1)
                in_next |= un[j] == u
        admit = ~hit & (in_next if carry else last_seen[u].long() > s)
        C = slot_row.numel()
        prot = torch.zeros(C + 1, dtype=torch.bool)
        for un in u_nexts:
            sn = slot_of[un].long()
            prot[torch.where(sn >= 0, sn, torch.full_like(sn, C))] = True
        dyn = dyn.long()
        unprot = ~prot[dyn]
        exp = unprot if carry else unprot & (last_seen[slot_row[dyn]].long() <= s)
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
        # class ranks: hits; admitted N, L, F; appended N, L; compacted N, L; transient F; S
        lut = torch.tensor([0, 1, 4, 6, 2, 5, 7, 3, 8, 9], dtype=torch.int8)
        order = torch.argsort(lut[cls.long()], stable=True)
        rank = torch.empty_like(order)
        rank[order] = torch.arange(n)
        dcls = torch.where(exp, 0, torch.where(pre, 1, 2)).to(torch.int8)
        dyn_out = torch.cat([dyn[torch.argsort(dcls, stable=True)], dyn[torch.argsort((~exp).to(torch.int8),
                                                                                      stable=True)]])
        counts = torch.cat([torch.bincount(cls.long(), minlength=10),
                            torch.stack([exp.sum(), pre.sum(), (dcls == 2).sum()]),
                            mat_top.reshape(1), log_top.reshape(1),
                            live.reshape(1) if live is not None else torch.zeros(1, dtype=torch.int64),
                            (((u < 0) | (u >= R)).sum() if R > 0 else torch.zeros((), dtype=torch.int64)).reshape(1)])
        # the rows in class order, and the L rows as the reference lists them: its stable class sort puts classes
        # 4, 5, 6 (admitted, append, compact) in that order, each in ascending position (srm2/elara.py:260-267)
        L_sel = [cls == 4, cls == 5, cls == 6]
        L_row = torch.cat([u[m] for m in L_sel])
        L_cnt = torch.cat([c[m] for m in L_sel]).to(torch.int32)
        return PlanClass(cls, flags, sl, c, order, rank, dyn_out, counts, u[order], c[order].long(),
                         sl[order].long(), L_row, L_cnt, loc[u[order]].long() if loc is not None else None)

    def segsum(self, g_occ, inv, U, perm=None):
        """Per-unique-row gradient sums (orc_segment_sum's order), row u into perm[u] when perm is given."""
        out = np.zeros((U, self.D), np.float32)
        if inv.numel():
            u, s, _ = O.segment_sum(inv.numpy().astype(np.int64), np.ascontiguousarray(g_occ.numpy()))
            out[u] = s
        if perm is not None:
            res = np.zeros_like(out)
            res[perm.numpy()] = out
            out = res
        return torch.from_numpy(out)

    def plan_admit(self, adm_rows, adm_slots, lazy_n, evl, s, n0, C, R, K, code, slot_of, slot_row, adm_c0, rj, rok,
                   pstep):
        """Admissions (srm2/elara.py:352-367) with torch ops on CPU tensors."""
        n = adm_rows.numel()
        if n == 0:
            return
        slot_of[adm_rows] = adm_slots.to(torch.int32)
        slot_row[adm_slots] = adm_rows
        c_adm = code[adm_rows].to(torch.int64)
        isIL = torch.arange(n) < lazy_n
        lazy = isIL & bool(evl)
        adm_c0[adm_slots] = torch.where(isIL, c_adm, torch.full_like(c_adm, -1)).to(torch.int8)
        rj[adm_slots] = lazy.to(torch.int8)
        rok[adm_slots] = lazy.to(torch.int8)
        if lazy_n and evl:
            pstep[adm_slots[:lazy_n] - n0, 0] = s

    def assemble(self, rows, segs, L_ids, L_steps, L_cnt, logs, mat, loc, K):
        """Full states of the work rows, segment by segment: oracle init (N), oracle replay of the log entries
        packed row by row (L), copies from the MAT arena at loc[row] (F)."""
        n = rows.numel()
        work = np.empty((n, 3, self.D), np.float32)
        lo = 0
        for end, kind, aux in segs:
            r = rows[lo:end].numpy()
            m = end - lo
            if m:
                if kind == 0:
                    work[lo:end] = O.init_rows(r, self.D, self.seed, self.bound)
                elif kind == 1:
                    cnt = L_cnt[aux:aux + m].numpy().astype(np.int32)
                    ids = L_ids[aux:aux + m].numpy().astype(np.int64)
                    steps = np.ascontiguousarray(L_steps[aux:aux + m].numpy().astype(np.int32))
                    offs = np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.int64)
                    kk = np.arange(K)[None, :]
                    sel = ids[kk < cnt[:, None]]
                    lg = np.ascontiguousarray(logs.numpy()[sel])
                    work[lo:end] = O.replay_rows(r, lg, offs, steps, cnt, self.D, K, self.seed, self.bound,
                                                 self.table, nthreads=self.nthreads)
                else:
                    work[lo:end] = mat.numpy()[loc.numpy()[r].astype(np.int64)]
            lo = end
        return torch.from_numpy(work)

    def adam_dense(self, state, grad, s):
        n = state.shape[0]
        if n:
            self.adam(state, torch.arange(n), grad, s)

    def _view(self, st, pv):
        v = object.__new__(O.DirState)
        for f, t in zip(O.DIR_FIELDS, st):
            setattr(v, f, t.numpy().reshape(-1))
        v.K = int(pv[1])
        return v

    def dir_a(self, st, pv, hs, L_row, L_cnt, ev_slot, s, deferred=False):
        out = O.dir_a(self._view(st, pv), pv, hs.numpy(), L_row.numpy(), L_cnt.numpy(), ev_slot.numpy(), s,
                      deferred=deferred)
        return [torch.from_numpy(np.ascontiguousarray(o)) for o in out]

    def dir_b(self, st, pv, a_rows, a_k, c_rows, c_cnt, s, rel=None):
        rel = None if rel is None else (rel[0].numpy(), rel[1].numpy())
        out = O.dir_b(self._view(st, pv), pv, a_rows.numpy(), a_k.numpy(), c_rows.numpy(), c_cnt.numpy(), s,
                      rel=rel)
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

    def glog_put(self, glog, dyn, j, g, dyn_off=0):
        """glog.index_put_((dyn - dyn_off, j), g) (srm2/elara.py:501, 524); j None: entry 0."""
        nd, K, W = glog.shape
        dd = dyn.long() - dyn_off
        jj = j.long() if j is not None else torch.zeros_like(dd)
        ok = (dd >= 0) & (dd < nd) & (jj >= 0) & (jj < K)
        glog[dd[ok], jj[ok]] = g.reshape(-1, W)[ok]

    def glog_take(self, logs, ids, glog, dyn):
        """The history entries of rows going back to L into the log arena: glog.view(-1, W) rows
        dyn * K + k (srm2/elara.py:396, 507) to logs[ids] (ids < 0: none)."""
        nd, K, W = glog.shape
        src = (dyn.long().clamp(min=0, max=nd - 1)[:, None] * K + torch.arange(K)[None, :]).reshape(-1)
        self.copy_rows(logs, ids.reshape(-1), glog.view(-1, W), src)
