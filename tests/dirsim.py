"""A small planner that drives the state-directory calls with inputs shaped like ELARA's (test helper).

It follows the structure of srm2/elara.py:209-386 (ELARAPlanner.plan) on host numpy arrays, for one pool of C
slots (n0 static) over T tables: per step a sorted unique batch u, hits = resident rows of u, admissions =
non-resident rows of u that appear in the next batch, evictions = dynamic slots whose row is not in the next batch
(TTL-like), classification of non-hit rows into N/L/F by row code and threshold, then

    elara_dir_a(hit slots, L rows, L counts, evicted slots)      -> admissions (elara.py:345-367)
    elara_dir_b(append rows/k, compaction rows/counts)

Each implementation (the reference's elara_dir.cpp build, the C oracle, the HIP library) keeps its own directory
state; the driver reads the classification inputs (code, slot_of) from the first implementation and applies the
same admission writes to all of them, so their states can be compared after every call.
"""
import numpy as np

from oracle import oracle as O

I8, I32, I64 = np.int8, np.int32, np.int64


class Sim:
    def __init__(self, R=2000, C=300, n0=40, K=3, T=4, seed=0, evl=True, batch=200, kthr=None, vocab_skew=1.1,
                 log_cap=None):
        self.rng = np.random.default_rng(seed)
        self.R, self.C, self.n0, self.K, self.T = R, C, n0, K, T
        self.Cdyn = C - n0
        self.MAT = K + 1
        self.evl = evl
        self.batch = batch
        cuts = np.sort(self.rng.choice(np.arange(1, R), T - 1, replace=False))
        self.toff = np.concatenate([[0], cuts]).astype(I64)
        self.kthr = (np.asarray(kthr, I8) if kthr is not None else self.rng.integers(1, K + 1, T).astype(I8))
        self.Lcap = log_cap or 2 * R
        self.pv = (R, K, self.Lcap, n0, self.Cdyn, self.MAT, R, int(evl))
        # Zipf-like row popularity so rows recur, get hit, evicted and re-admitted
        w = 1.0 / np.arange(1, R + 1) ** vocab_skew
        self.p = w / w.sum()
        self.perm = self.rng.permutation(R)
        self.static_rows = np.sort(self.perm[:n0]).astype(I64)
        # host planner state (elara.py:143-146)
        self.free = np.arange(C - 1, n0 - 1, -1, dtype=I64)
        self.dyn_slots = np.empty(0, I64)
        self.batches = [self._draw() for _ in range(2)]

    def _draw(self):
        ids = self.perm[self.rng.choice(self.R, self.batch, p=self.p)]
        return np.unique(ids).astype(I64)

    def initial_state(self):
        """The 17 arrays with srm2/elara.py:117-148's initial values, as a numpy DirState."""
        st = O.DirState(self.R, self.C, self.K, self.n0, self.toff, self.kthr, log_cap=self.Lcap)
        st.slot_of[self.static_rows] = np.arange(self.n0, dtype=I32)
        st.slot_row[:self.n0] = self.static_rows
        return st

    def step(self, s, impls):
        """One plan step over the implementations (list of objects with view(), dir_a(), admit(), dir_b()).
        Returns the outputs of each implementation: [(outs_a, outs_b), ...]."""
        K, n0 = self.K, self.n0
        u, u_next = self.batches[0], self.batches[1]
        self.batches = [u_next, self._draw()]
        v = impls[0].view()
        code, slot_of, slot_row = v['code'], v['slot_of'], v['slot_row']
        sl = slot_of[u].astype(I64)
        hit = sl >= 0
        in_next = np.isin(u, u_next)
        admit = ~hit & in_next
        dl = self.dyn_slots
        exp = ~np.isin(slot_row[dl], u_next) if dl.size else np.zeros(0, bool)
        o = np.argsort(~exp, kind='stable')
        n_exp = int(exp.sum())
        ev_slot, keep_dyn = dl[o[:n_exp]], dl[o[n_exp:]]
        self.nev_max = max(getattr(self, 'nev_max', 0), int(ev_slot.size))
        c = code[u].astype(I64)
        thr = self.kthr[np.searchsorted(self.toff, u, side='right') - 1].astype(I64)
        isN, isL = c == 0, (c >= 1) & (c <= K)
        app = c < thr
        # overflow: un-admit the last admissions that do not fit the free slots
        n_adm = int(admit.sum())
        room = self.free.size + ev_slot.size
        if n_adm > room:
            drop = np.nonzero(admit)[0][room:]
            admit[drop] = False
            n_adm = room
        cls = np.full(u.size, 9, I64)                      # S (not touched by the directory)
        isF = ~isN & ~isL
        cls[isF & admit] = 7
        cls[isF & ~admit] = 8
        cls[isL & admit] = 4
        cls[isL & ~admit & app] = 5
        cls[isL & ~admit & ~app] = 6
        cls[isN & admit] = 1
        cls[isN & ~admit & app] = 2
        cls[isN & ~admit & ~app] = 3
        cls[hit] = 0
        order = np.argsort(cls, kind='stable')
        pos = {k: order[cls[order] == k] for k in range(10)}
        hit_slot = sl[pos[0]]
        N_row = u[np.concatenate([pos[1], pos[2], pos[3]])]
        L_pos = np.concatenate([pos[4], pos[5], pos[6]])
        L_row, L_cnt = u[L_pos], c[L_pos].astype(I32)
        F_row = u[pos[7]]
        nNa, nNp, nLa, nLp, nFa = (pos[k].size for k in (1, 2, 4, 5, 7))
        outs_a = [m.dir_a(hit_slot, L_row, L_cnt, ev_slot, s) for m in impls]
        # admissions (elara.py:345-367)
        pool_free = np.concatenate([self.free, ev_slot])
        nf = pool_free.size
        adm_slots = pool_free[nf - n_adm:]
        self.free = pool_free[:nf - n_adm]
        adm_rows = np.concatenate([N_row[:nNa], L_row[:nLa], F_row[:nFa]])
        lazy_n = nNa + nLa
        c_adm = impls[0].view()['code'][adm_rows].astype(I64)
        isIL = np.arange(n_adm) < lazy_n
        adm_c0 = np.where(isIL, c_adm, -1).astype(I8)
        lazy = (isIL & self.evl).astype(I8)
        pst = adm_slots[:lazy_n] - n0 if self.evl else np.empty(0, I64)
        for m in impls:
            m.admit(adm_rows, adm_slots, adm_c0, lazy, pst, s)
        self.dyn_slots = np.concatenate([keep_dyn, adm_slots])
        a_rows = np.concatenate([N_row[nNa:nNa + nNp], L_row[nLa:nLa + nLp]]).astype(I64)
        a_k = np.concatenate([np.zeros(nNp, I64), L_cnt[nLa:nLa + nLp].astype(I64)])
        c_rows = np.concatenate([N_row[nNa + nNp:], L_row[nLa + nLp:]]).astype(I64)
        c_cnt = np.concatenate([np.zeros(N_row.size - nNa - nNp, I64), L_cnt[nLa + nLp:].astype(I64)])
        outs_b = [m.dir_b(a_rows, a_k, c_rows, c_cnt, s) for m in impls]
        return list(zip(outs_a, outs_b))


# ------------------------------------------------------------------------------------------------------------
# implementations
class OracleImpl:
    """The C oracle (oracle/elara_oracle.c) on numpy arrays.  triton: the allocation order of the reference's Triton
    directory (srm2/elara_kernels.py): call A keeps the releases of rows going to M for call B, which pushes them
    after its appends and ahead of the compacted rows' logs."""

    def __init__(self, sim, st, triton=False):
        self.sim, self.st, self.triton = sim, st.copy(), triton
        self.rel = None

    def view(self):
        return {f: getattr(self.st, f) for f in O.DIR_FIELDS}

    def dir_a(self, hs, L_row, L_cnt, ev_slot, s):
        out = O.dir_a(self.st, self.sim.pv, hs, L_row, L_cnt, ev_slot, s, deferred=self.triton)
        if self.triton:
            self.rel = (out[4], out[9])
            out = out[:9]
        return out

    def admit(self, rows, slots, adm_c0, lazy, pst, s):
        st = self.st
        st.slot_of[rows] = slots.astype(I32)
        st.slot_row[slots] = rows
        st.adm_c0[slots] = adm_c0
        st.rj[slots] = lazy
        st.rok[slots] = lazy
        st.pstep[pst * self.sim.K] = s

    def dir_b(self, a_rows, a_k, c_rows, c_cnt, s):
        return O.dir_b(self.st, self.sim.pv, a_rows, a_k, c_rows, c_cnt, s, rel=self.rel)


class TorchImpl:
    """The 17 directory tensors on a torch device, driven through a dir_ext()-like module (the reference's
    elara_dir.cpp build on CPU tensors, or elara_amd's HIP directory on the GPU)."""

    def __init__(self, sim, st, ext, device='cpu', triton=False):
        import torch
        self.torch, self.sim, self.ext, self.dev = torch, sim, ext, device
        self.triton, self.rel = triton, None   # triton: elara_amd's deferred-release calls, as OracleImpl
        self.st = [torch.from_numpy(np.ascontiguousarray(getattr(st, f))).to(device) for f in O.DIR_FIELDS]
        self.st[11] = self.st[11].reshape(sim.Cdyn + 1, sim.K)

    def t(self, a, dt=None):
        x = self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)
        return x if dt is None else x.to(dt)

    def view(self):
        return {f: self.st[i].cpu().numpy().reshape(-1) for i, f in enumerate(O.DIR_FIELDS)}

    def dir_a(self, hs, L_row, L_cnt, ev_slot, s):
        torch = self.torch
        kw = {'deferred': True} if self.triton else {}
        out = self.ext.elara_dir_a(self.st, list(self.sim.pv), self.t(hs, torch.int64), self.t(L_row, torch.int64),
                                   self.t(L_cnt, torch.int32), self.t(ev_slot, torch.int64), int(s), **kw)
        if self.triton:
            self.rel = (out[4], out[9])
            out = out[:9]
        return [o.cpu().numpy() for o in out]

    def admit(self, rows, slots, adm_c0, lazy, pst, s):
        torch = self.torch
        rows, slots = self.t(rows, torch.int64), self.t(slots, torch.int64)
        st = self.st
        st[14][rows] = slots.to(torch.int32)
        st[15][slots] = rows
        st[9][slots] = self.t(adm_c0)
        st[10][slots] = self.t(lazy)
        st[16][slots] = self.t(lazy)
        if len(pst):
            st[11][self.t(pst, torch.int64), 0] = int(s)

    def dir_b(self, a_rows, a_k, c_rows, c_cnt, s):
        torch = self.torch
        kw = {'rel': self.rel} if self.triton else {}
        out = self.ext.elara_dir_b(self.st, list(self.sim.pv), self.t(a_rows, torch.int64), self.t(a_k, torch.int64),
                                   self.t(c_rows, torch.int64), self.t(c_cnt, torch.int64), int(s), **kw)
        return [o.cpu().numpy() for o in out]


def comparable_state(view, sim):
    """The directory arrays minus the two trash elements whose contents the reference leaves unspecified
    (lstep[Lcap], lfree[Lcap]: its scatters route every invalid entry there)."""
    v = {k: np.asarray(a).reshape(-1).copy() for k, a in view.items()}
    v['lstep'] = v['lstep'][:sim.Lcap]
    v['lfree'] = v['lfree'][:sim.Lcap]
    return v


def diff_states(a, b):
    """Names of the arrays that differ."""
    return [k for k in a if not np.array_equal(a[k], b[k])]


def diff_outputs(oa, ob):
    bad = []
    for idx, (x, y) in enumerate(zip(oa, ob)):
        x, y = np.asarray(x), np.asarray(y)
        if x.dtype == bool or y.dtype == bool:
            x, y = x.astype(np.uint8), y.astype(np.uint8)
        if x.shape != y.shape or not np.array_equal(x.astype(np.int64), y.astype(np.int64)):
            bad.append(idx)
    return bad


def check_invariants(view, sim):
    """srm2/train.py:474-477 dir_check: live == #valid entries and live + n_lfree == log_top; plus: no log id is
    both live and free, every live id is below log_top, codes match entry counts for L rows."""
    K = sim.K
    ent = np.asarray(view['ent']).reshape(-1)[:sim.R * K].reshape(sim.R, K)
    live = int(view['live'][0])
    n_lfree = int(view['n_lfree'][0])
    log_top = int(view['log_top'][0])
    ids = ent[ent >= 0]
    assert live == ids.size, (live, ids.size)
    assert live + n_lfree == log_top, (live, n_lfree, log_top)
    assert np.unique(ids).size == ids.size, 'a log id is held twice'
    free = np.asarray(view['lfree'])[:n_lfree]
    assert not np.intersect1d(free, ids).size, 'a live log id is on the free stack'
    assert ids.size == 0 or ids.max() < log_top
    code = np.asarray(view['code'])
    isL = (code >= 1) & (code <= K)
    nent = (ent >= 0).sum(1)
    nonres = np.asarray(view['slot_of']) < 0
    # a non-resident L row holds exactly `code` entries
    assert np.array_equal(nent[isL & nonres], code[isL & nonres].astype(np.int64))
    # M rows have a MAT slot
    assert np.all(np.asarray(view['loc'])[:sim.R][code == sim.MAT] >= 0)


class FacadeImpl(TorchImpl):
    """The directory driven through the elara_kernels-style front end (hits / lsteps / Directory), in the call
    sequence of the reference planner's fused path (srm2/elara.py:281-283, 292-293, 312-318, 376-378), and with
    that path's allocation order (compare with OracleImpl(triton=True))."""

    class _Planner:
        pass

    def __init__(self, sim, st, device):
        from elara_amd import elara_kernels
        super().__init__(sim, st, None, device)
        self.ek = elara_kernels
        pl = self._Planner()
        for f, t in zip(O.DIR_FIELDS, self.st):
            setattr(pl, f, t)
        pl.R, pl.Kmax, pl.log_cap, pl.n0, pl.Cdyn = sim.R, sim.K, sim.Lcap, sim.n0, sim.Cdyn
        pl.MAT, pl.mat_trash, pl.evict_logs = sim.MAT, sim.R, sim.evl
        self.pl = pl
        self.dirk = elara_kernels.Directory(pl)

    def dir_a(self, hs, L_row, L_cnt, ev_slot, s):
        torch, pl, K = self.torch, self.pl, self.sim.K
        L_steps, L_ids = self.ek.lsteps(pl, self.t(L_row, torch.int64), self.t(L_cnt, torch.int32))
        hd, hj = self.ek.hits(pl, self.t(hs, torch.int64), int(s))
        ev_slot = self.t(ev_slot, torch.int64)
        ev_row = pl.slot_row[ev_slot]
        if ev_slot.numel():
            pl.slot_of[ev_row] = -1
            pl.slot_row[ev_slot] = -1
        thr = pl.kthr[torch.searchsorted(pl.toff, ev_row, right=True) - 1] if ev_slot.numel() else \
            torch.empty(0, dtype=torch.int8, device=self.dev)
        rep, evl_ids, evf, self.rel_ev = self.dirk.evict(ev_slot, ev_row, thr)
        out = [L_steps, L_ids.to(torch.int32), hd, hj, ev_row, rep.to(torch.bool), evl_ids, evf,
               ev_slot - self.sim.n0]
        assert L_ids.dtype == torch.int64 and L_ids.shape == (L_row.size, K)
        return [o.cpu().numpy() for o in out]

    def dir_b(self, a_rows, a_k, c_rows, c_cnt, s):
        torch = self.torch
        c_rows_t, c_cnt_t = self.t(c_rows, torch.int64), self.t(c_cnt, torch.int64)
        a_ids = self.dirk.appends(self.t(a_rows, torch.int64), self.t(a_k, torch.int64), int(s))
        c_slots = self.dirk.compact(c_rows_t, c_cnt_t)
        self.dirk.release([self.rel_ev, (c_rows_t, c_cnt_t)])
        return [a_ids.cpu().numpy(), c_slots.cpu().numpy()]
