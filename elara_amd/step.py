"""One ELARA training step with every arena in HBM (config C5): the caller of the sparse-update path.

Counterpart of srm2/elara.py ELARAPlanner.plan (209-414, the `cpp` directory path) and ELARAExecutor.assemble /
update (471-542) plus the host worker's writes (544-580), for a single GPU that holds everything:
    - the pool of C resident full states (n0 static hot rows pinned, C - n0 dynamic slots with TTL residency);
    - the MAT arena (full states of materialised rows) and the log arena (gradient-log entries), both in HBM, in
      place of the reference's host arenas (srm2/elara.py:40-103);
    - the state directory (elr_dir_a / elr_dir_b) and the resident histories glog.
Per step: plan (classify the batch's unique rows into hit / N / L / F / S classes, directory call A, admissions,
directory call B), assemble (counter-hash init of N rows, replay of L rows from the log arena, gather of F rows
from MAT), then update (Adam on hits, evictions to MAT or back to the log arena, Adam on N/L rows being admitted or
compacted, log appends, transient Adam of M rows).  The dense model is not part of this path: the caller supplies
the per-occurrence gradients, which are reduced per unique row (dedup + fixed-order segment sum) as the reference's
embedding backward does (srm2/train.py:352, 429).

Planner classification uses torch ops on the device, as the reference's does, with one host synchronisation per
plan for the class counts (elara.py:242).  The hot-path kernels come from a backend object (HipBackend: this
library's HIP kernels), so the same step can be driven by another implementation of the kernels for comparison.
"""
import torch

from . import _lib  # noqa: F401  (the library must be present)
from .dedup import embedding_dense_backward, unique
from .elara_dir import dir_ext
from .gpu_ops import ScalarTable, init_rows, replay_rows
from .ops import gpu_adam
from .planner import (CNT_EXP, CNT_LOG_TOP, CNT_MAT_TOP, CNT_PRE, F_ADMIT, F_NEXT, classify_from_flags,
                      plan_classify)
from .rows import copy_rows

I8, I32, I64 = torch.int8, torch.int32, torch.int64
# classes (srm2/elara.py:31-32): hit, N admitted / append / compact, L admitted / append / compact, F admitted /
# not admitted, S
C_HIT, C_NADM, C_NAPP, C_NCMP, C_LADM, C_LAPP, C_LCMP, C_FADM, C_FNADM, C_S = range(10)


class HipBackend:
    """The hot-path kernels of this library (HIP, through the C-ABI)."""

    def __init__(self, D, seed, bound, hp, max_step, device):
        self.D, self.seed, self.bound, self.hp = D, seed, bound, hp
        self.table = ScalarTable(*hp, max_step, device)
        self.dx = dir_ext()

    def unique(self, ids):
        return unique(ids)

    def plan_classify(self, *args):
        return plan_classify(*args)

    def segsum(self, g_occ, inv, U):
        return embedding_dense_backward(g_occ, inv, U)

    def dir_a(self, st, pv, hs, L_row, L_cnt, ev_slot, s):
        return self.dx.elara_dir_a(st, pv, hs, L_row, L_cnt, ev_slot, s)

    def dir_b(self, st, pv, a_rows, a_k, c_rows, c_cnt, s):
        return self.dx.elara_dir_b(st, pv, a_rows, a_k, c_rows, c_cnt, s)

    def init_rows(self, rows):
        return init_rows(rows, self.D, self.seed, self.bound)

    def replay(self, rows, logs, offs, steps, cnt, K):
        return replay_rows(rows, logs, offs, steps, cnt, self.D, K, self.seed, self.bound, self.table)

    def adam(self, state, slots, grad, s):
        gpu_adam(state, slots, grad, *self.hp, s)

    def copy_rows(self, dst, dst_idx, src, src_idx=None):
        copy_rows(dst, dst_idx, src, src_idx)


class Plan:
    pass


class ElaraStep:
    """Planner + executor of ELARA over HBM-resident arenas.

    toff: first row of each table (int64 [T]); R total rows; D width; C pool slots; static_rows: pinned hot rows
    (the `static` base, srm2/train.py:262-270) or None; K = Kmax; kthr: materialisation threshold per table (or one
    int); evl: residency-aware representation (evicted rows may return to L); L: TTL lookahead; depth: number of
    batches u_nexts covers plus one (srm2/train.py:366); st_mode 'T' (transient full-state updates on the GPU) or
    'S' (materialised cold rows updated in the MAT arena); log_cap / mat_cap: arena capacities in rows.
    """

    def __init__(self, toff, R, D, C, static_rows=None, K=3, kthr=3, evl=True, L=8, depth=3, st_mode='T', seed=42,
                 bound=0.01, hp=(1e-3, 0.9, 0.999, 1e-8), max_step=1000, log_cap=None, mat_cap=None, device='cuda',
                 backend=None):
        d = torch.device(device)
        self.d, self.R, self.D, self.C, self.K, self.L, self.depth = d, R, D, C, K, L, depth
        self.MAT = K + 1
        self.st_mode = st_mode
        self.evl = bool(evl)
        self.hp = hp
        self.be = backend or HipBackend(D, seed, bound, hp, max_step, d)
        self.toff = torch.as_tensor(toff, dtype=I64).to(d)
        T = self.toff.numel()
        self.kthr = (torch.full((T,), int(kthr), dtype=I8) if isinstance(kthr, int)
                     else torch.as_tensor(kthr, dtype=I8)).to(d)
        self.log_cap = int(log_cap or 2 * R)
        self.mat_cap = int(mat_cap or R + 1)
        # ---- state directory (srm2/elara.py:117-125) ----
        self.code = torch.zeros(R, dtype=I8, device=d)
        self.loc = torch.full((R + 1,), -1, dtype=I32, device=d)
        self.ent = torch.full(((R + 1) * K,), -1, dtype=I32, device=d)
        self.lstep = torch.zeros(self.log_cap + 1, dtype=I32, device=d)
        self.lfree = torch.zeros(self.log_cap + 1, dtype=I32, device=d)
        self.n_lfree, self.log_top, self.mat_top, self.live = (torch.zeros(1, dtype=I64, device=d) for _ in range(4))
        # ---- residency (srm2/elara.py:128-146) ----
        self.slot_of = torch.full((R,), -1, dtype=I32, device=d)
        self.slot_row = torch.full((C,), -1, dtype=I64, device=d)
        self.pinned = torch.zeros(C, dtype=torch.bool, device=d)
        self.last_seen = torch.full((R,), -1, dtype=I32, device=d)
        n0 = 0
        self.static_rows = None
        if static_rows is not None and len(static_rows):
            sr = torch.as_tensor(static_rows, dtype=I64).to(d)
            n0 = sr.numel()
            assert n0 <= C
            self.slot_of[sr] = torch.arange(n0, dtype=I32, device=d)
            self.slot_row[:n0] = sr
            self.pinned[:n0] = True
            self.static_rows = sr
        self.n0, self.Cdyn = n0, C - n0
        self.free = torch.arange(C - 1, n0 - 1, -1, dtype=I64, device=d)
        self.n_free = C - n0
        self.dyn_slots = torch.empty(0, dtype=I64, device=d)
        self.adm_c0 = torch.full((C,), -1, dtype=I8, device=d)
        self.rj = torch.zeros(C, dtype=I8, device=d)
        self.rok = torch.zeros(C, dtype=I8, device=d)
        self.pstep = torch.zeros(self.Cdyn + 1, K, dtype=I32, device=d)
        self.mat_trash = R
        # ---- arenas (HBM) ----
        self.pool = torch.zeros(C, 3, D, device=d)
        self.glog = torch.zeros(self.Cdyn + 1, K, D, device=d)
        self.mat = torch.empty(self.mat_cap, 3, D, device=d)
        self.logs = torch.empty(self.log_cap + 1, D, device=d)
        self.stats = {k: 0 for k in ('adm', 'ev', 'hits', 'N', 'L', 'F', 'S', 'overflow', 'preempt',
                                     'compactions', 'appends', 'syncs')}
        if self.static_rows is not None:   # srm2/elara.py:434-440 load_static: pinned rows' state lives in the pool
            self.pool[:n0] = self.be.init_rows(self.static_rows)
            self.code[self.static_rows] = self.MAT

    # ---- helpers ----
    def state_list(self):
        return [self.code, self.loc, self.ent, self.lstep, self.lfree, self.n_lfree, self.log_top, self.mat_top,
                self.live, self.adm_c0, self.rj, self.pstep, self.kthr, self.toff, self.slot_of, self.slot_row,
                self.rok]

    def params(self):
        return [self.R, self.K, self.log_cap, self.n0, self.Cdyn, self.MAT, self.mat_trash, int(self.evl)]

    def check_capacity(self):
        """Raise if an allocation ran past the MAT or log arena (rows beyond capacity are not written)."""
        mt, lt = self._host(self.mat_top, self.log_top)
        if mt > self.mat_cap - 1 or lt > self.log_cap:
            raise RuntimeError(f'arena capacity exceeded (MAT {mt}/{self.mat_cap - 1}, logs {lt}/{self.log_cap})')

    def observe(self, step, u):
        """Record that rows u appear at logical step `step` (the TTL lookahead, srm2/elara.py:160-161)."""
        self.last_seen[u] = step

    def _host(self, *ts):
        self.stats['syncs'] += 1
        return torch.stack([t.reshape(()).to(I64) for t in ts]).tolist()

    def _host_list(self, t):
        self.stats['syncs'] += 1
        return t.tolist()

    # ---- plan (srm2/elara.py:209-414, cpp directory path) ----
    def plan(self, s, u, u_nexts):
        d, K, C = self.d, self.K, self.C
        n = u.numel()
        # classes, class order, expired / preemptible / protected dynamic slots, counts (srm2/elara.py:214-267)
        pc = self.be.plan_classify(u, u_nexts, self.slot_of, self.last_seen, self.code, self.kthr, self.toff,
                                   self.dyn_slots, self.slot_row, self.mat_top, self.log_top, s, K,
                                   self.st_mode == 'T')
        vals = self._host_list(pc.counts)
        counts = vals[:10]
        n_exp, n_pre, mat_top, log_top = vals[CNT_EXP], vals[CNT_PRE], vals[CNT_MAT_TOP], vals[CNT_LOG_TOP]
        if mat_top > self.mat_cap - 1 or log_top > self.log_cap:
            raise RuntimeError(f'arena capacity exceeded (MAT {mat_top}/{self.mat_cap}, logs {log_top}/{self.log_cap})')
        sl, c, order = pc.sl, pc.c, pc.order
        n_adm = counts[C_NADM] + counts[C_LADM] + counts[C_FADM]
        nd = self.dyn_slots.numel()
        need = n_adm - (self.n_free + n_exp)
        take = min(need, n_pre) if need > 0 and nd > n_exp else 0
        if take:   # preempt residents not needed within the pipeline window
            ev_slot, keep_dyn = pc.dyn_out[:n_exp + take], pc.dyn_out[n_exp + take:nd]
            n_exp += take
            need -= take
            self.stats['preempt'] += take
        else:
            ev_slot, keep_dyn = pc.dyn_out[:n_exp], pc.dyn_out[nd + n_exp:]
        if need > 0:   # overflow: un-admit (non-carry first) and recount
            admit = (pc.flags & F_ADMIT) != 0
            in_next = (pc.flags & F_NEXT) != 0
            pri = (~admit).to(I32) * 4 + admit.to(I32) * (2 - 2 * in_next.to(I32))
            oo = torch.argsort(pri, stable=True)
            drop = oo[n_adm - need:n_adm]
            admit[drop] = False
            self.stats['overflow'] += need
            n_adm -= need
            cls = classify_from_flags(pc.flags, admit, self.st_mode == 'T')
            counts = self._host(*torch.bincount(cls.long(), minlength=10))
            order = torch.argsort(cls, stable=True)
        b_ = [0]
        for x in counts:
            b_.append(b_[-1] + x)
        rng = lambda lo, hi: order[b_[lo]:b_[hi + 1]]  # noqa: E731
        p = Plan()
        p.s, p.u, p.n = s, u, n
        hp_ = rng(C_HIT, C_HIT)
        p.hit_pos, p.hit_slot = hp_, sl[hp_].long()
        Npos, Lpos, Fpos, Spos = rng(C_NADM, C_NCMP), rng(C_LADM, C_LCMP), rng(C_FADM, C_FNADM), rng(C_S, C_S)
        p.N_pos, p.N_row = Npos, u[Npos]
        p.L_pos, p.L_row, p.L_cnt = Lpos, u[Lpos], c[Lpos].to(I32)
        p.F_pos, p.F_row, p.S_pos, p.S_row = Fpos, u[Fpos], Spos, u[Spos]
        nNa, nNp, nNc, nLa, nLp, nLc, nFa, nFn = counts[1:9]
        p.counts = counts
        st, pv = self.state_list(), self.params()
        (p.L_steps, p.L_ids, p.hrec_dyn, p.hrec_j, p.ev_row, p.ev_rep, p.evl_ids, p.evf_slots,
         p.ev_dyn) = self.be.dir_a(st, pv, p.hit_slot, p.L_row, p.L_cnt, ev_slot, s)
        p.ev_slot = ev_slot
        nev = ev_slot.numel()
        # admissions (srm2/elara.py:345-367)
        pool_free = torch.cat([self.free, ev_slot])
        nf = self.n_free + nev
        adm_slots = pool_free[nf - n_adm:]
        self.free = pool_free[:nf - n_adm]
        self.n_free = nf - n_adm
        adm_rows = torch.cat([p.N_row[:nNa], p.L_row[:nLa], p.F_row[:nFa]])
        ar = lambda a_, b2: torch.arange(a_, b2, device=d)  # noqa: E731
        ix = {'N_adm': ar(0, nNa), 'N_app': ar(nNa, nNa + nNp), 'N_cmp': ar(nNa + nNp, nNa + nNp + nNc),
              'L_adm': ar(0, nLa), 'L_app': ar(nLa, nLa + nLp), 'L_cmp': ar(nLa + nLp, nLa + nLp + nLc),
              'F_adm': ar(0, nFa), 'F_nadm': ar(nFa, nFa + nFn)}
        ix['N_upd'] = torch.cat([ix['N_adm'], ix['N_cmp']])
        ix['L_upd'] = torch.cat([ix['L_adm'], ix['L_cmp']])
        ix['N_adm_slot'] = adm_slots[:nNa]
        ix['L_adm_slot'] = adm_slots[nNa:nNa + nLa]
        ix['F_adm_slot'] = adm_slots[nNa + nLa:]
        p.ix = ix
        p.L_off = torch.cumsum(p.L_cnt.long(), 0) - p.L_cnt.long()
        lazy_n = nNa + nLa
        p.adm_rec_dyn = adm_slots[:lazy_n] - self.n0
        if n_adm:
            self.slot_of[adm_rows] = adm_slots.to(I32)
            self.slot_row[adm_slots] = adm_rows
            c_adm = self.code[adm_rows].to(I64)
            isIL = torch.cat([torch.ones(lazy_n, dtype=torch.bool, device=d),
                              torch.zeros(nFa, dtype=torch.bool, device=d)])
            lazy_adm = isIL & self.evl
            self.adm_c0[adm_slots] = torch.where(isIL, c_adm, torch.full_like(c_adm, -1)).to(I8)
            self.rj[adm_slots] = lazy_adm.to(I8)
            self.rok[adm_slots] = lazy_adm.to(I8)
            if lazy_n and self.evl:
                self.pstep[p.adm_rec_dyn, 0] = s
        self.dyn_slots = torch.cat([keep_dyn, adm_slots])
        # non-resident lazy rows: append (stay L) or compact (to M)
        p.a_rows = torch.cat([p.N_row[nNa:nNa + nNp], p.L_row[nLa:nLa + nLp]])
        a_k = torch.cat([torch.zeros(nNp, dtype=I64, device=d), p.L_cnt[nLa:nLa + nLp].long()])
        p.c_rows = torch.cat([p.N_row[nNa + nNp:], p.L_row[nLa + nLp:]])
        c_cnt = torch.cat([torch.zeros(nNc, dtype=I64, device=d), p.L_cnt[nLa + nLp:].long()])
        p.a_ids, p.c_slots = self.be.dir_b(st, pv, p.a_rows, a_k, p.c_rows, c_cnt, s)
        p.F_slot = self.loc[p.F_row].to(I64)
        p.S_slot = self.loc[p.S_row].to(I64)
        st_ = self.stats
        st_['adm'] += n_adm
        st_['ev'] += nev
        st_['hits'] += counts[C_HIT]
        st_['N'] += Npos.numel()
        st_['L'] += Lpos.numel()
        st_['F'] += Fpos.numel()
        st_['S'] += Spos.numel()
        st_['compactions'] += nNc + nLc
        st_['appends'] += nNp + nLp
        return p

    # ---- assemble (srm2/elara.py:471-489): states of the non-resident rows this step updates ----
    def assemble(self, p):
        be, D, K = self.be, self.D, self.K
        fullN = be.init_rows(p.N_row) if p.N_row.numel() else None
        fullL = None
        nL = p.L_row.numel()
        if nL:
            # the logged gradients of each L row, packed row by row (entry k of row i at L_off[i] + k)
            kk = torch.arange(K, device=self.d)
            valid = kk[None, :] < p.L_cnt.long()[:, None]
            dst = torch.where(valid, p.L_off[:, None] + kk[None, :], torch.full_like(p.L_off[:, None], -1))
            lg = torch.empty(nL * K, D, device=self.d)
            be.copy_rows(lg, dst.reshape(-1), self.logs, p.L_ids.reshape(-1).to(I64))
            fullL = be.replay(p.L_row, lg, p.L_off, p.L_steps, p.L_cnt, K)
        ff = None
        if p.F_row.numel():
            ff = torch.empty(p.F_row.numel(), 3, D, device=self.d)
            be.copy_rows(ff, None, self.mat, p.F_slot)
        return fullN, fullL, ff

    # ---- update (srm2/elara.py:491-542 and the host worker's writes 544-580, all in HBM) ----
    def update(self, p, G, bufs):
        be, s, D, K, ix = self.be, p.s, self.D, self.K, p.ix
        fullN, fullL, ff = bufs
        sel = lambda t, i: t.index_select(0, i)  # noqa: E731
        glog2 = self.glog.view(-1, D)
        if p.hit_pos.numel():
            gh = sel(G, p.hit_pos)
            if self.evl:
                be.copy_rows(glog2, p.hrec_dyn * K + p.hrec_j, gh)
            be.adam(self.pool, p.hit_slot, gh, s)
        if p.ev_slot.numel():
            # evicted slots are read before admissions reuse them: full states of rows going to M into their MAT
            # slots (rows going back to L carry the trash slot), history entries of rows going back to L into
            # their new log ids (-1 for none)
            be.copy_rows(self.mat, p.evf_slots, self.pool, p.ev_slot)
            src = (p.ev_dyn.clamp(min=0, max=self.Cdyn)[:, None] * K + torch.arange(K, device=self.d)[None, :])
            be.copy_rows(self.logs, p.evl_ids.reshape(-1), glog2, src.reshape(-1))
        adm_g = []
        nNc = ix['N_cmp'].numel()
        nNp = ix['N_app'].numel()
        for X, full, pos in (('N', fullN, p.N_pos), ('L', fullL, p.L_pos)):
            if full is None:
                continue
            up = ix[X + '_upd']
            if up.numel():
                be.adam(full, up, sel(G, sel(pos, up)), s)
            if ix[X + '_adm'].numel():
                be.copy_rows(self.pool, ix[X + '_adm_slot'], full, ix[X + '_adm'])
                adm_g.append(sel(G, sel(pos, ix[X + '_adm'])))
            if ix[X + '_cmp'].numel():
                cs = p.c_slots[:nNc] if X == 'N' else p.c_slots[nNc:]
                be.copy_rows(self.mat, cs, full, ix[X + '_cmp'])
            if ix[X + '_app'].numel():
                ai = p.a_ids[:nNp] if X == 'N' else p.a_ids[nNp:]
                be.copy_rows(self.logs, ai, G, sel(pos, ix[X + '_app']))
        if adm_g and self.evl:   # admission gradient = resident history entry 0
            ag = torch.cat(adm_g) if len(adm_g) > 1 else adm_g[0]
            be.copy_rows(glog2, p.adm_rec_dyn * K, ag)
        if ff is not None:
            be.adam(ff, torch.arange(p.F_row.numel(), device=self.d), sel(G, p.F_pos), s)
            if ix['F_adm'].numel():
                be.copy_rows(self.pool, ix['F_adm_slot'], ff, ix['F_adm'])
            if ix['F_nadm'].numel():
                be.copy_rows(self.mat, p.F_slot[ix['F_adm'].numel():], ff, ix['F_nadm'])
        if p.S_row.numel():
            be.adam(self.mat, p.S_slot, sel(G, p.S_pos), s)

    # ---- one step from a batch's occurrence ids and gradients ----
    def step(self, s, ids, g_occ, u, inv, u_nexts):
        """Logical step s (1-based): ids int64 [O] (occurrences), g_occ [O, D] their gradients, (u, inv) the
        batch's unique rows and inverse, u_nexts the unique rows of the next depth-1 batches."""
        p = self.plan(s, u, u_nexts)
        bufs = self.assemble(p)
        G = self.be.segsum(g_occ, inv, u.numel())
        self.update(p, G, bufs)
        return p

    # ---- eval-style materialisation (srm2/elara.py:582-604) ----
    def eval_weights(self, rows, full=False):
        """Current (w) -- or (w, m, v) with full=True -- of `rows`: resident rows from the pool, materialised rows
        from the MAT arena, logged and implicit rows by replay from the log arena."""
        K, D = self.K, self.D
        out = torch.empty(rows.numel(), 3, D, device=self.d)
        sl = self.slot_of[rows]
        res = sl >= 0
        ri = res.nonzero().flatten()
        if ri.numel():
            self.be.copy_rows(out, ri, self.pool, sl[ri].long())
        nr = (~res).nonzero().flatten()
        r = rows[nr]
        c = self.code[r]
        mat = c == self.MAT
        mi = mat.nonzero().flatten()
        if mi.numel():
            self.be.copy_rows(out, nr[mi], self.mat, self.loc[r[mi]].long())
        li = (~mat).nonzero().flatten()
        if li.numel():
            rl = r[li]
            cnt = c[li].to(I32)
            kk = torch.arange(K, device=self.d)
            e = self.ent[rl[:, None] * K + kk[None, :]]
            ids = torch.where(kk[None, :] < cnt[:, None], e, torch.full_like(e, -1))
            steps = torch.where(e >= 0, self.lstep[e.clamp(min=0).long()], torch.zeros_like(e))
            off = torch.cumsum(cnt.long(), 0) - cnt.long()
            valid = kk[None, :] < cnt.long()[:, None]
            dst = torch.where(valid, off[:, None] + kk[None, :], torch.full_like(off[:, None], -1))
            lg = torch.empty(rl.numel() * K, D, device=self.d)
            self.be.copy_rows(lg, dst.reshape(-1), self.logs, ids.reshape(-1).to(I64))
            fl = self.be.replay(rl, lg, off, steps, cnt, K)
            self.be.copy_rows(out, nr[li], fl)
        return out if full else out[:, 0]


def run(step, batches, grads, steps=None, on_step=None):
    """Drive `step` over a sequence of batches as srm2/train.py:344-444 does: the batch of logical step j+1 is
    deduplicated and observed L+1 steps ahead (TTL lookahead), plan(s) sees the next depth-1 batches, then the step
    assembles and updates.  batches[j]: int64 occurrence ids; grads(j) or grads[j]: [O_j, D] occurrence gradients.
    on_step(s, plan) is called after each step."""
    S = len(batches) if steps is None else steps
    U, INV = {}, {}
    dev = step.d

    def load(j):
        u, inv = step.be.unique(batches[j].to(dev))
        U[j], INV[j] = u, inv
        step.observe(j + 1, u)

    for j in range(min(S, step.L + 1)):
        load(j)
    for s in range(S):
        if s + step.L + 1 < S:
            load(s + step.L + 1)
        u_nexts = [U[s + k] for k in range(1, step.depth) if s + k < S]
        g = grads(s) if callable(grads) else grads[s]
        p = step.step(s + 1, batches[s].to(dev), g.to(dev), U.pop(s), INV.pop(s), u_nexts)
        if on_step is not None:
            on_step(s + 1, p)
    step.check_capacity()
