"""Golden vectors of the reference's planner: srm2/elara.py ELARAPlanner.plan run on CPU tensors.

Run only in the build container (it imports srm2 from /root/reference, read-only; the GPU box has no reference):
    python tests/golden/make_planner_vectors.py
It writes tests/golden/planner_vectors.npz.  For each configuration below the reference's ELARAPlanner with
dir_impl='ref' (its torch restatement of the directory, state-identical to the default 'cpp' one) plans a sequence
of batches, driven as srm2/train.py:359-370 drives it: the batches of logical steps 1..L+1 are observed first, then
before plan(s) the batch L+1 steps ahead, and plan(s) sees the next depth-1 batches.  Recorded per step: the class
counts, the evicted slots and their representation, the admitted slots, the L rows with their counts, steps and log
ids, the hit slots and their resident-history records, the append log ids, the compaction MAT slots, the transient
and S rows' MAT slots, the overflow barrier and whether the residency-aware representation is on; after the run the
whole directory and residency state.

Capacity-tier accounting (configurations with a host budget): the reference's own ArenaStore (srm2/elara.py:38-103)
is driven as the executor's update worker drives it (srm2/elara.py:555-557): after each plan its tops are set and its
arenas are faulted up to them; HostBudgetExceeded ends the run and its step is recorded.  ArenaStore pre-faults pages
through the extension's cpu_prefault, given here by the reference's srm2_cpu.cpp as oracle/Makefile compiles it
(oracle/_ref; the reference's JIT loader is not run).  Its fault granularity CHUNK (64 MiB, srm2/store.py:23) is set
to 64 KiB here so that a small configuration crosses several chunks; the fixture records the value.  The memory-
pressure gate of evict_logs=2 is the executor's (srm2/elara.py:423-425), reading the store's tops of the previous
step.  The pinned static rows get code MAT before the first plan, as the executor's load_static does at set-up
(srm2/elara.py:433-439).

The configurations named triton_* rerun a configuration above with dir_impl='triton', the reference's Triton
directory (srm2/elara_kernels.py), whose log ids follow its own allocation order (every allocation of a step before
any release).  Its kernels run in Triton's interpreter (TRITON_INTERPRET=1) on the same CPU tensors.

Batches come from elara_amd.synth (numpy, seeded): configuration inputs are stored in the fixture as well, so the
tests do not depend on the generator staying the same.
"""
import os
import sys
from pathlib import Path

os.environ.setdefault('TRITON_INTERPRET', '1')   # before srm2.elara_kernels imports triton

import numpy as np  # noqa: E402
import torch  # noqa: E402

ROOT = Path(__file__).resolve().parents[2]
REF = Path(os.environ.get('ELARA_REFERENCE', '/root/reference'))
OUT = Path(__file__).resolve().parent / 'planner_vectors.npz'
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(REF))
from elara_amd import synth  # noqa: E402

CHUNK_TEST = 64 << 10

# name: (T, lo, hi, B, steps, C, n_static, K, kthr, L, depth, st, dyn, evict_logs, budget_bytes, seed)
CONFIGS = {
    'ttl_evl': (5, 100, 3000, 300, 40, 700, 400, 3, 3, 8, 3, 'T', 'ttl', 1, 0, 1),
    'ttl_noevl': (5, 100, 3000, 300, 40, 700, 400, 3, 3, 8, 3, 'T', 'ttl', 0, 0, 2),
    'ttl_S_overflow': (6, 200, 20000, 600, 40, 900, 500, 3, 3, 8, 3, 'S', 'ttl', 1, 0, 3),
    'ttl_K4_kthr': (5, 100, 3000, 300, 40, 700, 400, 4, (0, 1, 2, 3, 4), 6, 3, 'T', 'ttl', 1, 0, 4),
    'carry_evl': (5, 100, 3000, 300, 40, 700, 400, 3, 3, 8, 3, 'T', 'carry', 1, 0, 5),
    'carry_overflow': (6, 200, 20000, 600, 40, 900, 500, 3, 3, 8, 3, 'T', 'carry', 1, 0, 6),
    'evl_gate': (5, 100, 3000, 300, 40, 700, 400, 3, 3, 8, 3, 'T', 'ttl', 2, 1_250_000, 7),
    'budget_raise': (5, 100, 3000, 300, 40, 700, 400, 3, 3, 8, 3, 'T', 'ttl', 1, 800_000, 8),
}
# the Triton directory's runs: name -> the configuration above it repeats
TRITON = {f'triton_{b}': b for b in ('ttl_evl', 'ttl_S_overflow', 'ttl_K4_kthr', 'carry_overflow', 'evl_gate')}
D = 32   # width used by the store accounting and the gate (the planner itself is width-free)


def batches_of(T, lo, hi, B, steps, seed):
    tabs = synth.C5Tables(T=T, lo=lo, hi=hi, alpha=1.1, seed=seed)
    rng = np.random.default_rng(seed + 100)
    return tabs, rng, [np.unique(tabs.batch(rng, B)) for _ in range(steps)]


def run(name, cfg, dir_impl='ref'):
    import srm2.elara as E
    from oracle import ref as REFBUILD
    (T, lo, hi, B, steps, C, n_static, K, kthr, L, depth, st, dyn, evl, budget, seed) = cfg
    tabs, rng, U = batches_of(T, lo, hi, B, steps, seed)
    static = tabs.static_rows(rng, B, n_static, n_batches=10)
    kt = torch.tensor(kthr if isinstance(kthr, tuple) else [kthr] * T, dtype=torch.int8)
    pl = E.ELARAPlanner(tabs.R, C, K, 'static', dyn, st, torch.from_numpy(static), L, torch.device('cpu'),
                        torch.from_numpy(tabs.toff), kt, evict_logs=evl, fused_dir=dir_impl == 'triton',
                        dir_impl=dir_impl)
    pl.code[pl.static_rows] = pl.MAT   # the executor's load_static (srm2/elara.py:433-439), run before training
    store = None
    if budget:
        E.CHUNK = CHUNK_TEST
        store = E.ArenaStore(tabs.R, D, REFBUILD.cpu(), 2, budget, log_cap=pl.log_cap)
        if evl == 2:   # the executor's gate (srm2/elara.py:423-425)
            frac = pl.evl_gate_frac
            pl.gate = lambda: store.budget > 0 and (store.top['mat'] * 3 + store.live_logs) * D * 4 >= frac * store.budget
    Ut = [torch.from_numpy(u) for u in U]
    rec = {k: [] for k in ('counts', 'ev_slot', 'ev_rep', 'adm_slots', 'L_row', 'L_cnt', 'L_steps', 'L_ids',
                           'hit_slot', 'hrec_dyn', 'hrec_j', 'a_ids', 'c_slots', 'FN_slot', 'S_slot', 'flags',
                           'tops')}
    raised_at = 0
    for j in range(min(steps, L + 1)):
        pl.observe(j + 1, Ut[j])
    done = 0
    for s in range(steps):
        if s + L + 1 < steps:
            pl.observe(s + L + 2, Ut[s + L + 1])
        p = pl.plan(s + 1, Ut[s], [Ut[s + k] for k in range(1, depth) if s + k < steps])
        ix = p.ix
        nNa, nNp, nNc = ix['N_adm'].numel(), ix['N_app'].numel(), ix['N_cmp'].numel()
        nLa, nLp, nLc = ix['L_adm'].numel(), ix['L_app'].numel(), ix['L_cmp'].numel()
        nFa, nFn = ix['F_adm'].numel(), ix['F_nadm'].numel()
        counts = [p.hit_pos.numel(), nNa, nNp, nNc, nLa, nLp, nLc, nFa, nFn, p.S_pos.numel()]
        c = p.cpu
        rec['counts'].append(np.array(counts, np.int64))
        rec['ev_slot'].append(p.ev_slot.numpy().astype(np.int64))
        rec['ev_rep'].append(p.ev_rep.numpy().astype(np.int64))
        rec['adm_slots'].append(torch.cat([ix['N_adm_slot'], ix['L_adm_slot'], ix['F_adm_slot']]).numpy()
                                .astype(np.int64))
        rec['L_row'].append(p.L_row.numpy().astype(np.int64))
        rec['L_cnt'].append(p.L_cnt.numpy().astype(np.int64))
        rec['L_steps'].append(p.L_steps.numpy().astype(np.int64).reshape(-1))
        rec['L_ids'].append(c['L_ids'].numpy().astype(np.int64))
        rec['hit_slot'].append(p.hit_slot.numpy().astype(np.int64))
        rec['hrec_dyn'].append(p.hrec_dyn.numpy().astype(np.int64))
        rec['hrec_j'].append(p.hrec_j.numpy().astype(np.int64))
        rec['a_ids'].append(c['A_ids'].numpy().astype(np.int64))
        rec['c_slots'].append(c['W_slot'][:nNc + nLc].numpy().astype(np.int64))
        rec['FN_slot'].append(c['F_slot'][nFa:].numpy().astype(np.int64))
        rec['S_slot'].append(c['S_slot'].numpy().astype(np.int64))
        rec['flags'].append(np.array([int(p.barrier), int(pl.evict_logs)], np.int64))
        rec['tops'].append(c['tops'][:3].numpy().astype(np.int64))
        done = s + 1
        if store is not None:   # the update worker's accounting of step s (srm2/elara.py:555-557)
            mt, lt, live, _ = c['tops'].tolist()
            store.set_tops(mt, lt, live)
            try:
                store.fault('mat', mt)
                store.fault('log', lt)
            except E.HostBudgetExceeded:
                raised_at = s + 1
                break
    out = {}
    for k, v in rec.items():
        out[f'{name}/{k}'] = np.concatenate(v) if v else np.zeros(0, np.int64)
        out[f'{name}/{k}_off'] = np.cumsum([0] + [x.size for x in v]).astype(np.int64)
    final = {'code': pl.code, 'loc': pl.loc, 'ent': pl.ent, 'lstep': pl.lstep[:-1], 'lfree': pl.lfree[:-1],
             'n_lfree': pl.n_lfree, 'log_top': pl.log_top, 'mat_top': pl.mat_top, 'live': pl.live,
             'adm_c0': pl.adm_c0, 'rj': pl.rj, 'pstep': pl.pstep, 'slot_of': pl.slot_of, 'slot_row': pl.slot_row,
             'rok': pl.rok, 'last_seen': pl.last_seen, 'dyn_slots': pl.dyn_slots, 'free': pl.free[:pl.n_free]}
    for k, v in final.items():
        out[f'{name}/final_{k}'] = v.numpy().copy()
    out[f'{name}/U'] = np.concatenate(U)
    out[f'{name}/U_off'] = np.cumsum([0] + [u.size for u in U]).astype(np.int64)
    out[f'{name}/static'] = static
    out[f'{name}/toff'] = tabs.toff
    out[f'{name}/kthr'] = kt.numpy()
    out[f'{name}/meta'] = np.array([tabs.R, C, K, L, depth, int(st == 'S'), int(dyn == 'carry'), evl, budget,
                                    CHUNK_TEST if budget else 0, D, done, raised_at, pl.log_cap,
                                    int(pl.stats.get('preempt', 0)), int(pl.stats['overflow']),
                                    int(dir_impl == 'triton')], np.int64)
    store_res = [0, 0] if store is None else [store.faulted['mat'], store.faulted['log']]
    out[f'{name}/store_faulted'] = np.array(store_res, np.int64)
    print(f'{name}: {done} steps, raised_at {raised_at}, stats {pl.stats}, evl_on {pl.evict_logs}, '
          f'faulted {store_res}', flush=True)
    return out


def main():
    vec = {'configs': np.array(list(CONFIGS) + list(TRITON))}
    for name, cfg in CONFIGS.items():
        vec.update(run(name, cfg))
    for name, base in TRITON.items():
        vec.update(run(name, CONFIGS[base], dir_impl='triton'))
    np.savez_compressed(OUT, **vec)
    print(f'wrote {OUT} ({OUT.stat().st_size} bytes)')


if __name__ == '__main__':
    main()
