"""The step's planner against the reference's own planner: tests/golden/planner_vectors.npz, written by
tests/golden/make_planner_vectors.py, which runs srm2/elara.py's ELARAPlanner (dir_impl='ref') on CPU tensors over
the configurations there (TTL and carry residency, evl off / on / gated by memory pressure, preemption, overflow
with carry barriers, per-table thresholds, a host budget that is exceeded) and drives the reference's ArenaStore
accounting; the triton_* configurations repeat five of them with the reference's Triton directory
(dir_impl='triton', srm2/elara_kernels.py, in Triton's interpreter), whose log ids follow its own allocation order,
and ElaraStep plans them with dir_impl='triton'.  ElaraStep plans the same batches -- on the oracle backend (CPU) and on this library's kernels (GPU) --
and must produce, step by step, the same classes, evictions, admissions, replay inputs, resident-history records,
log ids and MAT slots, the same barriers and representation switch, the same HostBudgetExceeded step, and at the
end the same directory and residency state."""
from pathlib import Path

import numpy as np
import pytest
import torch

from elara_amd import synth
from oracle.backend import OracleBackend

FIX = Path(__file__).resolve().parent / 'golden' / 'planner_vectors.npz'
HP = synth.ADAM
FIELDS = ('counts', 'ev_slot', 'ev_rep', 'adm_slots', 'L_row', 'L_cnt', 'L_steps', 'L_ids', 'hit_slot', 'hrec_dyn',
          'hrec_j', 'a_ids', 'c_slots', 'FN_slot', 'S_slot', 'flags', 'tops')


def _fix():
    return np.load(FIX)


def configs():
    return [str(c) for c in _fix()['configs']]


def per_step(z, name, key):
    v, off = z[f'{name}/{key}'], z[f'{name}/{key}_off']
    return [v[off[i]:off[i + 1]] for i in range(off.size - 1)]


def run_config(name, device, backend):
    from elara_amd.step import ElaraStep, HostBudgetExceeded, run
    z = _fix()
    meta = z[f'{name}/meta'].tolist()
    (R, C, K, L, depth, st_S, carry, evl, budget, chunk, D, done, raised_at, log_cap, _, _) = meta[:16]
    triton = len(meta) > 16 and meta[16] == 1
    U = per_step(z, name, 'U')
    steps = len(U)
    st = ElaraStep(z[f'{name}/toff'], R, D, C, static_rows=z[f'{name}/static'], K=K,
                   kthr=torch.from_numpy(z[f'{name}/kthr']), evl=evl, L=L, depth=depth, st_mode='S' if st_S else 'T',
                   dyn='carry' if carry else 'ttl', seed=42, bound=synth.bound_for(D), hp=HP, max_step=steps + 2,
                   log_cap=log_cap, mat_cap=R + 1, device=device, backend=backend, host_budget=budget,
                   budget_chunk=chunk or (64 << 20), dir_impl='triton' if triton else 'cpp')
    got = {k: [] for k in FIELDS}

    def on_step(s, p):
        t = lambda x: x.detach().cpu().numpy().astype(np.int64).reshape(-1)  # noqa: E731
        got['counts'].append(np.array(p.counts, np.int64))
        got['ev_slot'].append(t(p.ev_slot))
        got['ev_rep'].append(t(p.ev_rep))
        got['adm_slots'].append(t(p.adm_slots))
        got['L_row'].append(t(p.L_row))
        got['L_cnt'].append(t(p.L_cnt))
        got['L_steps'].append(t(p.L_steps))
        got['L_ids'].append(t(p.L_ids))
        got['hit_slot'].append(t(p.hit_slot))
        got['hrec_dyn'].append(t(p.hrec_dyn))
        got['hrec_j'].append(t(p.hrec_j))
        got['a_ids'].append(t(p.a_ids))
        got['c_slots'].append(t(p.c_slots))
        got['FN_slot'].append(t(p.FN_slot))
        got['S_slot'].append(t(p.S_slot))
        got['flags'].append(np.array([int(p.barrier), int(p.evl)], np.int64))
        got['tops'].append(np.array([int(st.mat_top), int(st.log_top), int(st.live)], np.int64))

    batches = [torch.from_numpy(u) for u in U]
    grads = [torch.zeros(u.size, D) for u in U]
    if raised_at:
        with pytest.raises(HostBudgetExceeded):
            run(st, batches, grads, on_step=on_step)
    else:
        run(st, batches, grads, on_step=on_step)
    return z, st, got, done


def check(name, device, backend):
    z, st, got, done = run_config(name, device, backend)
    assert len(got['counts']) == done - int(z[f'{name}/meta'][12] > 0), name   # the raising step records nothing
    n = len(got['counts'])
    for k in FIELDS:
        want = per_step(z, name, k)
        for s in range(n):
            assert np.array_equal(got[k][s], want[s]), (name, k, s + 1, got[k][s][:20], want[s][:20])
    R, K = st.R, st.K
    final = {'code': st.code, 'loc': st.loc, 'ent': st.ent, 'lstep': st.lstep[:-1], 'lfree': st.lfree[:-1],
             'n_lfree': st.n_lfree, 'log_top': st.log_top, 'mat_top': st.mat_top, 'live': st.live,
             'adm_c0': st.adm_c0, 'rj': st.rj, 'pstep': st.pstep, 'slot_of': st.slot_of, 'slot_row': st.slot_row,
             'rok': st.rok, 'last_seen': st.last_seen, 'dyn_slots': st.dyn_slots, 'free': st.free}
    trash = {'loc': R, 'ent': R * K, 'pstep': st.Cdyn}   # trash rows the two directory formulations fill differently
    for k, v in final.items():
        a = v.detach().cpu().numpy()
        b = z[f'{name}/final_{k}']
        if k in trash:
            a, b = a[:trash[k]], b[:trash[k]]
        assert a.shape == b.shape and np.array_equal(a.astype(np.int64), b.astype(np.int64)), (name, k)
    if z[f'{name}/meta'][8]:   # budget accounting as the reference's ArenaStore faulted it
        assert [st.faulted['mat'], st.faulted['log']] == z[f'{name}/store_faulted'].tolist(), name


@pytest.mark.parametrize('name', configs())
def test_planner_matches_reference_on_cpu(name):
    """ElaraStep on the oracle backend (CPU tensors) plans exactly as the reference's planner."""
    check(name, 'cpu', OracleBackend(32, 42, synth.bound_for(32), HP, 64))


@pytest.mark.gpu
@pytest.mark.parametrize('name', configs())
def test_planner_matches_reference_on_gpu(dev, name):
    """ElaraStep on this library's kernels plans exactly as the reference's planner."""
    print(f'[gpu-test] planner golden {name}', flush=True)
    check(name, dev, None)
