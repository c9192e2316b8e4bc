"""The whole ELARA step with HBM-resident arenas (config C5; elara_amd.step, the counterpart of srm2/elara.py's
planner and executor): the HIP kernels against the CPU oracle driving the identical step.

Both runs see the same batches and occurrence gradients; the planner's glue is shared (torch ops on each device),
the hot-path kernels and the planner classification differ (HIP vs oracle/elara_oracle.c and the torch
restatement in oracle/backend.py).  After the run the directory, the pool, the resident
histories, the MAT and log arenas and the eval-style weights of every touched row (srm2/elara.py:582-604) must be
bitwise equal.  Trash rows (whose contents the reference leaves unspecified) are excluded.
"""
import numpy as np
import pytest
import torch

from elara_amd import synth
from oracle.backend import OracleBackend

HP = synth.ADAM


def make(cfg, device, backend=None):
    from elara_amd.step import ElaraStep
    return ElaraStep(cfg['toff'], cfg['R'], cfg['D'], cfg['C'], static_rows=cfg['static'], K=cfg.get('K', 3),
                     kthr=cfg.get('kthr', 3), evl=cfg.get('evl', True), L=cfg.get('L', 8), depth=3,
                     st_mode=cfg.get('st', 'T'), seed=42, bound=cfg['bound'], hp=HP, max_step=cfg['steps'] + 2,
                     log_cap=cfg['log_cap'], mat_cap=cfg['mat_cap'], device=device, backend=backend,
                     host_arenas=cfg.get('host', False), dyn=cfg.get('dyn', 'ttl'), host_budget=cfg.get('budget', 0),
                     budget_chunk=cfg.get('chunk', 64 << 20), dir_impl=cfg.get('dir_impl', 'cpp'),
                     sync_free=cfg.get('sync_free', True), link_stream=cfg.get('link'),
                     field_layout=cfg.get('field', False))


def same_stats(a, b):
    """The two runs' planner counts, except the number of host synchronisations (the device-driven step has none
    per step; the oracle-driven step reads its counts every step)."""
    strip = lambda st: {k: v for k, v in st.items() if k != 'syncs'}  # noqa: E731
    return strip(a.stats) == strip(b.stats)


def config(T, lo, hi, B, steps, C, n_static, D=128, seed=0, **kw):
    tabs = synth.C5Tables(T=T, lo=lo, hi=hi, alpha=1.1, seed=seed)
    rng = np.random.default_rng(seed + 7)
    static = tabs.static_rows(rng, B, n_static, n_batches=10) if n_static else None
    batches = [torch.from_numpy(tabs.batch(rng, B)) for _ in range(steps)]
    O = B * T
    cfg = dict(toff=tabs.toff, R=tabs.R, D=D, C=C, static=static, steps=steps, bound=synth.bound_for(D),
               log_cap=steps * O + 16, mat_cap=min(tabs.R + 1, steps * O + 16), batches=batches, seed=seed)
    cfg.update(kw)
    return cfg


def grads_fn(cfg, device):
    D = cfg['D']

    def g(j):
        gen = torch.Generator().manual_seed(1000 + j)
        return (torch.randn(cfg['batches'][j].numel(), D, generator=gen, dtype=torch.float64) * 1e-3).float()
    return g


def compare(a, b, cfg):
    """Assert the two steps' states are equal; returns the number of touched rows compared."""
    def eq(x, y, what):
        x, y = x.detach().cpu(), y.detach().cpu()
        if x.dtype == torch.float32:
            x, y = x.view(torch.int32), y.view(torch.int32)
        assert x.shape == y.shape and torch.equal(x, y), what
    for name in ('code', 'loc', 'ent', 'n_lfree', 'log_top', 'mat_top', 'live', 'adm_c0', 'rj', 'pstep', 'slot_of',
                 'slot_row', 'rok'):
        eq(getattr(a, name), getattr(b, name), name)
    eq(a.lstep[:-1], b.lstep[:-1], 'lstep')
    eq(a.lfree[:-1], b.lfree[:-1], 'lfree')
    eq(a.pool, b.pool, 'pool')
    eq(a.glog[:-1], b.glog[:-1], 'glog')
    mt, lt = int(a.mat_top), int(a.log_top)
    eq(a.mat[:min(mt, a.R)], b.mat[:min(mt, b.R)], 'MAT arena')
    eq(a.logs[:lt], b.logs[:lt], 'log arena')
    rows = torch.unique(torch.cat(cfg['batches']))
    eq(a.eval_weights(rows.to(a.d), full=True), b.eval_weights(rows.to(b.d), full=True), 'eval weights')
    return rows.numel()


def test_step_runs_on_cpu_with_oracle_backend():
    """The step itself on CPU tensors with the oracle kernels: invariants of srm2/train.py:474-477 hold and every
    class of rows occurs."""
    from elara_amd.step import run
    cfg = config(T=5, lo=100, hi=3000, B=300, steps=40, C=700, n_static=400)
    st = make(cfg, 'cpu', OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2))
    run(st, cfg['batches'], grads_fn(cfg, 'cpu'))
    K = st.K
    ent = st.ent[:st.R * K].view(st.R, K)
    assert int(st.live) == int((ent >= 0).sum()) and int(st.live) + int(st.n_lfree) == int(st.log_top)
    s = st.stats
    assert s['hits'] and s['adm'] and s['ev'] and s['compactions'] and s['appends'] and s['F'], s
    # rows that reached M hold MAT slots; codes are I, L_1..L_K or M only
    assert torch.all(st.loc[:st.R][st.code == st.MAT][st.slot_of[st.code == st.MAT] < 0] >= 0)
    assert int(st.code.min()) >= 0 and int(st.code.max()) <= st.MAT


def test_step_weights_do_not_depend_on_the_allocation_order():
    """Log ids are storage addresses only (srm2/elara_kernels.py:5-7): the same batches planned in the default and in
    the Triton directory's allocation order give bitwise the same weights and moments for every touched row, the
    same codes, MAT slots and residency, while the log ids themselves differ."""
    from elara_amd.step import run
    cfg = config(T=5, lo=100, hi=3000, B=300, steps=30, C=700, n_static=400, kthr=2)
    steps = {}
    for impl in ('cpp', 'triton'):
        st = make({**cfg, 'dir_impl': impl}, 'cpu', OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2))
        run(st, cfg['batches'], grads_fn(cfg, 'cpu'))
        steps[impl] = st
    a, b = steps['cpp'], steps['triton']
    rows = torch.unique(torch.cat(cfg['batches']))
    wa, wb = a.eval_weights(rows, full=True), b.eval_weights(rows, full=True)
    assert torch.equal(wa.view(torch.int32), wb.view(torch.int32))
    for name in ('code', 'loc', 'mat_top', 'live', 'slot_of', 'slot_row', 'adm_c0', 'rj', 'rok', 'pstep'):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert torch.equal(a.ent >= 0, b.ent >= 0) and not torch.equal(a.ent, b.ent)
    assert a.stats == b.stats and a.stats['compactions'] and a.stats['ev']


@pytest.mark.parametrize('where', ['cpu', pytest.param('gpu', marks=pytest.mark.gpu)])
def test_step_raises_on_rows_out_of_range(where, request):
    """A batch row outside [0, R) is an error of the caller (undefined in the reference): the plan raises before it
    changes the directory, instead of the kernels skipping the row."""
    from elara_amd.step import run
    cfg = config(T=4, lo=200, hi=2000, B=200, steps=4, C=800, n_static=300)
    dev = request.getfixturevalue('dev') if where == 'gpu' else 'cpu'
    st = make(cfg, dev, OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2) if where == 'cpu' else None)
    batches = [b.clone() for b in cfg['batches']]
    batches[2][5] = cfg['R'] + 7
    with pytest.raises(ValueError, match='outside'):
        run(st, batches, grads_fn(cfg, None))


@pytest.mark.gpu
@pytest.mark.parametrize('sync_free', [True, False])
def test_gpu_step_field_layout_raises_on_row_of_another_table(dev, sync_free):
    """With field_layout, a batch row that belongs to another table than its column's breaks the declared layout:
    the per-table sort reports it as a row outside [0, R), device-driven and host-planned, and the step raises."""
    from elara_amd.step import run
    print(f'[gpu-test] elara step field layout, row of another table, sync_free={sync_free}', flush=True)
    cfg = config(T=4, lo=200, hi=2000, B=1000, steps=4, C=800, n_static=300, field=True, sync_free=sync_free)
    st = make(cfg, dev)
    batches = [b.clone() for b in cfg['batches']]
    batches[2][5] = int(cfg['toff'][3]) + 1          # sample 1, table 1's column: a row of table 3
    with pytest.raises(ValueError, match='outside'):
        run(st, batches, grads_fn(cfg, None))


@pytest.mark.gpu
@pytest.mark.parametrize('name', ['small_evl', 'small_no_evl', 'small_S', 'small_overflow', 'host_arenas',
                                  'host_arenas_S', 'host_arenas_overflow', 'D64_K2', 'D256_K4', 'K1_kthr0',
                                  'L40_no_ring', 'D32_K8', 'D96', 'D200_K5_S', 'carry', 'carry_overflow_host',
                                  'evl_gate', 'triton', 'triton_host_S', 'small_overflow_hostsync',
                                  'triton_hostsync', 'carry_overflow', 'triton_overflow_S', 'host_arenas_hostsync',
                                  'hot_ids', 'small_batch'])
def test_gpu_step_matches_oracle_step(dev, name):
    """host_arenas*: the MAT and log arenas in pinned host memory (the capacity tier), read and written by the
    kernels over the host link -- with the update's host-arena writes on a link stream (the default:
    host_arenas_overflow, carry_overflow_host, triton_host_S), by the device-driven step on one stream (host_arenas,
    host_arenas_S), or by the native host-planned step on one stream (host_arenas_hostsync).  L40_no_ring: a look-ahead too long for the 32-bit ring of loaded batches, so the
    planner searches the next batches' sorted rows instead.  D32_K8, D96, D200_K5_S: widths the wave-per-row
    kernels do not take (the generic assembly and update kernels, srm2/gpu_ops.py:97 takes any D) and up to K = 8
    log entries per row.  carry*: carry residency (srm2/train.py:43 elara_carry); evl_gate: the representation
    switched on by memory pressure part way through (the reference's default, srm2/train.py:128-130).  triton*: the
    Triton directory's allocation order (srm2/elara_kernels.py), through the native step executor and, with host
    arenas and a link stream, through the call-by-call directory entry points.  Every configuration without a link
    stream, a host budget or a look-ahead beyond the ring runs the device-driven step (elr_step_dev: one native call and no host
    synchronisation per step, overflow and preemption resolved on the GPU); *_hostsync run the step that reads its
    class counts on the host instead.  hot_ids: ids of more than 240 occurrences in a batch (the segment
    sum's hot segments, summed from their partial chunks only); small_batch: 2,400 occurrences per batch (ATen's
    windowed order, no partial chunks)."""
    from elara_amd.step import run
    print(f'[gpu-test] elara step {name}', flush=True)
    kw = {'small_evl': {}, 'small_no_evl': {'evl': False}, 'small_S': {'st': 'S'}, 'small_overflow': {'C': 2000},
          'host_arenas': {'host': True, 'link': False}, 'host_arenas_S': {'host': True, 'st': 'S', 'link': False},
          'host_arenas_overflow': {'host': True, 'C': 2000},
          'host_arenas_hostsync': {'host': True, 'sync_free': False, 'link': False},
          'D64_K2': {'D': 64, 'K': 2, 'kthr': 2}, 'D256_K4': {'D': 256, 'K': 4, 'kthr': 3},
          'K1_kthr0': {'K': 1, 'kthr': 0}, 'L40_no_ring': {'L': 40}, 'D32_K8': {'D': 32, 'K': 8, 'kthr': 6},
          'D96': {'D': 96}, 'D200_K5_S': {'D': 200, 'K': 5, 'kthr': 4, 'st': 'S'}, 'carry': {'dyn': 'carry'},
          'carry_overflow_host': {'dyn': 'carry', 'C': 1800, 'host': True},
          'evl_gate': {'evl': 2, 'budget': 14_000_000, 'chunk': 64 << 10}, 'triton': {'dir_impl': 'triton'},
          'triton_host_S': {'dir_impl': 'triton', 'host': True, 'st': 'S', 'kthr': 2},
          'small_overflow_hostsync': {'C': 2000, 'sync_free': False}, 'triton_hostsync': {'dir_impl': 'triton',
                                                                                          'sync_free': False},
          'carry_overflow': {'dyn': 'carry', 'C': 1800}, 'triton_overflow_S': {'dir_impl': 'triton', 'C': 2000,
                                                                               'st': 'S', 'kthr': 2},
          'hot_ids': {'lo': 30, 'B': 1500}, 'small_batch': {'B': 400}}[name]
    cfg = config(**{'T': 6, 'lo': 200, 'hi': 20000, 'B': 1000, 'steps': 40, 'C': 2500, 'n_static': 1500, **kw})
    g = make(cfg, dev)
    assert (g.next_bits is None) == (name == 'L40_no_ring')
    c = make(cfg, 'cpu', OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2))
    gf = grads_fn(cfg, None)
    run(g, cfg['batches'], gf)
    run(c, cfg['batches'], gf)
    torch.cuda.synchronize()
    assert compare(g, c, cfg) > 0
    assert same_stats(g, c), (g.stats, c.stats)
    if g.sync_free:   # the device-driven step: no host synchronisation in the steps (one at the end of the run)
        assert g.stats['syncs'] <= 1, g.stats
    link = cfg.get('host', False) if cfg.get('link') is None else cfg['link']   # the default: on with host arenas
    assert (g._link is not None) == link, name
    assert g.sync_free == (not link and not cfg.get('budget') and name != 'L40_no_ring'
                           and cfg.get('sync_free', True)), name
    if name in ('host_arenas_overflow', 'carry_overflow_host'):
        assert g.stats['overflow'] > 0 and g._link is not None, g.stats
    if name == 'carry_overflow_host':
        assert g.stats['barriers'] > 0, g.stats
    if name == 'evl_gate':
        assert 1 < g.stats.get('evl_on_step', 0) < cfg['steps'], g.stats


@pytest.mark.gpu
def test_gpu_device_driven_step_raises_capacity_like_host_planned(dev):
    """A log arena too small for the run: the host-planned step raises at the plan of the step that could run past
    it, before any directory call; the device-driven step finds it on the GPU, that step and every later one do
    nothing, and the run raises the same error (same step, same bounds) when the host reads it.  The directory,
    the pool, the resident histories and the arenas are then equal in both."""
    from elara_amd.step import run
    print('[gpu-test] device-driven capacity error', flush=True)
    cfg = config(T=6, lo=200, hi=20000, B=1000, steps=30, C=2500, n_static=1500)
    cfg['log_cap'] = 8_000   # the run needs about 13,900 log entries: step 12 or so runs past this
    runs, msgs = {}, {}
    for sf in (False, True):
        st = make({**cfg, 'sync_free': sf}, dev)
        assert st.sync_free == sf
        with pytest.raises(RuntimeError, match='arena capacity') as ei:
            run(st, cfg['batches'], grads_fn(cfg, None))
        runs[sf], msgs[sf] = st, str(ei.value)
    assert msgs[True] == msgs[False], msgs
    a, b = runs[True], runs[False]
    torch.cuda.synchronize()
    for name in ('code', 'loc', 'ent', 'n_lfree', 'log_top', 'mat_top', 'live', 'adm_c0', 'rj', 'pstep', 'slot_of',
                 'slot_row', 'rok', 'pool', 'glog'):
        x, y = getattr(a, name), getattr(b, name)
        if name == 'glog':   # its last row is the trash row of the hits that record nothing (contents unspecified)
            x, y = x[:-1], y[:-1]
        if x.dtype == torch.float32:
            x, y = x.view(torch.int32), y.view(torch.int32)
        assert torch.equal(x, y), name
    lt, mt = int(a.log_top), int(a.mat_top)
    assert torch.equal(a.logs[:lt].view(torch.int32), b.logs[:lt].view(torch.int32))
    assert torch.equal(a.mat[:mt].view(torch.int32), b.mat[:mt].view(torch.int32))
    assert torch.equal(a.dyn_slots, b.dyn_slots) and torch.equal(a.free, b.free)


@pytest.mark.gpu
@pytest.mark.parametrize('name', ['evl', 'no_evl_S', 'host_arenas'])
def test_gpu_native_update_matches_python_update(dev, name):
    """elr_step_exec (directory calls, admissions, assembly and update in one native call; host arenas: the
    update's two parts by elr_step_update) against the same step issued call by call from Python over the same HIP
    kernels."""
    from elara_amd.step import HipBackend, run

    class CallByCall(HipBackend):
        step_update = None
        step_exec = None
        step_dev = None

    print(f'[gpu-test] native update {name}', flush=True)
    kw = {'evl': {}, 'no_evl_S': {'evl': False, 'st': 'S'}, 'host_arenas': {'host': True}}[name]
    cfg = config(T=6, lo=200, hi=20000, B=1000, steps=30, **{'C': 2500, 'n_static': 1500, **kw})
    a = make(cfg, dev)
    b = make(cfg, dev, CallByCall(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2, dev))
    gf = grads_fn(cfg, None)
    run(a, cfg['batches'], gf)
    run(b, cfg['batches'], gf)
    torch.cuda.synchronize()
    assert compare(a, b, cfg) > 0
    assert same_stats(a, b)
    assert a.sync_free == (name != 'host_arenas') and not b.sync_free
    s = a.stats
    need = ('hits', 'adm', 'ev', 'appends', 'S') if name == 'no_evl_S' else ('hits', 'adm', 'ev', 'appends',
                                                                            'compactions')
    assert all(s[k] for k in need), s


@pytest.mark.gpu
@pytest.mark.parametrize('name', ['one_batch_repeated', 'two_batches_alternating'])
def test_gpu_step_degenerate_batches(dev, name):
    """Batches that repeat: one batch over and over (from its second step most rows are hits, and steps come with
    few or no admissions, appends or compactions, so the native executor issues paired launches with an empty
    side), and two batches alternating (rows leave and come back every other step).  Equal to the oracle-driven
    step."""
    from elara_amd.step import run
    print(f'[gpu-test] elara step {name}', flush=True)
    cfg = config(T=6, lo=200, hi=20000, B=1000, steps=12, C=9000, n_static=1500)
    b = cfg['batches']
    cfg['batches'] = [b[0]] * 12 if name == 'one_batch_repeated' else [b[0], b[1]] * 6
    g = make(cfg, dev)
    c = make(cfg, 'cpu', OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2))
    gf = grads_fn(cfg, None)
    run(g, cfg['batches'], gf)
    run(c, cfg['batches'], gf)
    torch.cuda.synchronize()
    assert compare(g, c, cfg) > 0
    assert same_stats(g, c)
    assert g.stats['hits'] > g.stats['adm'] > 0, g.stats


@pytest.mark.gpu
@pytest.mark.parametrize('sync_free,ahead,field,fold', [(True, True, False, True), (False, True, False, True),
                                                        (True, False, False, True), (True, True, True, True),
                                                        (False, True, True, True), (True, True, False, False)])
def test_gpu_step_ragged_batches(dev, sync_free, ahead, field, fold):
    """Batches of changing sizes (a later batch larger than any before it, then smaller ones): run() takes each
    batch's dedup-plan buffers from its pool, and a batch that outgrows every free entry gets new ones.  Device-
    driven and host-planned, with the sorts on a second stream or on the step's own, sorted per table (the smallest
    batches, of at most 3,072 ids, then take the general sort), and device-driven with each batch loaded ahead
    marked by the step before (the default) or by a launch of its own.  Equal to the oracle-driven step."""
    from elara_amd.step import run
    print(f'[gpu-test] elara step ragged batches sync_free={sync_free} ahead={ahead} field={field} fold={fold}',
          flush=True)
    sizes = [300, 100, 800, 200, 1600, 50, 1200, 400, 2400, 150, 700, 1000, 90, 3000, 500, 250]
    tabs = synth.C5Tables(T=6, lo=200, hi=20000, alpha=1.1, seed=5)
    rng = np.random.default_rng(12)
    static = tabs.static_rows(rng, 1000, 1500, n_batches=10)
    batches = [torch.from_numpy(tabs.batch(rng, b)) for b in sizes]
    O = sum(b.numel() for b in batches)
    cfg = dict(toff=tabs.toff, R=tabs.R, D=128, C=9000, static=static, steps=len(sizes), bound=synth.bound_for(128),
               log_cap=O + 16, mat_cap=min(tabs.R + 1, O + 16), batches=batches, sync_free=sync_free, field=field)
    g = make(cfg, dev)
    g.dedup_ahead = ahead
    g.fold_mark = fold
    c = make(cfg, 'cpu', OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2))
    gf = grads_fn(cfg, None)
    run(g, cfg['batches'], gf)
    run(c, cfg['batches'], gf)
    torch.cuda.synchronize()
    assert compare(g, c, cfg) > 0
    assert same_stats(g, c)
    assert g.sync_free == sync_free
    pool = g._plan_pool
    assert pool is not None and pool.made >= 2, 'the dedup plans come from the pool'


@pytest.mark.gpu
@pytest.mark.parametrize('dir_impl,steps,field', [('cpp', 200, True), ('triton', 100, False)])
def test_gpu_step_c5_full_shape(dev, dir_impl, steps, field):
    """Config C5 shapes: 26 tables (vocab log-uniform in [1e3, 4e7], ~75M rows), batch 16,384 x 26 Zipf(1.1),
    D = 128, pool 337,626 (321,242 static hot rows), K = 3, evl on; 200 steps (the pool's steady-state churn and
    m / v of hot rows over many steps), HIP vs oracle bitwise: directory, pool, histories, arenas and the
    eval-style weights of every touched row.  Arena capacities as measured at this shape (about 47k log entries
    and 7k MAT rows per step in steady state) with headroom; the plan's capacity check raises if they run out.
    The 200 steps sort each batch per table (as bench.py's C5 line does), the 100 steps in the Triton directory's
    allocation order with the general sort."""
    from elara_amd.step import run
    print(f'[gpu-test] elara step C5 full shape, {steps} steps, {dir_impl} order, field={field}', flush=True)
    cfg = config(T=26, lo=1e3, hi=4e7, B=16384, steps=steps, C=337_626, n_static=337_626 - 16_384,
                 dir_impl=dir_impl, field=field)
    cfg['log_cap'] = 2_000_000 + steps * 60_000
    cfg['mat_cap'] = 1_000_000 + steps * 12_000
    g = make(cfg, dev)
    c = make(cfg, 'cpu', OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2, nthreads=16))

    def grads(j):   # the same occurrence gradients for both runs, drawn on the GPU (drawing 54M fp64 normals
        gen = torch.Generator(dev).manual_seed(1000 + j)   # per step on the host would dominate the test's time)
        return torch.randn(cfg['batches'][j].numel(), cfg['D'], device=dev, generator=gen) * 1e-3

    run(g, cfg['batches'], grads)
    torch.cuda.synchronize()
    run(c, cfg['batches'], lambda j: grads(j).cpu(),
        on_step=lambda s, p: print(f'[gpu-test] C5 oracle step {s}', flush=True) if s % 50 == 0 else None)
    assert compare(g, c, cfg) > 1_000_000
    assert same_stats(g, c)
    assert g.sync_free and g.stats['syncs'] <= 1, g.stats   # no host synchronisation in the 200 steps


@pytest.mark.gpu
@pytest.mark.parametrize('name', ['small_evl', 'small_S', 'carry'])
def test_gpu_plan_classify_matches_oracle(dev, name):
    """elr_plan_classify against the oracle's torch restatement of the planner classification, on every plan of
    a run (states as the step produces them, including steps that preempt and overflow): every output bitwise,
    with the next batches given as sorted lists and again as a ring of loaded batches (which the plan updates by
    clearing its own step's bit)."""
    from elara_amd.planner import plan_classify
    from elara_amd.step import run
    print(f'[gpu-test] plan classify {name}', flush=True)
    kw = {'small_evl': {}, 'small_S': {'st': 'S'}, 'carry': {'dyn': 'carry', 'C': 1800}}[name]
    cfg = config(T=6, lo=200, hi=20000, B=1000, steps=30, **{'C': 2000, 'n_static': 1500, **kw})
    be = OracleBackend(cfg['D'], 42, cfg['bound'], HP, cfg['steps'] + 2)
    calls = []
    orig = be.plan_classify

    def both(*args, **kw):
        want = orig(*args, **kw)
        kw = {k: v.to(dev) if isinstance(v, torch.Tensor) else v for k, v in kw.items()}
        g = [a.to(dev) if isinstance(a, torch.Tensor) else a for a in args]
        g[1] = [x.to(dev) for x in args[1]]
        s, R = int(args[11]), int(args[15])
        # the same plan with a ring of loaded batches in place of the sorted next batches: bit (s + k) % 32 set on
        # the rows of next batch k, the batch's own bit on its rows, and unrelated bits as noise
        bits = torch.zeros(R, dtype=torch.int32, device=dev)
        mask = 0
        for k, x in enumerate(g[1], start=1):
            b = (s + k) % 32
            bits[x] |= (1 << b) - (1 << 32 if b == 31 else 0)
            mask |= 1 << b
        noise = (1 << ((s + 7) % 32)) | (1 << ((s + 20) % 32))
        noise_rows = torch.arange(0, R, 3, device=dev)
        bits[noise_rows] |= noise - (1 << 32 if noise >= 1 << 31 else 0)
        own = 1 << (s % 32)
        bits[g[0]] |= own - (1 << 32 if own >= 1 << 31 else 0)
        before = bits.clone()
        for ring in (None, (bits, mask)):
            got = (plan_classify(*g, **kw) if ring is None
                   else plan_classify(*g, next_bits=ring[0], next_mask=ring[1], **kw))
            for f in want._fields:
                x, y = getattr(want, f), getattr(got, f).cpu()
                if f in ('L_row', 'L_cnt'):   # valid up to the L-row count
                    assert int(want.counts[4] + want.counts[5] + want.counts[6]) == x.numel() <= y.numel(), f
                    y = y[:x.numel()]
                assert x.dtype == y.dtype and torch.equal(x, y), (len(calls), f, ring is not None)
        # the plan cleared its own step's bit on the batch's rows and nothing else
        expect = before.clone()
        expect[g[0]] &= ~own if own < 1 << 31 else ~(own - (1 << 32))
        assert torch.equal(bits, expect), len(calls)
        calls.append(int(want.counts[10]))
        return want
    be.plan_classify = both
    st = make(cfg, 'cpu', be)
    run(st, cfg['batches'], grads_fn(cfg, 'cpu'))
    assert len(calls) == cfg['steps']
    assert (name == 'carry' or st.stats['preempt'] > 0) and st.stats['overflow'] > 0 and sum(calls) > 0, st.stats


@pytest.mark.gpu
@pytest.mark.parametrize('n_occ,D', [(2_000, 128), (60_000, 128), (400_000, 128), (150_000, 96), (100_000, 64)])
def test_gpu_plan_classify_seg_matches_separate_calls(dev, n_occ, D):
    """elr_plan_classify_seg (the classification with the segment sum's partial chunks in its first launch) and
    elr_segment_sum_plan_final give bitwise what elr_plan_classify and elr_segment_sum_plan give, on Zipf batches
    with hot ids (partial chunks), a batch on ATen's windowed path (no partial chunks) and widths of the generic
    kernels.  The split call runs first, on its own freshly sorted plan, so that it cannot read partial chunks the
    other call left behind."""
    from elara_amd.dedup import segment_sum_plan, unique_plan
    from elara_amd.planner import plan_classify
    print(f'[gpu-test] plan classify seg n={n_occ} D={D}', flush=True)
    g = torch.Generator(device='cpu').manual_seed(n_occ + D)
    R, C, T, K = 200_000, 6_000, 4, 3
    vocab = torch.randperm(R, generator=g)[:50_000]
    w = 1.0 / torch.arange(1, vocab.numel() + 1, dtype=torch.float64) ** 1.1
    ids = vocab[torch.multinomial(w, n_occ, replacement=True, generator=g)].to(dev)
    grad = (torch.randn(n_occ, D, generator=g) * 1e-2).to(dev)
    slot_of = torch.full((R,), -1, dtype=torch.int32)
    held = torch.randperm(R, generator=g)[:C - 100]
    slot_of[held] = torch.arange(C - 100, dtype=torch.int32)
    slot_row = torch.full((C,), -1, dtype=torch.int64)
    slot_row[:C - 100] = held
    state = dict(slot_of=slot_of, last_seen=torch.randint(0, 12, (R,), generator=g, dtype=torch.int32),
                 code=torch.randint(0, K + 2, (R,), generator=g, dtype=torch.int8),
                 kthr=torch.randint(0, K + 1, (T,), generator=g, dtype=torch.int8),
                 toff=torch.tensor([0, R // 4, R // 2, 3 * R // 4], dtype=torch.int64),
                 dyn=torch.arange(500, C - 100, dtype=torch.int64), slot_row=slot_row,
                 mat_top=torch.tensor([7], dtype=torch.int64), log_top=torch.tensor([11], dtype=torch.int64))
    st = {k: v.to(dev) for k, v in state.items()}
    nxt = [torch.unique(vocab[torch.randint(0, 20_000, (3_000,), generator=g)]).to(dev)]
    loc = torch.randint(-1, 1000, (R + 1,), generator=g, dtype=torch.int32).to(dev)
    args = lambda u: (u, nxt, st['slot_of'], st['last_seen'], st['code'], st['kthr'], st['toff'],  # noqa: E731
                      st['dyn'], st['slot_row'], st['mat_top'], st['log_top'], 6, K, True)
    u_b, plan_b = unique_plan(ids, D, R)
    pc_b = plan_classify(*args(u_b), loc=loc, R=R, seg=(grad, plan_b))
    G_b = segment_sum_plan(grad, plan_b, torch.empty(u_b.numel(), D, device=dev), pc_b.rank, partials_done=True)
    u_a, plan_a = unique_plan(ids, D, R)
    pc_a = plan_classify(*args(u_a), loc=loc, R=R)
    G_a = segment_sum_plan(grad, plan_a, torch.empty(u_a.numel(), D, device=dev), pc_a.rank)
    torch.cuda.synchronize()
    assert torch.equal(u_a, u_b)
    nL = int(pc_a.counts[4] + pc_a.counts[5] + pc_a.counts[6])
    for f in pc_a._fields:
        x, y = getattr(pc_a, f), getattr(pc_b, f)
        if f in ('L_row', 'L_cnt'):   # valid up to the L-row count
            x, y = x[:nL], y[:nL]
        assert (x is None) == (y is None) and (x is None or torch.equal(x, y)), f
    assert torch.equal(G_a, G_b)
    hot = int(torch.bincount(ids).max())
    assert (n_occ <= 3072) or hot > 240, hot   # partial chunks exist beyond the windowed path


@pytest.mark.gpu
def test_gpu_plan_classify_skips_rows_out_of_range(dev):
    """Rows of u outside [0, R) come out as class S with no pool slot, code K+1 and MAT slot -1 (which every later
    copy and update skips) and are read nowhere out of bounds; the rows in range are classified as without them."""
    from elara_amd.planner import plan_classify
    print('[gpu-test] plan classify, rows out of range', flush=True)
    cfg = config(T=4, lo=200, hi=2000, B=200, steps=4, C=800, n_static=300)
    st = make(cfg, dev)
    R, K = st.R, st.K
    u = torch.unique(cfg['batches'][0].to(dev))
    bad = torch.tensor([R, R + 5, 2**40], dtype=torch.int64, device=dev)

    def classify(uu):
        return plan_classify(uu, [], st.slot_of, st.last_seen, st.code, st.kthr, st.toff, st.dyn_slots, st.slot_row,
                             st.mat_top, st.log_top, 1, K, True, st.loc, R)
    a, b = classify(u), classify(torch.cat([u, bad]))
    torch.cuda.synchronize()
    n = u.numel()
    for f in ('cls', 'flags', 'sl', 'c'):
        assert torch.equal(getattr(b, f)[:n].cpu(), getattr(a, f).cpu()), f
    assert (b.cls[n:] == 9).all() and (b.sl[n:] == -1).all() and (b.c[n:] == K + 1).all() and (b.flags[n:] == 0).all()
    assert (b.loc_ord[b.rank[n:]] == -1).all()
    assert int(b.counts[9]) == int(a.counts[9]) + 3
    assert int(b.counts[16]) == 3 and int(a.counts[16]) == 0   # counted for the step, which raises on them


@pytest.mark.gpu
def test_gpu_assemble_and_admit_match_oracle(dev):
    """elr_assemble (init / replay by entry id / MAT gather segments, including empty ones) and elr_plan_admit
    against the oracle backend's restatements, on synthetic arenas."""
    from elara_amd.step import HipBackend
    print('[gpu-test] assemble + admit', flush=True)
    rng = np.random.default_rng(21)
    D, K, R, S = 128, 3, 5000, 40
    hb = HipBackend(D, 42, synth.bound_for(D), HP, S, dev)
    ob = OracleBackend(D, 42, synth.bound_for(D), HP, S)
    logs = torch.from_numpy(rng.standard_normal((700, D)).astype(np.float32) * 1e-3)
    mat = torch.from_numpy(rng.standard_normal((300, 3, D)).astype(np.float32))
    loc = torch.full((R + 1,), -1, dtype=torch.int32)
    nL = 90
    L_cnt = torch.from_numpy(rng.integers(1, K + 1, nL).astype(np.int32))
    L_ids = torch.full((nL, K), -1, dtype=torch.int32)
    L_steps = torch.zeros((nL, K), dtype=torch.int32)
    perm = rng.permutation(700)
    q = 0
    for i in range(nL):
        c = int(L_cnt[i])
        L_ids[i, :c] = torch.from_numpy(perm[q:q + c].astype(np.int32))
        L_steps[i, :c] = torch.from_numpy(np.sort(rng.choice(np.arange(1, S), c, replace=False)).astype(np.int32))
        q += c
    sizes = [17, 30, 0, 25, 40, 11, 20, 9]        # NADM, LADM, FADM, NAPP, LAPP, NCMP, LCMP, FN
    kinds = [0, 1, 2, 0, 1, 0, 1, 2]
    rows = torch.from_numpy(rng.choice(R, sum(sizes), replace=False).astype(np.int64))
    segs, end, aux = [], 0, 0
    for m, kd in zip(sizes, kinds):
        end += m
        segs.append((end, kd, aux if kd == 1 else 0))
        if kd == 1:
            aux += m
        if kd == 2:
            r = rows[end - m:end]
            loc[r] = torch.from_numpy(rng.choice(300, m, replace=False).astype(np.int32))
    want = ob.assemble(rows, segs, L_ids, L_steps, L_cnt, logs, mat, loc, K)
    got = hb.assemble(rows.to(dev), segs, L_ids.to(dev), L_steps.to(dev), L_cnt.to(dev), logs.to(dev),
                      mat.to(dev), loc.to(dev), K)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int32), want.view(torch.int32))
    # admissions: 60 rows into dynamic slots, the first 35 lazy (N/L)
    C, n0 = 400, 100
    code = torch.from_numpy(rng.integers(0, K + 2, R).astype(np.int8))
    st = lambda: [torch.full((R,), -1, dtype=torch.int32), torch.full((C,), -1, dtype=torch.int64),  # noqa: E731
                  torch.full((C,), -1, dtype=torch.int8), torch.zeros(C, dtype=torch.int8),
                  torch.zeros(C, dtype=torch.int8), torch.zeros((C - n0 + 1, K), dtype=torch.int32)]
    a_rows = torch.from_numpy(rng.choice(R, 60, replace=False).astype(np.int64))
    a_slots = torch.from_numpy(rng.choice(np.arange(n0, C), 60, replace=False).astype(np.int64))
    for evl in (True, False):
        o = st()
        ob.plan_admit(a_rows, a_slots, 35, evl, 7, n0, C, R, K, code, *o)
        g = [t.to(dev) for t in st()]
        hb.plan_admit(a_rows.to(dev), a_slots.to(dev), 35, evl, 7, n0, C, R, K, code.to(dev), *g)
        torch.cuda.synchronize()
        for x, y in zip(o, g):
            assert torch.equal(x, y.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize('n_free,nev,n_adm,nkeep', [(50, 20, 30, 40), (50, 20, 60, 10), (10, 30, 40, 0),
                                                    (40, 0, 15, 25), (5, 8, 0, 30), (0, 12, 12, 3)])
def test_gpu_plan_admit_slots_matches_stack_arithmetic(dev, n_free, nev, n_adm, nkeep):
    """elr_plan_admit_slots against the free-stack arithmetic it replaces (srm2/elara.py:345-347, 368, as the step
    writes it with torch ops): pool_free = cat(free, ev_slot), the top n_adm entries admitted, the rest the new
    stack, the new slot list cat(keep, admitted); and the admissions' directory fields against plan_admit."""
    from elara_amd.step import HipBackend
    print(f'[gpu-test] admit_slots n_free={n_free} nev={nev} n_adm={n_adm} nkeep={nkeep}', flush=True)
    rng = np.random.default_rng(n_free * 7 + nev * 3 + n_adm)
    D, K, R, C, n0 = 64, 3, 3000, 400, 100
    hb = HipBackend(D, 42, synth.bound_for(D), HP, 20, dev)
    ob = OracleBackend(D, 42, synth.bound_for(D), HP, 20)
    slots = rng.permutation(np.arange(n0, C)).astype(np.int64)
    free, ev_slot, keep = slots[:n_free], slots[n_free:n_free + nev], slots[n_free + nev:n_free + nev + nkeep]
    pool_free = np.concatenate([free, ev_slot])
    adm = pool_free[pool_free.size - n_adm:]
    a_rows = torch.from_numpy(rng.choice(R, n_adm, replace=False).astype(np.int64))
    lazy = n_adm // 2
    code = torch.from_numpy(rng.integers(0, K + 2, R).astype(np.int8))
    st = lambda: [torch.full((R,), -1, dtype=torch.int32), torch.full((C,), -1, dtype=torch.int64),  # noqa: E731
                  torch.full((C,), -1, dtype=torch.int8), torch.zeros(C, dtype=torch.int8),
                  torch.zeros(C, dtype=torch.int8), torch.zeros((C - n0 + 1, K), dtype=torch.int32)]
    o = st()
    ob.plan_admit(a_rows, torch.from_numpy(adm.copy()), lazy, True, 9, n0, C, R, K, code, *o)
    fbuf = torch.full((C,), -7, dtype=torch.int64)
    fbuf[:n_free] = torch.from_numpy(free)
    fbuf = fbuf.to(dev)
    dyn = torch.full((C,), -7, dtype=torch.int64, device=dev)
    g = [t.to(dev) for t in st()]
    got = hb.plan_admit_slots(fbuf, n_free, torch.from_numpy(ev_slot).to(dev), torch.from_numpy(keep).to(dev),
                              a_rows.to(dev), lazy, True, 9, n0, C, R, K, code.to(dev), *g, dyn)
    torch.cuda.synchronize()
    rest = pool_free.size - n_adm
    assert np.array_equal(got.cpu().numpy(), adm)
    assert np.array_equal(fbuf.cpu().numpy()[:rest], pool_free[:rest])
    assert np.array_equal(fbuf.cpu().numpy()[rest:], np.full(C - rest, -7)) or rest < n_free
    assert np.array_equal(dyn.cpu().numpy()[:nkeep + n_adm], np.concatenate([keep, adm]))
    assert (dyn.cpu().numpy()[nkeep + n_adm:] == -7).all()
    for x, y in zip(o, g):
        assert torch.equal(x, y.cpu())
