"""State directory (srm2/csrc/elara_dir.cpp elara_dir_a / elara_dir_b): the C oracle against the reference's own
build (oracle/_ref, CPU tensors) and the HIP path (elr_dir_a / elr_dir_b through the C-ABI) against both.  The
Triton path's allocation order (srm2/elara_kernels.py; the oracle's deferred releases, elr_dir_a_deferred,
elr_dir_evict_deferred, elr_dir_b_release) is pinned by the reference planner's golden vectors
(tests/test_planner_golden.py), by a hand-worked step and by its equality with the default order in everything
but the log ids; the GPU calls and the Triton front end are checked against it here.

Every step compares all 9 + 2 outputs and the whole directory (17 arrays) bitwise, except the two trash elements
lstep[Lcap] and lfree[Lcap], whose contents the reference leaves unspecified.  Each run also checks the invariants
of srm2/train.py:474-477 (dir_check) and a few more (no id both live and free, codes match entry counts).
"""
import numpy as np
import pytest

from dirsim import (FacadeImpl, OracleImpl, Sim, TorchImpl, check_invariants, comparable_state, diff_outputs,
                    diff_states)
from oracle import oracle as O
from oracle import ref

needs_ref = pytest.mark.skipif(ref.dir() is None, reason='oracle/_ref not built (needs /root/reference)')

CONFIGS = {
    'default': dict(seed=1),
    'k4_no_static': dict(seed=2, K=4, R=3000, C=500, n0=0, batch=400),
    'evl_off': dict(seed=3, evl=False),
    'k1_one_table': dict(seed=4, K=1, T=1, kthr=[1]),
    'tight_pool': dict(seed=5, R=1500, C=120, n0=10, batch=300),
}


def run(sim, impls, steps):
    """Drive `steps` plan steps; assert every implementation equals the first one after each call."""
    for s in range(1, steps + 1):
        outs = sim.step(s, impls)
        va = comparable_state(impls[0].view(), sim)
        for m, o in zip(impls[1:], outs[1:]):
            d = diff_states(va, comparable_state(m.view(), sim))
            ba, bb = diff_outputs(outs[0][0], o[0]), diff_outputs(outs[0][1], o[1])
            assert not (d or ba or bb), f'step {s}: {type(m).__name__} differs: state {d}, outputs A {ba}, B {bb}'
        check_invariants(impls[0].view(), sim)
    return impls


@needs_ref
@pytest.mark.parametrize('name', sorted(CONFIGS))
def test_oracle_matches_reference_directory(name):
    sim = Sim(**CONFIGS[name])
    st0 = sim.initial_state()
    run(sim, [TorchImpl(sim, st0, ref.dir()), OracleImpl(sim, st0)], 60)


def test_oracle_allocators_by_hand():
    """Hand-worked allocation sequence: bump, release onto the stack, pops top-down (elara_dir.cpp:13-34)."""
    R, C, K = 10, 4, 3
    st = O.DirState(R, C, K, 0, np.array([0], np.int64), np.array([3], np.int8), log_cap=20)
    pv = st.params(True)
    # appends: rows 2, 5, 7 at k = 0 -> ids 0, 1, 2 (bump), code 1
    a_ids, c_slots = O.dir_b(st, pv, [2, 5, 7], [0, 0, 0], [], [], 4)
    assert a_ids.tolist() == [0, 1, 2] and st.log_top[0] == 3 and st.live[0] == 3 and st.n_lfree[0] == 0
    assert st.code[[2, 5, 7]].tolist() == [1, 1, 1] and st.lstep[:3].tolist() == [4, 4, 4]
    # compact rows 5 and 2 (1 entry each): MAT slots 0, 1; ids 1, 0 pushed in that order
    a_ids, c_slots = O.dir_b(st, pv, [], [], [5, 2], [1, 1], 5)
    assert c_slots.tolist() == [0, 1] and st.mat_top[0] == 2
    assert st.lfree[:2].tolist() == [1, 0] and st.n_lfree[0] == 2 and st.live[0] == 1
    assert st.code[[5, 2]].tolist() == [4, 4] and st.ent[5 * K] == -1 and st.ent[2 * K] == -1
    # three appends: pop 0 (top), then 1, then bump 3
    a_ids, _ = O.dir_b(st, pv, [1, 3, 4], [0, 0, 0], [], [], 6)
    assert a_ids.tolist() == [0, 1, 3] and st.n_lfree[0] == 0 and st.log_top[0] == 4 and st.live[0] == 4
    # compacting row 2 again keeps its MAT slot
    _, c_slots = O.dir_b(st, pv, [], [], [2], [0], 7)
    assert c_slots.tolist() == [1] and st.mat_top[0] == 2


def test_oracle_triton_order_by_hand():
    """One step in both orders.  Row 1 (two host-log entries, ids 0 and 1) is evicted to M; then rows 3 and 4 are
    appended and row 2 (one entry, id 2) compacted.  Default order (elara_dir.cpp:80-94, 102-108): the eviction
    pushes ids 0 and 1 at once, the appends pop them (1, then 0), the compaction pushes 2.  Triton order
    (srm2/elara_kernels.py:152-209): the appends bump ids 3 and 4, then the releases push 0, 1 (the eviction's part)
    and 2 (the compaction's)."""
    R, C, K = 10, 4, 3
    res = {}
    for triton in (False, True):
        st = O.DirState(R, C, K, 0, np.array([0], np.int64), np.array([1], np.int8), log_cap=20)
        pv = st.params(True)
        a_ids, _ = O.dir_b(st, pv, [1, 1, 2], [0, 1, 0], [], [], 1)
        assert a_ids.tolist() == [0, 1, 2] and st.code[[1, 2]].tolist() == [2, 1]
        st.slot_of[1], st.slot_row[0], st.adm_c0[0], st.rj[0], st.rok[0] = 0, 1, 2, 0, 1   # row 1 admitted (L)
        e = np.empty(0, np.int64)
        out = O.dir_a(st, pv, e, e, np.empty(0, np.int32), [0], 2, deferred=triton)
        assert out[4].tolist() == [1] and not out[5][0] and out[7].tolist() == [0]      # to M, MAT slot 0
        if triton:
            assert out[9].tolist() == [2] and st.n_lfree[0] == 0 and st.ent[1 * K:1 * K + 2].tolist() == [0, 1]
        else:
            assert st.lfree[:2].tolist() == [0, 1] and st.n_lfree[0] == 2 and st.ent[1 * K] == -1
        a_ids, c_slots = O.dir_b(st, pv, [3, 4], [0, 0], [2], [1], 3, rel=(out[4], out[9]) if triton else None)
        assert c_slots.tolist() == [1] and st.code[[1, 2, 3, 4]].tolist() == [4, 4, 1, 1]
        res[triton] = (a_ids.tolist(), st.lfree[:int(st.n_lfree[0])].tolist(), int(st.log_top[0]), int(st.live[0]))
    assert res[False] == ([1, 0], [2], 3, 2)
    assert res[True] == ([3, 4], [0, 1, 2], 5, 2)


def test_oracle_triton_release_counts_every_entry():
    """The Triton path's release reserves stack positions by the requested counts and skips missing entries
    (srm2/elara_kernels.py:104-116, 199-209); this build packs the live ones.  They agree only while every counted
    entry exists, which the oracle asserts on every Triton-order release: a release item counting an entry the row
    does not hold fails loudly instead of giving other log ids."""
    R, C, K = 10, 4, 3
    st = O.DirState(R, C, K, 0, np.array([0], np.int64), np.array([3], np.int8), log_cap=20)
    pv = st.params(True)
    O.dir_b(st, pv, [2], [0], [], [], 1)                                  # row 2 holds one entry
    O.dir_b(st, pv, [], [], [], [], 2, rel=(np.array([2]), np.array([1])))   # counted 1, holds 1: fine
    O.dir_b(st, pv, [5], [0], [], [], 3)                                  # row 5 holds one entry
    with pytest.raises(AssertionError, match='2 entries counted, 1 live'):
        O.dir_b(st, pv, [], [], [5], [2], 4, rel=(np.zeros(0, np.int64),) * 2)


@pytest.mark.parametrize('name', sorted(CONFIGS))
def test_oracle_triton_order_changes_only_log_ids(name):
    """Over 60 planned steps the two orders agree on every state and output except the log ids: the same codes,
    MAT slots, residency and resident histories, the same rows holding log entries and the same logical step in
    each (lstep[ent[r, k]]), and only the ids themselves (and the free stack holding them) may differ; both keep
    the allocator invariants."""
    sim = Sim(**CONFIGS[name])
    st0 = sim.initial_state()
    a, b = OracleImpl(sim, st0), OracleImpl(sim, st0, triton=True)
    K, differs = sim.K, 0
    for s in range(1, 61):
        (A0, A1), (B0, B1) = sim.step(s, [a, b])   # calls A and B of each order
        va, vb = a.view(), b.view()
        for f in ('code', 'loc', 'mat_top', 'live', 'adm_c0', 'rj', 'rok', 'pstep', 'slot_of', 'slot_row'):
            assert np.array_equal(va[f], vb[f]), (s, f)
        ea, eb = va['ent'][:sim.R * K], vb['ent'][:sim.R * K]
        assert np.array_equal(ea >= 0, eb >= 0), s
        assert np.array_equal(va['lstep'][ea[ea >= 0]], vb['lstep'][eb[eb >= 0]]), s
        for k in (0, 2, 3, 4, 5, 7, 8):                   # call A's outputs except L_ids and evl_ids
            assert np.array_equal(np.asarray(A0[k]), np.asarray(B0[k])), (s, k)
        for k in (1, 6):
            assert np.array_equal(np.asarray(A0[k]) >= 0, np.asarray(B0[k]) >= 0), (s, k)
        assert np.array_equal(A1[1], B1[1]) and A1[0].size == B1[0].size, s     # c_slots; as many append ids
        differs += int(not np.array_equal(ea, eb))
        check_invariants(vb, sim)
    assert differs > 0 or not sim.evl   # the orders do differ once rows go to M with host logs


# ------------------------------------------------------------------------------------------------------------- GPU
def gpu_impl(sim, st0, dev, triton=False):
    from elara_amd.elara_dir import dir_ext
    return TorchImpl(sim, st0, dir_ext(), device=dev, triton=triton)


@pytest.mark.gpu
@pytest.mark.parametrize('name', sorted(CONFIGS))
def test_gpu_directory_matches_oracle_and_reference(dev, name):
    print(f'[gpu-test] directory {name}', flush=True)
    sim = Sim(**CONFIGS[name])
    st0 = sim.initial_state()
    impls = [OracleImpl(sim, st0), gpu_impl(sim, st0, dev)]
    if ref.dir() is not None:
        # the reference's own elara_dir.cpp, on CPU tensors and on the same GPU (ATen dispatches to HIP kernels)
        impls += [TorchImpl(sim, st0, ref.dir()), TorchImpl(sim, st0, ref.dir(), device=dev)]
    run(sim, impls, 60)


@pytest.mark.gpu
@pytest.mark.parametrize('name', sorted(CONFIGS))
def test_gpu_directory_facade_matches_oracle(dev, name):
    """The elara_kernels-style front end (hits / lsteps / Directory.evict / appends / compact / release), driven in
    the reference planner's fused-path call sequence, gives the same outputs and states as the oracle in the Triton
    path's allocation order, and so do elr_dir_a_deferred / elr_dir_b_release called as the step calls them."""
    print(f'[gpu-test] directory facade {name}', flush=True)
    sim = Sim(**CONFIGS[name])
    st0 = sim.initial_state()
    run(sim, [OracleImpl(sim, st0, triton=True), FacadeImpl(sim, st0, dev), gpu_impl(sim, st0, dev, True)], 60)


@pytest.mark.gpu
def test_gpu_directory_large_multiblock(dev):
    """Thousands of items per call: block offsets across many blocks of the grid-wide scans."""
    print('[gpu-test] directory large', flush=True)
    sim = Sim(seed=11, R=400_000, C=60_000, n0=5_000, K=3, T=6, batch=40_000, vocab_skew=0.9)
    st0 = sim.initial_state()
    run(sim, [OracleImpl(sim, st0), gpu_impl(sim, st0, dev)], 12)


@pytest.mark.gpu
def test_gpu_directory_evictions_beyond_fused_scan(dev):
    """More than 65,536 evictions in a call (more than 256 blocks): the eviction counts are scanned in a launch of
    their own instead of inside the apply kernel (the smaller calls of every other test take the fused path)."""
    print('[gpu-test] directory evictions beyond the fused scan', flush=True)
    sim = Sim(seed=14, R=600_000, C=400_000, n0=2_000, K=3, T=4, batch=500_000, vocab_skew=0.3)
    st0 = sim.initial_state()
    run(sim, [OracleImpl(sim, st0), gpu_impl(sim, st0, dev)], 5)
    assert sim.nev_max > 256 * 256


@pytest.mark.gpu
def test_gpu_directory_triton_order_beyond_fused_scan(dev):
    """The Triton path's order with more than 65,536 evictions per call: call B's release items (one per eviction,
    ahead of the compactions) take it past 256 blocks, so its counts are scanned in a launch of their own."""
    print('[gpu-test] directory triton order beyond the fused scan', flush=True)
    sim = Sim(seed=15, R=600_000, C=400_000, n0=2_000, K=3, T=4, batch=500_000, vocab_skew=0.3)
    st0 = sim.initial_state()
    run(sim, [OracleImpl(sim, st0, triton=True), gpu_impl(sim, st0, dev, True)], 5)
    assert sim.nev_max > 256 * 256


@pytest.mark.gpu
@pytest.mark.parametrize('nev', [256 * 256, 256 * 256 + 1])
def test_gpu_directory_evictions_at_the_fused_scan_limit(dev, nev):
    """Exactly 256 blocks of evictions (the apply kernel sums the block counts itself) and one item more (the
    counts are scanned in a launch of their own): call A's outputs and the whole directory equal the oracle's.  The
    evicted slots hold N, L and F rows with host-log entries, MAT slots and resident histories of every length, so
    that every allocator (log ids from the free stack and the bump pointer, MAT slots, releases) takes part."""
    import torch
    from elara_amd.elara_dir import dir_ext
    print(f'[gpu-test] directory evictions nev={nev}', flush=True)
    R, K, n0, Cdyn = 400_000, 3, 10, 70_000
    st = O.DirState(R, n0 + Cdyn, K, n0, np.array([0, R // 2], np.int64), np.array([2, 3], np.int8))
    pv = st.params(True)
    rng = np.random.default_rng(21 + nev)
    rows = rng.permutation(R)[:Cdyn].astype(np.int64)
    kind = rng.random(Cdyn)
    c0 = np.where(kind < 0.4, rng.integers(1, K + 1, Cdyn), np.where(kind < 0.7, 0, -1)).astype(np.int64)
    for k in range(K):                                  # the L rows' host-log entries (appends, oracle only)
        sel = rows[c0 > k]
        O.dir_b(st, pv, sel, np.full(sel.size, k, np.int64), [], [], 1 + k)
    f_rows = rows[c0 < 0]                               # F rows: materialised, half of them with a MAT slot
    st.code[f_rows] = st.MAT
    held = f_rows[::2]
    st.loc[held] = np.arange(held.size, dtype=np.int32)
    st.mat_top[0] = held.size
    some = rows[(c0 == 0) & (kind < 0.5)]               # and some N rows holding a MAT slot from earlier
    st.loc[some] = np.arange(held.size, held.size + some.size, dtype=np.int32)
    st.mat_top[0] += some.size
    free = rng.permutation(int(st.log_top[0]))[:5_000].astype(np.int32)   # a free stack to pop from
    st.ent[np.isin(st.ent, free)] = -1
    st.lfree[:free.size] = free
    st.n_lfree[0] = free.size
    st.live[0] = int((st.ent >= 0).sum())
    slots = np.arange(n0, n0 + Cdyn, dtype=np.int64)    # admissions, as the planner makes them
    st.slot_of[rows] = slots.astype(np.int32)
    st.slot_row[slots] = rows
    st.adm_c0[slots] = c0.astype(np.int8)
    j = rng.integers(0, K + 1, Cdyn)
    st.rj[slots] = j.astype(np.int8)
    st.rok[slots] = (rng.random(Cdyn) < 0.8).astype(np.int8)
    st.pstep[:Cdyn * K] = rng.integers(1, 50, Cdyn * K).astype(np.int32)
    ev_slot = rng.permutation(slots)[:nev]
    gst = [torch.from_numpy(getattr(st, f).copy()).to(dev) for f in O.DIR_FIELDS]
    e = np.empty(0, np.int64)
    want = O.dir_a(st, pv, e, e, np.empty(0, np.int32), ev_slot, 60)
    T = lambda a, dt=torch.int64: torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)  # noqa: E731
    got = dir_ext().elara_dir_a(gst, list(pv), T(e), T(e), T(e, torch.int32), T(ev_slot), 60)
    torch.cuda.synchronize()
    for k, (w, g) in enumerate(zip(want, got)):
        assert np.array_equal(np.asarray(w).reshape(-1), g.cpu().numpy().reshape(-1)), k
    for i, f in enumerate(O.DIR_FIELDS):
        a, b = getattr(st, f).reshape(-1), gst[i].cpu().numpy().reshape(-1)
        if f in ('lstep', 'lfree'):
            a, b = a[:-1], b[:-1]
        assert np.array_equal(a, b), f
    rep = np.asarray(want[5]).astype(bool)
    assert 0 < rep.sum() < nev and int(st.n_lfree[0]) > 0


@pytest.mark.gpu
def test_gpu_dir_b_scan_beyond_one_scan_block(dev):
    """300,000 compactions in one call (more than 1024 blocks: the single-block scan loops over chunks with a
    carry), then 200,000 appends that pop the whole free stack and continue with the bump pointer."""
    import torch
    from elara_amd.elara_dir import dir_ext
    print('[gpu-test] dir_b large scan', flush=True)
    rng = np.random.default_rng(12)
    R, K, C = 1_200_000, 3, 8
    st = O.DirState(R, C, K, 0, np.array([0], np.int64), np.array([3], np.int8))
    pv = st.params(True)
    perm = rng.permutation(R).astype(np.int64)
    logged, fresh = perm[:700_000], perm[700_000:900_000]
    cnt = rng.integers(1, 4, logged.size)
    for k in range(3):                                  # rows get 1..3 log entries (oracle only)
        sel = logged[cnt > k]
        O.dir_b(st, pv, sel, np.full(sel.size, k, np.int64), [], [], 1 + k)
    crow = logged[:300_000]
    ccnt = np.where(rng.random(crow.size) < 0.1, cnt[:300_000], 0).astype(np.int64)
    pre = crow[::2]                                     # half of them already hold a MAT slot
    st.loc[pre] = np.arange(pre.size, dtype=np.int32)
    st.mat_top[0] = pre.size
    gst = [torch.from_numpy(getattr(st, f).copy()).to(dev) for f in O.DIR_FIELDS]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    e = np.empty(0, np.int64)
    calls = [(e, e, crow, ccnt), (fresh, np.zeros(fresh.size, np.int64), e, e)]
    for s, (ar, ak, cr, cc) in enumerate(calls, start=10):
        want = O.dir_b(st, pv, ar, ak, cr, cc, s)
        got = dir_ext().elara_dir_b(gst, list(pv), T(ar), T(ak), T(cr), T(cc), s)
        torch.cuda.synchronize()
        for w, g in zip(want, got):
            assert np.array_equal(w, g.cpu().numpy())
        for i, f in enumerate(O.DIR_FIELDS):
            a, b = getattr(st, f).reshape(-1), gst[i].cpu().numpy().reshape(-1)
            if f in ('lstep', 'lfree'):
                a, b = a[:-1], b[:-1]
            assert np.array_equal(a, b), (s, f)
    assert 0 < st.n_lfree[0] or st.log_top[0] > 0


@pytest.mark.gpu
@pytest.mark.parametrize('nc', [256 * 256, 256 * 256 + 1])
@pytest.mark.parametrize('order', ['cpp', 'triton'])
def test_gpu_dir_b_at_the_fused_scan_limit(dev, nc, order):
    """Call B with exactly 256 blocks of items (the compaction kernel sums the block counts itself) and one item
    more (a scan launch of its own), together with appends that pop the free stack: outputs and directory equal the
    oracle's.  Items: nc compactions (cpp), or a third of them release items ahead of the compactions (triton,
    elr_dir_b_release)."""
    import torch
    from elara_amd.elara_dir import dir_ext
    print(f'[gpu-test] dir_b nc={nc} {order}', flush=True)
    rng = np.random.default_rng(30 + nc)
    R, K, C = 400_000, 3, 8
    st = O.DirState(R, C, K, 0, np.array([0], np.int64), np.array([3], np.int8))
    pv = st.params(True)
    perm = rng.permutation(R).astype(np.int64)
    logged, fresh = perm[:150_000], perm[150_000:160_000]
    cnt = rng.integers(1, 4, logged.size)
    for k in range(3):
        sel = logged[cnt > k]
        O.dir_b(st, pv, sel, np.full(sel.size, k, np.int64), [], [], 1 + k)
    crow = logged[:nc]
    ccnt = cnt[:nc].astype(np.int64)
    pre = crow[::3]                                     # a third already hold a MAT slot
    st.loc[pre] = np.arange(pre.size, dtype=np.int32)
    st.mat_top[0] = pre.size
    done = logged[nc:nc + 2_000]                        # their entries released earlier: a free stack to pop
    O.dir_b(st, pv, [], [], done, cnt[nc:nc + 2_000].astype(np.int64), 5)
    gst = [torch.from_numpy(getattr(st, f).copy()).to(dev) for f in O.DIR_FIELDS]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int64)).to(dev)  # noqa: E731
    rel = None
    if order == 'triton':
        nr = nc // 3
        rel = (crow[:nr], ccnt[:nr])
        crow, ccnt = crow[nr:], ccnt[nr:]
    want = O.dir_b(st, pv, fresh, np.zeros(fresh.size, np.int64), crow, ccnt, 9, rel=rel)
    got = dir_ext().elara_dir_b(gst, list(pv), T(fresh), T(np.zeros(fresh.size)), T(crow), T(ccnt), 9,
                                rel=None if rel is None else (T(rel[0]), T(rel[1])))
    torch.cuda.synchronize()
    for w, g in zip(want, got):
        assert np.array_equal(w, g.cpu().numpy())
    for i, f in enumerate(O.DIR_FIELDS):
        a, b = getattr(st, f).reshape(-1), gst[i].cpu().numpy().reshape(-1)
        if f in ('lstep', 'lfree'):
            a, b = a[:-1], b[:-1]
        assert np.array_equal(a, b), f


@pytest.mark.gpu
def test_gpu_directory_empty_calls(dev):
    import torch
    from elara_amd.elara_dir import dir_ext
    sim = Sim(seed=13)
    st0 = sim.initial_state()
    g = gpu_impl(sim, st0, dev)
    before = comparable_state(g.view(), sim)
    z = torch.empty(0, dtype=torch.int64, device=dev)
    out = dir_ext().elara_dir_a(g.st, list(sim.pv), z, z, z.to(torch.int32), z, 3)
    assert [tuple(o.shape) for o in out] == [(0, 3), (0, 3), (0,), (0,), (0,), (0,), (0, 3), (0,), (0,)]
    assert [o.dtype for o in out] == [torch.int32, torch.int32] + [torch.int64] * 3 + [torch.bool] + [torch.int64] * 3
    a_ids, c_slots = dir_ext().elara_dir_b(g.st, list(sim.pv), z, z, z, z, 3)
    assert a_ids.numel() == 0 and c_slots.numel() == 0
    torch.cuda.synchronize()
    assert not diff_states(before, comparable_state(g.view(), sim))
    with pytest.raises(RuntimeError):
        dir_ext().elara_dir_a(g.st[:16], list(sim.pv), z, z, z.to(torch.int32), z, 3)


@pytest.mark.gpu
def test_gpu_facade_release_pushes_parts_in_the_order_given(dev):
    """Directory.release(parts) pushes the parts' entries in the order of the list (srm2/elara_kernels.py:199-209),
    whatever that order: with the compactions' part before the evictions' (the reverse of the planner's call), the
    free stack, the counters and the later allocations equal the oracle's pushes in that order."""
    import torch
    print('[gpu-test] facade release order', flush=True)
    sim = Sim(**CONFIGS['default'])
    st0 = sim.initial_state()
    o, f = OracleImpl(sim, st0, triton=True), FacadeImpl(sim, st0, dev)

    def o_b(a_rows, a_k, c_rows, c_cnt, s):
        a_ids, c_slots = O.dir_b(o.st, sim.pv, a_rows, a_k, c_rows, c_cnt, s, c_release=False)
        O.dir_b(o.st, sim.pv, [], [], [], [], s, rel=(np.concatenate([c_rows, o.rel[0]]),
                                                      np.concatenate([c_cnt, o.rel[1]])))
        return [a_ids, c_slots]

    def f_b(a_rows, a_k, c_rows, c_cnt, s):
        c_rows_t, c_cnt_t = f.t(c_rows, torch.int64), f.t(c_cnt, torch.int64)
        a_ids = f.dirk.appends(f.t(a_rows, torch.int64), f.t(a_k, torch.int64), int(s))
        c_slots = f.dirk.compact(c_rows_t, c_cnt_t)
        f.dirk.release([(c_rows_t, c_cnt_t), f.rel_ev])
        return [a_ids.cpu().numpy(), c_slots.cpu().numpy()]

    o.dir_b, f.dir_b = o_b, f_b
    released = 0
    for s in range(1, 41):
        sim.step(s, [o, f])
        d = diff_states(comparable_state(o.view(), sim), comparable_state(f.view(), sim))
        assert not d, (s, d)
        released += int(o.rel[1].sum())
        check_invariants(o.view(), sim)
    assert released > 0
