"""GPU parity of Adam, init and replay (through the C-ABI) against the CPU oracle and the reference's vectors.

Bar: bitwise fp32 equality.  Mirrors the reference's tests/test_ops.py:10-24 and tests/test_replay.py:16-33 with
assertions, plus the benchmark configs C1 (full size) and C2 (full size).
"""
import numpy as np
import pytest
import torch

from elara_amd import synth
from elara_amd.gpu_ops import ScalarTable, init_rows, replay_rows
from elara_amd.ops import adam_scalars, gpu_adam
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HP = synth.ADAM


def same(a, b):
    a = a.detach().cpu().contiguous() if torch.is_tensor(a) else torch.from_numpy(np.ascontiguousarray(a))
    b = b.detach().cpu().contiguous() if torch.is_tensor(b) else torch.from_numpy(np.ascontiguousarray(b))
    return a.shape == b.shape and torch.equal(a.view(torch.int32), b.view(torch.int32))


def step_banner(msg):
    print(f'[gpu-test] {msg}', flush=True)


# ------------------------------------------------------------------------------------------------ Adam
@pytest.mark.parametrize('D', [128, 256, 30])
def test_adam_dense_equals_identity_slots(dev, D):
    """elr_adam_rows without a slot list (row i of grad -> state row i) equals the call with slots 0..n-1."""
    from elara_amd.ops import adam_rows_dense
    step_banner(f'adam dense D={D}')
    g0 = torch.Generator().manual_seed(3)
    n = 9_001
    a = (torch.randn(n, 3, D, generator=g0) * 0.05).to(dev)
    b = a.clone()
    for step in (1, 2, 5):
        grad = (torch.randn(n, D, generator=g0) * 1e-3).to(dev)
        adam_rows_dense(a, grad, *HP, step)
        gpu_adam(b, torch.arange(n, device=dev), grad, *HP, step)
    torch.cuda.synchronize()
    assert same(a, b)


@pytest.mark.parametrize('D,idx', [(128, torch.int64), (128, torch.int32), (64, torch.int64), (64, torch.int32),
                                   (256, torch.int64), (512, torch.int32), (30, torch.int64), (100, torch.int64),
                                   (192, torch.int32)])
def test_adam_matches_oracle(dev, D, idx):
    """tests/test_ops.py:12-24: several steps with repeated rows across steps and grads at 3 magnitudes."""
    step_banner(f'adam D={D} idx={idx}')
    g0 = torch.Generator().manual_seed(0)
    R = 50_000
    host = torch.randn(R, 3, D, generator=g0) * 0.05
    host[:, 1:] = 0
    mine = host.numpy().copy()
    gpu = host.to(dev)
    for step in range(1, 7):
        rows = torch.randperm(R, generator=g0)[:7_000]
        if step % 2:
            rows = rows.sort().values
        grad = torch.randn(len(rows), D, generator=g0) * (10.0 ** (step % 3 - 2))
        O.cpu_adam(mine, rows.numpy(), grad.numpy(), O.adam_scalars(*HP, step), 8)
        gpu_adam(gpu, rows.to(dev, idx), grad.to(dev), *HP, step)
    torch.cuda.synchronize()
    assert same(gpu, mine)


def test_adam_matches_triton_golden(dev, golden):
    from elara_amd import _lib
    for ci in range(4):
        # every device buffer is held by a name until the launch has completed
        st = torch.from_numpy(golden[f'adam{ci}_state'].copy()).to(dev)
        slots = torch.from_numpy(golden[f'adam{ci}_slots']).to(dev)
        grad = torch.from_numpy(golden[f'adam{ci}_grad']).to(dev)
        s = golden[f'adam{ci}_scalars']
        rc = _lib.lib().elr_adam_rows(_lib.ptr(st), st.shape[0], _lib.ptr(slots), 1, _lib.ptr(grad), slots.numel(),
                                      st.shape[2], _lib.scalars8(s.tolist()), _lib.stream_of(st))
        assert rc == 0
        torch.cuda.synchronize()
        assert same(st, golden[f'adam{ci}_out']), ci


def test_adam_subnormals_and_extremes(dev):
    """Gradients whose squares underflow into fp32 subnormals, huge gradients, zero rows: IEEE behaviour equal to
    the x86 oracle (denormals kept, correctly rounded division and square root)."""
    rng = np.random.default_rng(9)
    D = 128
    mags = np.array([1e-30, 1e-23, 1e-20, 3e-19, 1e-10, 1.0, 1e10, 1e18, 0.0], dtype=np.float64)
    n = mags.size * 16
    state = np.zeros((n, 3, D), np.float32)
    state[:, 0] = rng.standard_normal((n, D))
    state[:, 1] = (rng.standard_normal((n, D)) * 1e-38).astype(np.float32)   # subnormal m
    state[:, 2] = np.abs(rng.standard_normal((n, D)) * 1e-39).astype(np.float32)
    g = (rng.standard_normal((n, D)) * np.repeat(mags, 16)[:, None]).astype(np.float32)
    rows = rng.permutation(n).astype(np.int64)
    gpu = torch.from_numpy(state).to(dev)
    for step in (1, 2, 50):
        O.cpu_adam(state, rows, g, O.adam_scalars(*HP, step), 1)
        gpu_adam(gpu, torch.from_numpy(rows).to(dev), torch.from_numpy(g).to(dev), *HP, step)
    torch.cuda.synchronize()
    assert same(gpu, state)


def test_adam_edge_cases(dev):
    pool = torch.randn(100, 3, 64, device=dev)
    ref = pool.clone()
    gpu_adam(pool, torch.empty(0, dtype=torch.int64, device=dev), torch.empty(0, 64, device=dev), *HP, 1)
    torch.cuda.synchronize()
    assert torch.equal(pool, ref)
    # an out-of-range slot is skipped by the kernel's index check (the reference leaves it undefined)
    gpu_adam(pool, torch.tensor([5, 100, 1 << 40], device=dev), torch.ones(3, 64, device=dev), *HP, 1)
    torch.cuda.synchronize()
    changed = (pool != ref).any(dim=2).any(dim=1).nonzero().flatten().tolist()
    assert changed == [5]
    with pytest.raises(RuntimeError):
        gpu_adam(pool, torch.tensor([1], device=dev), torch.ones(2, 64, device=dev), *HP, 1)


def test_c1_row_sparse_adam_full_size(dev):
    """Config C1: 1,048,576 x 64 table, 65,536 unique rows per step, t = 1..10, bitwise vs the oracle."""
    step_banner('C1 full size')
    R, D, n = 1 << 20, 64, 65_536
    rng = np.random.default_rng(0)
    ridx = np.arange(R, dtype=np.int64)
    host = O.init_rows(ridx, D, 0, synth.bound_for(D))
    gpu = init_rows(torch.from_numpy(ridx).to(dev), D, 0, synth.bound_for(D))
    torch.cuda.synchronize()
    assert same(gpu, host)
    for t in range(1, 11):
        rows = synth.unique_rows(rng, R, n)
        g = synth.grads(rng, n, D)
        O.cpu_adam(host, rows, g, O.adam_scalars(*HP, t), 8)
        gpu_adam(gpu, torch.from_numpy(rows).to(dev), torch.from_numpy(g).to(dev), *HP, t)
    torch.cuda.synchronize()
    assert same(gpu, host)


# ------------------------------------------------------------------------------------------------ init
def test_init_matches_golden_and_oracle(dev, golden):
    for ci in range(5):
        D, seed = (int(x) for x in golden[f'init{ci}_meta'])
        bound = float(golden[f'init{ci}_bound'][0])
        rows = torch.from_numpy(golden[f'init{ci}_rows']).to(dev)
        out = init_rows(rows, D, seed, bound)
        torch.cuda.synchronize()
        assert same(out, golden[f'init{ci}_out']), ci
    rng = np.random.default_rng(1)
    rows = np.concatenate([rng.integers(0, 2**40, 5000), rng.integers(0, 100, 50)]).astype(np.int64)
    for D in (64, 128, 256, 30):
        out = init_rows(torch.from_numpy(rows).to(dev), D, 42, 0.0625)
        torch.cuda.synchronize()
        assert same(out, O.init_rows(rows, D, 42, 0.0625)), D


def test_init_deterministic_under_permutation(dev):
    """tests/test_replay.py:16-18."""
    rows = torch.randint(0, 30_000_000, (5000,), dtype=torch.int64).unique().to(dev)
    a = init_rows(rows, 128, 1234, 0.01)
    perm = torch.randperm(rows.numel(), device=dev)
    b = init_rows(rows[perm], 128, 1234, 0.01)
    torch.cuda.synchronize()
    assert torch.equal(a[perm], b)


# ------------------------------------------------------------------------------------------------ replay
def test_replay_matches_golden(dev, golden):
    for ci in range(2):
        D, K, seed = (int(x) for x in golden[f'replay{ci}_meta'])
        g = {k: torch.from_numpy(golden[f'replay{ci}_{k}']).to(dev) for k in ('rows', 'logs', 'offs', 'steps', 'cnt',
                                                                               'table')}
        out = replay_rows(g['rows'], g['logs'], g['offs'], g['steps'], g['cnt'], D, K, seed,
                          float(golden[f'replay{ci}_bound'][0]), g['table'])
        torch.cuda.synchronize()
        assert same(out, golden[f'replay{ci}_out']), ci


@pytest.mark.parametrize('D,K', [(128, 3), (64, 4), (256, 3), (30, 2), (128, 1), (512, 3), (100, 8), (192, 5)])
def test_replay_equals_eager(dev, D, K):
    """tests/test_replay.py:19-33 as an assertion: replay == eager GPU Adam == oracle, bitwise; cnt in {0..K}."""
    step_banner(f'replay D={D} K={K}')
    seed, bound = 1234, 0.01
    rows = torch.randint(0, 2**34, (4000,), dtype=torch.int64).unique().to(dev)
    n = rows.numel()
    st = torch.stack([torch.randint(1 + 400 * k, 400 * (k + 1), (n,)) for k in range(K)], 1).to(torch.int32).to(dev)
    g = torch.randn(n, K, D, device=dev) * 1e-2
    cnt = torch.randint(0, K + 1, (n,), dtype=torch.int32, device=dev)
    table = ScalarTable(*HP, 400 * K + 100, dev)
    eg = init_rows(rows, D, seed, bound).contiguous()
    for k in range(K):
        sel = (cnt > k).nonzero().flatten()
        for s_val in st[sel, k].unique().tolist():
            idx = sel[st[sel, k] == s_val]
            gpu_adam(eg, idx, g[idx, k].contiguous(), *HP, s_val)
    offs = torch.arange(n, device=dev) * K
    rp = replay_rows(rows, g.reshape(-1, D).contiguous(), offs, st.contiguous(), cnt, D, K, seed, bound, table)
    torch.cuda.synchronize()
    assert torch.equal(rp.view(torch.int32), eg.view(torch.int32))
    ora = O.replay_rows(rows.cpu().numpy(), g.reshape(-1, D).cpu().numpy(), offs.cpu().numpy(), st.cpu().numpy(),
                        cnt.cpu().numpy(), D, K, seed, bound, table.t.cpu().numpy(), nthreads=8)
    assert same(rp, ora)


def test_c2_replay_full_size(dev):
    """Config C2: 262,144 rows x 128, k in {1,2,3}, gaps 1..50; replay == eager Adam step by step == oracle."""
    step_banner('C2 full size')
    w = synth.ReplayLog(n=262_144, D=128, K=3, seed=0)
    D, K, seed, bound = w.D, w.K, 0, synth.bound_for(128)
    d = {k: torch.from_numpy(getattr(w, k)).to(dev) for k in ('rows', 'logs', 'offs', 'steps', 'cnt')}
    table = ScalarTable(*HP, w.max_step, dev)
    rp = replay_rows(d['rows'], d['logs'], d['offs'], d['steps'], d['cnt'], D, K, seed, bound, table)
    eg = init_rows(d['rows'], D, seed, bound)
    for t in range(1, w.max_step + 1):
        i, e = w.entries_of_step(t)
        if i.size:
            gpu_adam(eg, torch.from_numpy(i).to(dev), d['logs'][torch.from_numpy(e).to(dev)], *HP, t)
    torch.cuda.synchronize()
    assert torch.equal(rp.view(torch.int32), eg.view(torch.int32))
    ora = O.replay_rows(w.rows, w.logs, w.offs, w.steps, w.cnt, D, K, seed, bound, table.t.cpu().numpy(), nthreads=16)
    assert same(rp, ora)


def test_replay_edge_cases(dev):
    table = ScalarTable(*HP, 10, dev)
    z = torch.empty(0, dtype=torch.int64, device=dev)
    out = replay_rows(z, torch.empty(0, 64, device=dev), z, torch.empty(0, 3, dtype=torch.int32, device=dev),
                      torch.empty(0, dtype=torch.int32, device=dev), 64, 3, 0, 0.1, table)
    assert out.shape == (0, 3, 64)
    # all counts zero with an empty log: replay == init
    rows = torch.arange(10, device=dev)
    out = replay_rows(rows, torch.empty(0, 64, device=dev), torch.zeros(10, dtype=torch.int64, device=dev),
                      torch.zeros(10, 3, dtype=torch.int32, device=dev), torch.zeros(10, dtype=torch.int32, device=dev),
                      64, 3, 5, 0.1, table)
    torch.cuda.synchronize()
    assert torch.equal(out, init_rows(rows, 64, 5, 0.1))
    with pytest.raises(RuntimeError):
        replay_rows(rows, torch.empty(0, 64, device=dev), torch.zeros(10, dtype=torch.int64, device=dev),
                    torch.zeros(10, 9, dtype=torch.int32, device=dev), torch.zeros(10, dtype=torch.int32, device=dev),
                    64, 9, 5, 0.1, table)
    assert adam_scalars(*HP, 3) == O.adam_scalars(*HP, 3).tolist()


def test_replay_without_reciprocal_table(dev):
    """elr_replay_rows with recip = NULL (a C caller without elr_scalar_recip): the kernels compute the
    reciprocals themselves; results are the same bits."""
    from elara_amd import _lib
    w = synth.ReplayLog(n=3000, D=128, K=3, seed=3, rows=np.arange(3000, dtype=np.int64) * 977 + 2**33)
    table = ScalarTable(*HP, w.max_step + 1, dev)
    d = {k: torch.from_numpy(np.ascontiguousarray(getattr(w, k))).to(dev) for k in ('rows', 'logs', 'offs', 'steps',
                                                                                      'cnt')}
    out = torch.empty(w.n, 3, 128, device=dev)
    rc = _lib.lib().elr_replay_rows(_lib.ptr(out), _lib.ptr(d['rows']), _lib.ptr(d['logs']), d['logs'].shape[0],
                                    _lib.ptr(d['offs']), _lib.ptr(d['steps']), _lib.ptr(d['cnt']), w.n, 128, 3, 11,
                                    0.05, _lib.ptr(table.t), None, table.t.shape[0], _lib.stream_of(out))
    _lib.check(rc, 'elr_replay_rows')
    torch.cuda.synchronize()
    ref = O.replay_rows(w.rows, w.logs, w.offs, w.steps, w.cnt, 128, 3, 11, 0.05, table.t.cpu().numpy())
    assert same(out, ref)


@pytest.mark.parametrize('D', [128, 64])
def test_replay_extreme_gradients(dev, D):
    """Logged gradients whose squares underflow into fp32 subnormals, zeros (incl. -0), and huge values: the
    replayed state is bitwise the oracle's."""
    rng = np.random.default_rng(21)
    n, K = 900, 3
    mags = np.array([0.0, 1e-38, 1e-30, 1e-23, 3e-19, 1e-10, 1.0, 1e10, 1e18], np.float64)
    cnt = np.full(n, K, np.int32)
    steps = np.tile(np.array([1, 2, 7], np.int32), (n, 1))
    logs = (rng.standard_normal((n * K, D)) * np.repeat(mags, n * K // mags.size)[:, None]).astype(np.float32)
    logs[::17] = -0.0
    rows = rng.integers(0, 2**40, n).astype(np.int64)
    offs = (np.arange(n) * K).astype(np.int64)
    table = ScalarTable(*HP, 10, dev)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    out = replay_rows(t(rows), t(logs), t(offs), t(steps), t(cnt), D, K, 5, 0.03, table)
    torch.cuda.synchronize()
    assert same(out, O.replay_rows(rows, logs, offs, steps, cnt, D, K, 5, 0.03, table.t.cpu().numpy()))


@pytest.mark.gpu
def test_timed_launches_record_kernel_events(dev):
    """elr_replay_rows_timed / elr_adam_rows_timed (gpu_ops.replay_rows / ops.gpu_adam with events): the same bits as
    the untimed calls, and the two events the launch records bracket the kernel (positive, plausible duration)."""
    import bench
    print('[gpu-test] timed launches', flush=True)
    w = synth.ReplayLog(n=4096, D=128, K=3, seed=9)
    table = ScalarTable(*HP, w.max_step + 2, dev)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    args = (t(w.rows), t(w.logs), t(w.offs), t(w.steps), t(w.cnt), 128, 3, 5, 0.03, table)
    a = replay_rows(*args)
    ev = [bench.HipEvent() for _ in range(4)]
    b = replay_rows(*args, events=(ev[0].h.value, ev[1].h.value))
    g = t(synth.grads(np.random.default_rng(2), w.n, 128))
    idx = torch.arange(w.n, device=dev)
    gpu_adam(a, idx, g, *HP, w.max_step + 1)
    gpu_adam(b, idx, g, *HP, w.max_step + 1, events=(ev[2].h.value, ev[3].h.value))
    torch.cuda.synchronize()
    assert same(a, b.cpu().numpy())
    for x, y in ((ev[0], ev[1]), (ev[2], ev[3])):
        ms = x.elapsed_time(y)
        assert 0.0 < ms < 50.0, ms
    for e in ev:
        e.destroy()


@pytest.mark.gpu
def test_gpu_adam_check_raises_on_rows_out_of_range(dev):
    """gpu_adam / adam_dedup skip a row outside [0, C) (undefined in the reference); with check=True they raise
    IndexError before any launch, and run as usual on valid rows."""
    from elara_amd.dedup import adam_dedup
    from elara_amd.ops import gpu_adam
    print('[gpu-test] adam check', flush=True)
    pool = torch.zeros(10, 3, 64, device=dev)
    g = torch.ones(3, 64, device=dev)
    for bad in ([0, 4, 10], [-1, 2, 3]):
        with pytest.raises(IndexError):
            gpu_adam(pool, torch.tensor(bad, device=dev), g, *synth.ADAM, 1, check=True)
        with pytest.raises(IndexError):
            adam_dedup(pool, torch.tensor(bad, device=dev), g, *synth.ADAM, 1, check=True)
    torch.cuda.synchronize()
    assert not pool.any()                                      # nothing was launched
    gpu_adam(pool, torch.tensor([0, 4, 9], device=dev), g, *synth.ADAM, 1, check=True)
    adam_dedup(pool, torch.tensor([1, 1, 2], device=dev), g, *synth.ADAM, 1, check=True)
    torch.cuda.synchronize()
    assert pool[[0, 4, 9, 1, 2], 0].ne(0).all() and not pool[[3, 5, 6, 7, 8]].any()
