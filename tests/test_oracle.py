"""The CPU oracle, pinned against the reference (oracle/_ref build, Triton golden vectors) and closed forms.

CPU only.  Mirrors the reference's exactness scripts (tests/test_ops.py:10-24, tests/test_replay.py:16-33) as
asserting tests.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import ref

HP = (1e-3, 0.9, 0.999, 1e-8)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint8)


def eq(a, b):
    return a.shape == b.shape and np.array_equal(bits(np.asarray(a)), bits(np.asarray(b)))


needs_ref = pytest.mark.skipif(ref.cpu() is None, reason='oracle/_ref not built (needs /root/reference)')


# ---------------------------------------------------------------------------------------------- scalars
@needs_ref
@pytest.mark.parametrize('hp', [HP, (1e-2, 0.8, 0.99, 1e-6), (3e-4, 0.95, 0.9999, 1e-10)])
def test_scalars_match_reference(hp):
    r = ref.cpu()
    for t in list(range(0, 2000)) + [10**4, 123457]:
        a = np.array(r.adam_scalars(*hp, t), np.float32)
        assert eq(a, O.adam_scalars(*hp, t)), t


def test_scalars_closed_forms():
    s1 = O.adam_scalars(*HP, 1)
    assert s1[5] == np.float32(1 - 0.9) and s1[6] == np.float32(1 - 0.999)
    assert s1[0] == np.float32(1e-3) and s1[7] == np.float32(1e-8) and s1[2] == np.float32(0.1)
    assert np.all(O.scalar_table(*HP, 5)[0] == 0)


# ---------------------------------------------------------------------------------------------- Adam
@needs_ref
@pytest.mark.parametrize('nthreads', [1, 4, 16])
def test_cpu_adam_matches_reference(nthreads):
    """tests/test_ops.py:12-24 as an assertion: repeated rows across steps, grads at 3 magnitudes."""
    g0 = torch.Generator().manual_seed(0)
    R, D = 20_000, 128
    host = torch.randn(R, 3, D, generator=g0) * 0.05
    host[:, 1:] = 0
    mine = host.numpy().copy()
    for step in range(1, 7):
        rows = torch.randperm(R, generator=g0)[:3000]
        if step % 2:
            rows = rows.sort().values
        grad = torch.randn(len(rows), D, generator=g0) * (10.0 ** (step % 3 - 2))
        ref.cpu().cpu_adam(host, rows, grad, *HP, step, nthreads)
        O.cpu_adam(mine, rows.numpy(), grad.numpy(), O.adam_scalars(*HP, step), nthreads)
    assert eq(host.numpy(), mine)


def test_cpu_adam_matches_triton_golden(golden):
    for ci in range(4):
        st = golden[f'adam{ci}_state'].copy()
        O.cpu_adam(st, golden[f'adam{ci}_slots'], golden[f'adam{ci}_grad'], golden[f'adam{ci}_scalars'])
        assert eq(st, golden[f'adam{ci}_out']), ci


def test_cpu_adam_invariants():
    rng = np.random.default_rng(1)
    R, D = 100, 16
    st = np.zeros((R, 3, D), np.float32)
    st[:, 0] = rng.standard_normal((R, D)).astype(np.float32)
    before = st.copy()
    rows = np.array([3, 50, 7], np.int64)
    g = rng.standard_normal((3, D)).astype(np.float32)
    sc = O.adam_scalars(*HP, 1)
    O.cpu_adam(st, rows, g, sc)
    untouched = np.setdiff1d(np.arange(R), rows)
    assert eq(st[untouched], before[untouched])
    assert eq(st[rows, 1], (sc[2] * g).astype(np.float32))
    assert eq(st[rows, 2], ((sc[4] * g).astype(np.float32) * g).astype(np.float32))
    # order of rows within a call does not matter
    st2 = before.copy()
    O.cpu_adam(st2, rows[::-1].copy(), g[::-1].copy(), sc)
    assert eq(st, st2)


# ---------------------------------------------------------------------------------------------- hash / init
def test_fmix32_published_vectors():
    # MurmurHash3_x86_32 of the empty key is fmix32(seed ^ 0): published values of the reference implementation
    assert O.fmix32(0) == 0
    assert O.fmix32(1) == 0x514E28B7
    assert O.fmix32(0xFFFFFFFF) == 0x81F16F39


def _unfmix32(h):
    def unxorshift(x, s):
        y = x
        for _ in range(32 // s + 1):
            y = x ^ (y >> s)
        return y & 0xFFFFFFFF
    h = unxorshift(h, 16)
    h = (h * pow(0xC2B2AE35, -1, 2**32)) & 0xFFFFFFFF
    h = unxorshift(h, 13)
    h = (h * pow(0x85EBCA6B, -1, 2**32)) & 0xFFFFFFFF
    return unxorshift(h, 16)


def test_fmix32_bijective():
    rng = np.random.default_rng(2)
    for x in [0, 1, 2**31, 2**32 - 1] + [int(v) for v in rng.integers(0, 2**32, 200)]:
        assert _unfmix32(O.fmix32(x)) == x


def test_init_matches_triton_golden(golden):
    for ci in range(5):
        D, seed = golden[f'init{ci}_meta']
        out = O.init_rows(golden[f'init{ci}_rows'], int(D), int(seed), float(golden[f'init{ci}_bound'][0]))
        assert eq(out, golden[f'init{ci}_out']), ci


def test_init_properties():
    D, bound = 128, np.float32(0.01)
    rows = np.array([0, 1, 5, 2**32 // D, 2**32 + 3], np.int64)
    a = O.init_rows(rows, D, 0, bound)
    assert a[0, 0, 0] == -bound                         # fmix32(0) = 0 -> u = 0 -> w0 = -bound
    assert np.all(a[:, 1:] == 0)
    assert np.all(a[:, 0] >= -bound) and np.all(a[:, 0] < bound)
    # u32(r*D + j) wraps: rows r and r + 2^32/D share the low key; the high word (r >> 32) is equal for both
    # while both are < 2^32, so they collide exactly; crossing 2^32 changes the high word and the values
    b = O.init_rows(np.array([0, 2**32 // D, 2**32], np.int64), D, 7, bound)
    assert eq(b[0], b[1]) and not eq(b[0], b[2])
    # permutation invariance (tests/test_replay.py:17-18)
    perm = np.random.default_rng(3).permutation(rows.size)
    assert eq(O.init_rows(rows[perm], D, 0, bound), a[perm])
    # distribution: uniform on [-bound, bound)
    big = O.init_rows(np.arange(2000, dtype=np.int64), D, 42, np.float32(1.0))[:, 0].ravel()
    assert abs(big.mean()) < 0.01 and abs(big.var() - 1 / 3) < 0.01


# ---------------------------------------------------------------------------------------------- replay
def test_replay_matches_triton_golden(golden):
    for ci in range(2):
        D, K, seed = (int(x) for x in golden[f'replay{ci}_meta'])
        out = O.replay_rows(golden[f'replay{ci}_rows'], golden[f'replay{ci}_logs'], golden[f'replay{ci}_offs'],
                            golden[f'replay{ci}_steps'], golden[f'replay{ci}_cnt'], D, K, seed,
                            float(golden[f'replay{ci}_bound'][0]), golden[f'replay{ci}_table'])
        assert eq(out, golden[f'replay{ci}_out']), ci


@needs_ref
def test_replay_equals_eager_reference_adam():
    """tests/test_replay.py:19-33: replay(init, log) == init followed by eager cpu_adam at the logged steps."""
    rng = np.random.default_rng(4)
    D, K, seed, bound = 128, 3, 1234, 0.01
    rows = np.unique(rng.integers(0, 2**33, 1500)).astype(np.int64)
    n = rows.size
    st = np.stack([rng.integers(1, 400, n), rng.integers(400, 800, n), rng.integers(800, 1200, n)], 1).astype(np.int32)
    g = (rng.standard_normal((n, K, D)) * 1e-2).astype(np.float32)
    cnt = rng.integers(0, K + 1, n).astype(np.int32)
    table = O.scalar_table(*HP, 1300)
    eager = torch.from_numpy(O.init_rows(rows, D, seed, bound))
    for k in range(K):
        sel = np.nonzero(cnt > k)[0]
        for s_val in np.unique(st[sel, k]):
            idx = sel[st[sel, k] == s_val]
            ref.cpu().cpu_adam(eager, torch.from_numpy(idx.astype(np.int64)), torch.from_numpy(g[idx, k].copy()), *HP,
                               int(s_val), 4)
    rp = O.replay_rows(rows, g.reshape(-1, D), np.arange(n) * K, st, cnt, D, K, seed, bound, table, nthreads=4)
    assert eq(rp, eager.numpy())


# ---------------------------------------------------------------------------------------------- segment sum
def test_segment_sum_order_and_values():
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 50, 600).astype(np.int64)
    g = rng.standard_normal((600, 8)).astype(np.float32)
    u, s, inv = O.segment_sum(ids, g)
    assert np.array_equal(u, np.unique(ids))
    assert np.array_equal(u[inv], ids)
    tu, tinv = torch.unique(torch.from_numpy(ids), return_inverse=True)
    assert np.array_equal(tu.numpy(), u) and np.array_equal(tinv.numpy(), inv)
    # 600 indices: ATen's windowed path.  Per id, its occurrences grouped by window (index // 16), each group
    # summed left to right, the group sums added to zero -- the per-id form the HIP kernels use, against the
    # oracle's window-by-window form.
    for q, i in enumerate(u):
        occ = np.nonzero(ids == i)[0]
        tot = np.zeros(8, np.float32)
        for w in np.unique(occ // 16):
            grp = occ[occ // 16 == w]
            acc = g[grp[0]].copy()
            for o in grp[1:]:
                acc = (acc + g[o]).astype(np.float32)
            tot = (tot + acc).astype(np.float32)
        assert eq(s[q], tot)
