"""Row copies (elara_amd.rows: elr_copy_rows, elr_glog_put, elr_glog_take): the executor's gathers and scatters, the
gradient-log appends (srm2/elara.py:569-570) and the resident-history record and take (elara.py:396, 501, 507,
524).  Pure data movement, so the check is bitwise against plain indexing on the CPU, with the items the kernels
must skip (indices out of range) left out of the expected result.  Widths cover the item-tile kernel (16-byte
rows of up to 1,536 floats) and the one-row-per-wave fallback (other widths); sizes cover the tile lengths
(8, 16 and 32 items per wave)."""
import numpy as np
import pytest
import torch

from elara_amd.rows import copy_rows, glog_put, glog_take

WIDTHS = [128, 384, 1536, 100, 2048]
SIZES = [1, 7, 1000, 70_000, 300_000]


def _case(n, W, seed):
    """A destination with rows to be overwritten, a source, and index lists with a few items out of range."""
    rng = np.random.default_rng(seed)
    nd, ns = n + 50, n + 30
    dst = rng.random((nd, W), dtype=np.float32)
    src = rng.random((ns, W), dtype=np.float32)
    di = rng.permutation(nd)[:n].astype(np.int64)      # distinct destinations (duplicates race by contract)
    si = rng.integers(0, ns, n).astype(np.int64)
    bad = rng.random(n) < 0.02
    di[bad & (rng.random(n) < 0.5)] = -1
    di[bad & (di >= 0)] = nd + 5
    si[rng.random(n) < 0.01] = ns
    return dst, src, di, si


@pytest.mark.gpu
@pytest.mark.parametrize('n,W', [(n, W) for n in SIZES for W in WIDTHS if n * W <= 150_000_000])   # under 0.6 GB
def test_gpu_copy_rows_matches_indexing(dev, n, W):
    print(f'[gpu-test] copy_rows n={n} W={W}', flush=True)
    dst, src, di, si = _case(n, W, seed=n + W)
    want = dst.copy()
    ok = (di >= 0) & (di < dst.shape[0]) & (si >= 0) & (si < src.shape[0])
    want[di[ok]] = src[si[ok]]
    g = torch.from_numpy(dst).to(dev)
    copy_rows(g, torch.from_numpy(di).to(dev), torch.from_numpy(src).to(dev), torch.from_numpy(si).to(dev))
    assert np.array_equal(g.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize('W', [128, 384, 100])
def test_gpu_copy_rows_identity_source(dev, W):
    """src_idx None: item i reads source row i (the log appends, logs[ids] = g)."""
    n = 5000
    dst, src, di, _ = _case(n, W, seed=7)
    want = dst.copy()
    ok = (di >= 0) & (di < dst.shape[0])
    want[di[ok]] = src[:n][ok]
    g = torch.from_numpy(dst).to(dev)
    copy_rows(g, torch.from_numpy(di).to(dev), torch.from_numpy(src).to(dev))
    assert np.array_equal(g.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize('with_j', [True, False])
@pytest.mark.parametrize('n', [9, 20_000])
def test_gpu_glog_put_matches_index_put(dev, n, with_j):
    """glog.index_put_((dyn - off, j), g) with j None meaning entry 0; items whose slot or entry is out of range
    are skipped."""
    rng = np.random.default_rng(n)
    nd, K, W, off = n + 40, 3, 128, 11
    glog = rng.standard_normal((nd, K, W)).astype(np.float32)
    g = rng.standard_normal((n, W)).astype(np.float32)
    dyn = (rng.permutation(nd)[:n] + off).astype(np.int64)   # distinct slots
    dyn[:3] = [off - 1, nd + off, nd + off + 7]               # out of range after the offset
    j = rng.integers(0, K, n).astype(np.int64)
    j[3:5] = [K, -1]
    want = glog.copy()
    jj = j if with_j else np.zeros(n, np.int64)
    slot = dyn - off
    ok = (slot >= 0) & (slot < nd) & (jj >= 0) & (jj < K)
    want[slot[ok], jj[ok]] = g[ok]
    t = torch.from_numpy(glog).to(dev)
    glog_put(t, torch.from_numpy(dyn).to(dev), torch.from_numpy(j).to(dev) if with_j else None,
             torch.from_numpy(g).to(dev), off)
    assert np.array_equal(t.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize('n', [5, 30_000])
def test_gpu_glog_take_matches_gather(dev, n):
    """logs[ids[r*K + k]] = glog[clamp(dyn[r], 0, nd-1), k]; ids out of range (-1: none) are skipped."""
    rng = np.random.default_rng(n + 1)
    nd, K, W = 500, 3, 128
    nl = n * K + 100
    glog = rng.standard_normal((nd, K, W)).astype(np.float32)
    logs = rng.standard_normal((nl, W)).astype(np.float32)
    dyn = rng.integers(-3, nd + 3, n).astype(np.int64)
    ids = rng.permutation(nl)[:n * K].astype(np.int64)
    ids[rng.random(n * K) < 0.3] = -1
    ids[:2] = [nl, nl + 9]
    want = logs.copy()
    src = glog[np.clip(dyn, 0, nd - 1)].reshape(n * K, W)
    ok = (ids >= 0) & (ids < nl)
    want[ids[ok]] = src[ok]
    t = torch.from_numpy(logs).to(dev)
    glog_take(t, torch.from_numpy(ids).to(dev), torch.from_numpy(glog).to(dev), torch.from_numpy(dyn).to(dev))
    assert np.array_equal(t.cpu().numpy().view(np.uint32), want.view(np.uint32))
