"""elr_adam_dedup_noalloc: duplicate-id row-sparse Adam whose scratch is the library's own per-GPU device array.

No counterpart in the reference: it is elr_adam_dedup (dedup + segment sum in ATen's order + Adam on the unique
rows; srm2/train.py:352, 429 followed by srm2/ops.py:59-67) for callers that cannot allocate device memory.  Both
entry points are called through the C-ABI and must give the same bits on two calls in a row, the second one
smaller (the array keeps the first call's contents).
"""
import ctypes

import numpy as np
import pytest
import torch

from elara_amd import _lib, synth

HP = synth.ADAM
MAX_BYTES = 64 << 20   # ELR_NOALLOC_SCRATCH_BYTES


def _scalars(step):
    sc = (ctypes.c_float * 8)()
    _lib.lib().elr_adam_scalars(*HP, step, sc)
    return sc


def _zipf_ids(rng, R, n, alpha=1.05):
    z = synth.ZipfFields([R], alpha, seed=int(rng.integers(1 << 30)), offsets=[0])
    return z.draw(rng, n)


def _call_alloc(state, ids, g, step):
    L = _lib.lib()
    n, D = g.shape
    nb = int(L.elr_dedup_scratch_bytes(n, D))
    scratch = torch.empty(max(nb, 8), dtype=torch.uint8, device=state.device)
    rc = L.elr_adam_dedup(_lib.ptr(state), state.shape[0], _lib.ptr(ids), _lib.ptr(g), n, D, _scalars(step),
                          _lib.ptr(scratch), nb, _lib.stream_of(state))
    _lib.check(rc, 'elr_adam_dedup')
    return scratch


def _call_noalloc(state, ids, g, step):
    L = _lib.lib()
    n, D = g.shape
    rc = L.elr_adam_dedup_noalloc(_lib.ptr(state), state.shape[0], _lib.ptr(ids), _lib.ptr(g), n, D,
                                  _scalars(step), _lib.stream_of(state))
    _lib.check(rc, 'elr_adam_dedup_noalloc')


def test_noalloc_capacity_limit_on_host():
    """The size limit is checked on the host, before any launch: a batch whose scratch would exceed the array
    returns ELR_ECAPACITY (-3); so do the usual argument checks (no GPU touched, so this runs on the CPU)."""
    L = _lib.lib()
    D = 128
    n_max = 1
    while L.elr_dedup_scratch_bytes(2 * n_max, D) <= MAX_BYTES:
        n_max *= 2
    lo, hi = n_max, 2 * n_max   # largest n that fits, by bisection on the byte count
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if L.elr_dedup_scratch_bytes(mid, D) <= MAX_BYTES:
            lo = mid
        else:
            hi = mid
    assert 500_000 < lo < 700_000   # covers a C5 batch (16,384 x 26 = 425,984 occurrences) at D = 128
    fake = ctypes.c_void_p(256)    # never dereferenced: the calls below return before any launch
    assert L.elr_adam_dedup_noalloc(fake, 10, fake, fake, hi, D, _scalars(1), None) == -3
    assert L.elr_adam_dedup_noalloc(fake, 10, fake, fake, 16, 513, _scalars(1), None) == -2
    assert L.elr_adam_dedup_noalloc(None, 10, fake, fake, 16, D, _scalars(1), None) == -1
    assert L.elr_adam_dedup_noalloc(fake, 10, fake, fake, 0, D, _scalars(1), None) == 0


@pytest.mark.gpu
@pytest.mark.parametrize('D', [128, 64])
def test_noalloc_equals_allocating_entry_point(dev, D):
    """Two calls in a row on the same GPU (a large Zipf batch over the hot-id and sort paths, then a smaller one
    that leaves most of the array holding the first call's data), each bitwise equal to elr_adam_dedup with a
    scratch buffer of its own.  The whole state table is compared, so rows outside the batch must be untouched."""
    rng = np.random.default_rng(11 + D)
    R = 400_000
    base = (torch.randn(R, 3, D, generator=torch.Generator().manual_seed(D)) * 0.05)
    base[:, 1:] = 0
    a = base.to(dev)
    b = base.to(dev)
    for call, n in enumerate((300_000, 2_500)):
        ids_np = _zipf_ids(rng, R, n)
        print(f'noalloc D={D} call={call} n={n} unique={np.unique(ids_np).size}', flush=True)
        ids = torch.from_numpy(ids_np).to(dev)
        g = torch.from_numpy(synth.grads(rng, n, D)).to(dev)
        keep = _call_alloc(a, ids, g, call + 1)
        _call_noalloc(b, ids, g, call + 1)
        torch.cuda.synchronize()
        del keep
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f'call {call}: results differ'
        assert not torch.equal(a.view(torch.int32), base.to(dev).view(torch.int32))
