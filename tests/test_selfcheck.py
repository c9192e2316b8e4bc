"""Exhaustive GPU checks of the arithmetic shortcuts.  elr_selfcheck_div: for each divisor b of the
scalar table (1 - b1^t, 1 - b2^t) and a few others, RN_f32((double)a * RN_f64(1/b)) equals the correctly rounded
fp32 quotient a / b for all 2^32 bit patterns of a."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def divisors():
    out = set()
    for hp in [(1e-3, 0.9, 0.999, 1e-8), (1e-3, 0.95, 0.9999, 1e-8)]:
        for t in [1, 2, 3, 4, 5, 7, 10, 17, 50, 100, 150, 201, 1000, 5000, 17000]:
            sc = O.adam_scalars(*hp, t)
            out.update([float(sc[5]), float(sc[6])])
    rng = np.random.default_rng(0)
    out.update(float(x) for x in rng.uniform(1e-4, 1.0, 6).astype(np.float32))
    out.update([1.0, float(np.float32(1 - 2**-24)), float(np.float32(2**-20)), float(np.float32(3.0))])
    return sorted(out)


def test_gpu_division_by_reciprocal_is_exact_for_all_floats(dev):
    from elara_amd import _lib
    ds = divisors()
    print(f'[gpu-test] selfcheck division: {len(ds)} divisors x 2^32 dividends', flush=True)
    bad = torch.zeros(len(ds), dtype=torch.int64, device=dev)
    first = torch.full((len(ds),), -1, dtype=torch.int32, device=dev)
    for i, b in enumerate(ds):
        rc = _lib.lib().elr_selfcheck_div(float(b), _lib.ptr(bad[i:]), _lib.ptr(first[i:]), _lib.stream_of(bad))
        _lib.check(rc, 'elr_selfcheck_div')
    torch.cuda.synchronize()
    fails = [(b, int(n), int(f) & 0xFFFFFFFF) for b, n, f in zip(ds, bad.tolist(), first.tolist()) if n]
    assert not fails, fails


def test_gpu_sqrt_is_correctly_rounded_for_all_floats(dev):
    from elara_amd import _lib
    print('[gpu-test] selfcheck sqrt: 2^32 inputs', flush=True)
    bad = torch.zeros(1, dtype=torch.int64, device=dev)
    first = torch.full((1,), -1, dtype=torch.int32, device=dev)
    _lib.check(_lib.lib().elr_selfcheck_sqrt(_lib.ptr(bad), _lib.ptr(first), _lib.stream_of(bad)), 'elr_selfcheck_sqrt')
    torch.cuda.synchronize()
    assert int(bad) == 0, f'{int(bad)} mismatches, first at 0x{int(first) & 0xFFFFFFFF:08x}'
