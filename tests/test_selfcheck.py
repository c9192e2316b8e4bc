"""Exhaustive GPU checks of the arithmetic shortcuts.  elr_selfcheck_div: for each divisor b of the
scalar table (1 - b1^t, 1 - b2^t) and a few others, RN_f32((double)a * RN_f64(1/b)) equals the correctly rounded
fp32 quotient a / b for all 2^32 bit patterns of a.  elr_selfcheck_sqrt: the square root over all 2^32 inputs.
elr_selfcheck_quot: the division core used for num / den equals the correctly rounded division over its range."""
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


def quot_denominators():
    """d values for the division-core check: both ends of its range [2^-48, 2^65), powers of two and their
    neighbours, typical Adam denominators sqrt(vh) + eps, and log-uniform random values."""
    f = np.float32
    out = {float(f(2.0 ** -48)), float(np.nextafter(f(2.0 ** -48), f(1))), float(np.nextafter(f(2.0 ** 65), f(0))),
           float(f(2.0 ** 64)), 1.0, float(np.nextafter(f(1), f(0))), float(np.nextafter(f(1), f(2))), 1.5, 3.0,
           float(f(1e-3) + f(1e-8)), float(f(3.1622776e-4) + f(1e-8)), float(f(1e-8)), float(f(2.0 ** -24) * 3)}
    rng = np.random.default_rng(1)
    out.update(float(x) for x in np.exp2(rng.uniform(-48, 65, 40)).astype(np.float32))
    return sorted(x for x in out if 2.0 ** -48 <= x < 2.0 ** 65)


def test_gpu_division_core_matches_division_in_its_range(dev):
    from elara_amd import _lib
    ds = quot_denominators()
    print(f'[gpu-test] selfcheck division core: {len(ds)} denominators x 2^32 numerators', flush=True)
    bad = torch.zeros(len(ds), dtype=torch.int64, device=dev)
    tested = torch.zeros(len(ds), dtype=torch.int64, device=dev)
    first = torch.full((len(ds),), -1, dtype=torch.int32, device=dev)
    for i, d in enumerate(ds):
        rc = _lib.lib().elr_selfcheck_quot(float(d), _lib.ptr(bad[i:]), _lib.ptr(tested[i:]), _lib.ptr(first[i:]),
                                           _lib.stream_of(bad))
        _lib.check(rc, 'elr_selfcheck_quot')
    torch.cuda.synchronize()
    fails = [(d, int(n), int(fb) & 0xFFFFFFFF) for d, n, fb in zip(ds, bad.tolist(), first.tolist()) if n]
    assert not fails, fails
    # every n with 2^-60 <= |n| < 2^40: 100 binades x 2^23 significands x 2 signs
    assert tested.tolist() == [100 * 2 ** 24] * len(ds)


def test_gpu_division_core_rejects_denominators_out_of_range(dev):
    from elara_amd import _lib
    bad = torch.zeros(2, dtype=torch.int64, device=dev)
    first = torch.full((1,), -1, dtype=torch.int32, device=dev)
    for d in [2.0 ** -49, float(np.nextafter(np.float32(2.0 ** -48), np.float32(0))), 2.0 ** 65, float('inf'), 0.0,
              -1.0, float('nan')]:
        rc = _lib.lib().elr_selfcheck_quot(d, _lib.ptr(bad), _lib.ptr(bad[1:]), _lib.ptr(first), _lib.stream_of(bad))
        assert rc == -1, (d, rc)  # ELR_EINVAL
    torch.cuda.synchronize()
    assert bad.tolist() == [0, 0]
