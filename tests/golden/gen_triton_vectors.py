"""Golden vectors of the reference's Triton kernels, computed by Triton's CPU interpreter.

Run only in the build container (it imports srm2 from /root/reference, read-only; the GPU box has no reference):
    python tests/golden/gen_triton_vectors.py
It writes tests/golden/triton_vectors.npz with inputs and outputs of
  - srm2/gpu_ops.py:26-38  _init_rows   (counter-hash init; ids include values >= 2^32 and several seeds/D)
  - srm2/gpu_ops.py:51-79  _replay      (init + K logged Adam steps)
  - srm2/ops.py:42-56      _adam_rows   (row-sparse Adam)
The Adam scalars handed to the kernels come from our own fp64->fp32 restatement (the reference's `ext()` loader
is not invoked: it would run the reference's JIT build), and the scalar table is passed in the form the kernel
reads (`table.t`).  Only the reference's jit functions are executed; nothing else of srm2 runs.
"""
import os
import sys
from pathlib import Path

os.environ['TRITON_INTERPRET'] = '1'
import numpy as np
import torch

REF = Path(os.environ.get('ELARA_REFERENCE', '/root/reference'))
OUT = Path(__file__).resolve().parent / 'triton_vectors.npz'
sys.path.insert(0, str(REF))
from srm2 import gpu_ops as ref_gpu_ops  # noqa: E402
from srm2 import ops as ref_ops  # noqa: E402


def scalars(lr, b1, b2, eps, t):
    return [np.float32(lr), np.float32(b1), np.float32(1.0 - b1), np.float32(b2), np.float32(1.0 - b2),
            np.float32(1.0 - b1 ** t), np.float32(1.0 - b2 ** t), np.float32(eps)]


def next_pow2(x):
    return 1 << (int(x) - 1).bit_length()


def run_init(rows, D, seed, bound):
    out = torch.empty(rows.numel(), 3, D)
    ref_gpu_ops._init_rows[(rows.numel(),)](out, rows, seed, bound, D, BLOCK=next_pow2(D))
    return out


def main():
    rng = np.random.default_rng(20261201)
    vec = {}
    # ---- init: several (D, seed, bound) cases; rows cover small ids, ids near 2^32 / D wrap, and ids >= 2^32
    cases = [(128, 0, float(np.float32(1 / np.sqrt(128)))), (64, 1234, 0.01), (256, 42, 0.125), (24, 7, 0.5),
             (128, 2**31 + 5, 0.01)]
    for ci, (D, seed, bound) in enumerate(cases):
        rows = np.concatenate([np.arange(4), rng.integers(0, 30_000_000, 6),
                               [2**32 // D - 1, 2**32 // D, 2**32 // D + 1],
                               [2**32 - 1, 2**32, 2**32 + 1, 2**33 + 12345, 2**40 + 7, 2**62 + 3]]).astype(np.int64)
        out = run_init(torch.from_numpy(rows), D, seed, bound)
        vec[f'init{ci}_rows'] = rows
        vec[f'init{ci}_meta'] = np.array([D, seed], dtype=np.int64)
        vec[f'init{ci}_bound'] = np.array([bound], dtype=np.float64)
        vec[f'init{ci}_out'] = out.numpy()
    # ---- replay: D=128, K=3 (and a K=4 case), counts 0..K, steps in disjoint increasing ranges
    for ci, (D, K, seed, bound, n) in enumerate([(128, 3, 1234, 0.01, 40), (64, 4, 9, 0.05, 24)]):
        rows = rng.choice(2**34, n, replace=False).astype(np.int64)
        cnt = rng.integers(0, K + 1, n).astype(np.int32)
        steps = np.stack([rng.integers(1 + 100 * k, 100 * (k + 1), n) for k in range(K)], 1).astype(np.int32)
        logs = (rng.standard_normal((n * K, D)) * 1e-2).astype(np.float32)
        offs = (np.arange(n) * K).astype(np.int64)
        table = np.array([[0.0] * 8] + [scalars(1e-3, 0.9, 0.999, 1e-8, t) for t in range(1, 100 * K + 1)],
                         dtype=np.float32)
        out = torch.empty(n, 3, D)
        ref_gpu_ops._replay[(n,)](out, torch.from_numpy(rows), torch.from_numpy(logs), torch.from_numpy(offs),
                                  torch.from_numpy(steps), torch.from_numpy(cnt), seed, bound, torch.from_numpy(table),
                                  D, K, BLOCK=next_pow2(D))
        for k_, v_ in dict(rows=rows, cnt=cnt, steps=steps, logs=logs, offs=offs, table=table,
                           meta=np.array([D, K, seed], dtype=np.int64), bound=np.array([bound]),
                           out=out.numpy()).items():
            vec[f'replay{ci}_{k_}'] = v_
    # ---- adam: [C,3,D] state with nonzero m, v; grads at three magnitudes; steps 1, 2, 7, 1000
    for ci, (D, step, gs) in enumerate([(128, 1, 1e-2), (64, 2, 1.0), (128, 7, 1e-1), (32, 1000, 1e-3)]):
        C, n = 64, 40
        state = np.concatenate([rng.standard_normal((C, 1, D)) * 0.05, rng.standard_normal((C, 1, D)) * 1e-3,
                                np.abs(rng.standard_normal((C, 1, D))) * 1e-6], 1).astype(np.float32)
        slots = rng.choice(C, n, replace=False).astype(np.int64)
        grad = (rng.standard_normal((n, D)) * gs).astype(np.float32)
        s = scalars(1e-3, 0.9, 0.999, 1e-8, step)
        pool = torch.from_numpy(state.copy())
        ref_ops._adam_rows[(n,)](pool, torch.from_numpy(slots), torch.from_numpy(grad), D, *[float(x) for x in s],
                                 BLOCK=next_pow2(D))
        for k_, v_ in dict(state=state, slots=slots, grad=grad, scalars=np.array(s, dtype=np.float32),
                           out=pool.numpy()).items():
            vec[f'adam{ci}_{k_}'] = v_
    np.savez_compressed(OUT, **vec)
    print(f'wrote {OUT} ({OUT.stat().st_size} bytes, {len(vec)} arrays)')


if __name__ == '__main__':
    main()
