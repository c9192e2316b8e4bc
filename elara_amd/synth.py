"""Synthetic inputs of the benchmark configurations (host numpy; callers copy what they need to HBM).

Common settings: Adam lr=1e-3, b1=0.9, b2=0.999, eps=1e-8; gradients N(0, sigma=1e-3) drawn in fp64 and rounded to
fp32; RNG numpy.random.default_rng(seed).
"""
import numpy as np

ADAM = (1e-3, 0.9, 0.999, 1e-8)


def bound_for(D):
    """fp32(1/sqrt(D)), the init bound of the configs."""
    return float(np.float32(1.0 / np.sqrt(D)))


def grads(rng, n, D, sigma=1e-3):
    return (rng.standard_normal((n, D)) * sigma).astype(np.float32)


class ReplayLog:
    """Config C2 shape: n rows, each with c ~ U{1..K} logged gradients at strictly increasing steps (gaps U{1..50}).

    rows int64 [n]; cnt int32 [n]; steps int32 [n,K] (0 for unused slots); offs int64 [n] (exclusive cumsum of cnt);
    logs fp32 [sum(cnt), D] (row i's entries contiguous at offs[i]); max_step = largest logged step.
    """

    def __init__(self, n=262_144, D=128, K=3, seed=0, rows=None, max_gap=50, cmin=1):
        rng = np.random.default_rng(seed)
        self.n, self.D, self.K = n, D, K
        self.rows = np.arange(n, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
        self.cnt = rng.integers(cmin, K + 1, n).astype(np.int32)
        st = np.cumsum(rng.integers(1, max_gap + 1, (n, K)), 1)
        st[np.arange(K)[None, :] >= self.cnt[:, None]] = 0
        self.steps = st.astype(np.int32)
        self.offs = (np.cumsum(self.cnt, dtype=np.int64) - self.cnt).astype(np.int64)
        self.logs = grads(rng, int(self.cnt.sum()), D)
        self.max_step = int(self.steps.max()) if n else 0

    def entries_of_step(self, t):
        """(row index i, log entry index) of every row whose log holds step t."""
        i, k = np.nonzero(self.steps == t)
        return i.astype(np.int64), (self.offs[i] + k).astype(np.int64)


def unique_rows(rng, R, n):
    """n distinct row ids from [0, R), uniform without replacement, unsorted."""
    return rng.choice(R, n, replace=False).astype(np.int64)


class ZipfFields:
    """Row ids of a batch of `fields` categorical fields with bounded Zipf(alpha) popularity (configs C3-C5).

    Field f has vocabulary vocab[f] and rows [offset[f], offset[f] + vocab[f]) of the table.  A rank k in
    [0, vocab) is drawn by inverting the CDF of the continuous power law x^-alpha on [1, vocab + 1) and flooring
    (a bounded Zipf up to discretisation); it is mapped to a row through a per-field bijection of [0, vocab),
    k -> (a_f * k + b_f) mod vocab with gcd(a_f, vocab) = 1, so every field has its own hot rows.  draw() returns
    int64 ids [batch * fields] in (sample, field) order: occurrence index = sample * fields + field.
    """

    def __init__(self, vocab, alpha, seed=0, offsets=None):
        import math
        self.vocab = np.asarray(vocab, dtype=np.int64)
        self.F = self.vocab.size
        self.alpha = float(alpha)
        self.offsets = (np.concatenate([[0], np.cumsum(self.vocab)[:-1]]) if offsets is None
                        else np.asarray(offsets, dtype=np.int64))
        rng = np.random.default_rng(seed)
        self.a = np.empty(self.F, np.int64)
        self.b = np.empty(self.F, np.int64)
        for f, V in enumerate(self.vocab.tolist()):
            while True:
                a = int(rng.integers(1, max(2, V)))
                if math.gcd(a, V) == 1:
                    break
            self.a[f], self.b[f] = a, int(rng.integers(0, V))

    def ranks(self, rng, batch):
        """[batch, F] ranks in [0, vocab_f)."""
        u = rng.random((batch, self.F))
        e = 1.0 - self.alpha
        top = (self.vocab.astype(np.float64) + 1.0) ** e - 1.0
        x = (1.0 + u * top[None, :]) ** (1.0 / e)
        return np.minimum(np.floor(x).astype(np.int64) - 1, self.vocab[None, :] - 1)

    def draw(self, rng, batch):
        k = self.ranks(rng, batch)
        # (a*k + b) mod V without int64 overflow for V < 2^31: a, k < V
        ids = (self.a[None, :].astype(object) * k.astype(object) + self.b[None, :]) % self.vocab[None, :] \
            if self.vocab.max() >= (1 << 31) else (self.a[None, :] * k + self.b[None, :]) % self.vocab[None, :]
        return (np.asarray(ids, dtype=np.int64) + self.offsets[None, :]).reshape(-1)


class C5Tables:
    """Config C5: `T` tables with vocabularies round(exp(U(ln lo, ln hi))), one Zipf(alpha) field per table
    (ZipfFields), rows of table t at toff[t] + [0, vocab_t)."""

    def __init__(self, T=26, lo=1e3, hi=4e7, alpha=1.1, seed=0):
        rng = np.random.default_rng(seed)
        self.vocab = np.round(np.exp(rng.uniform(np.log(lo), np.log(hi), T))).astype(np.int64)
        self.toff = np.concatenate([[0], np.cumsum(self.vocab)[:-1]]).astype(np.int64)
        self.R = int(self.vocab.sum())
        self.fields = ZipfFields(self.vocab, alpha, seed=seed + 1, offsets=self.toff)

    def batch(self, rng, B):
        return self.fields.draw(rng, B)

    def static_rows(self, rng, B, n_static, n_batches=20):
        """The n_static most frequent rows over n_batches profiling batches (ties: lower row first), sorted
        ascending -- the reference's static hot set (srm2/train.py:262-270) on synthetic data."""
        ids = np.concatenate([self.batch(rng, B) for _ in range(n_batches)])
        u, c = np.unique(ids, return_counts=True)
        top = np.lexsort((u, -c))[:n_static]
        return np.sort(u[top]).astype(np.int64)


def unique_zipf(rng, fields, n_unique, draw=1 << 20):
    """Config C4: draw ids from `fields` (one ZipfFields field) until n_unique distinct ids are collected; returns
    them in first-appearance order (int64 [n_unique])."""
    seen = np.empty(0, np.int64)
    while seen.size < n_unique:
        ids = fields.draw(rng, draw)
        allv = np.concatenate([seen, ids])
        _, first = np.unique(allv, return_index=True)
        first.sort()
        seen = allv[first]
    return seen[:n_unique]
