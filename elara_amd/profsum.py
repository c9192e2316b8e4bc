"""Summaries of rocprofv3 result databases (rocpd SQLite, the default output of rocprofv3 in ROCm 7.x).

Counterpart of the reference's torch.profiler summary (srm2/profsum.py:10-25), for rocprofv3 runs:

    python -m elara_amd.profsum stats  <run>_results.db            per-kernel calls / total / mean / share
    python -m elara_amd.profsum stats --last N <run>_results.db    the same over each kernel's last N dispatches
                                                                   (the timed steps of a run whose untimed
                                                                   warm-up came first), with min and median
    python -m elara_amd.profsum steps --marker SUBSTR --last N <run>_results.db
                                                                   per-step kernel time of the last N steps: the
                                                                   window starts at the N-th last dispatch of the
                                                                   marker kernel (one launch per step); for each
                                                                   kernel, launches and microseconds per step
    python -m elara_amd.profsum pmc    <run>_results.db            per-kernel mean of each PMC counter per dispatch
    python -m elara_amd.profsum traffic --kernel SUBSTR \
        --fetch F.db --write W.db --copy-fetch CF.db --copy-write CW.db --copy-bytes N
                                                                   HBM bytes per launch of one kernel, with
                                                                   FETCH_SIZE / WRITE_SIZE (KiB per dispatch)
                                                                   scaled by what the same counters read for a
                                                                   plain copy kernel of N bytes read and written

Only the standard library is used, so the summaries can be made on any host from the .db files.
"""
import argparse
import sqlite3
import sys


def _rows(db, sql):
    con = sqlite3.connect(db)
    try:
        return con.execute(sql).fetchall()
    finally:
        con.close()


def kernel_stats(db):
    """[(name, calls, total_us, mean_us, pct)] from the top_kernels view (durations in microseconds)."""
    return [(n, int(c), float(t), float(a), float(p))
            for n, c, t, a, p in _rows(db, 'select name, total_calls, total_duration, average, percentage '
                                           'from top_kernels order by total_duration desc')]


def kernel_stats_last(db, last):
    """[(name, calls, total_us, mean_us, pct, min_us, median_us)] over each kernel's last `last` dispatches."""
    per = {}
    for n, d in _rows(db, 'select name, duration from kernels order by start'):
        per.setdefault(n, []).append(float(d) / 1e3)
    out = []
    for n, ds in per.items():
        ds = ds[-last:]
        srt = sorted(ds)
        out.append((n, len(ds), sum(ds), sum(ds) / len(ds), 0.0, srt[0], srt[len(srt) // 2]))
    tot = sum(r[2] for r in out) or 1.0
    out = [r[:4] + (100.0 * r[2] / tot,) + r[5:] for r in out]
    return sorted(out, key=lambda r: -r[2])


def step_window(db, marker, last):
    """(total_us_per_step, launches_per_step, [(name, launches_per_step, us_per_step)]) over the last `last` steps,
    a step starting at each dispatch of the kernel whose name contains `marker`."""
    rows = _rows(db, 'select name, start, end from kernels order by start')
    starts = [st for n, st, _ in rows if marker in n]
    if len(starts) < last:
        raise SystemExit(f'{marker!r}: {len(starts)} dispatches, fewer than {last}')
    t0 = starts[-last]
    agg = {}
    for n, st, en in rows:
        if st >= t0:
            a = agg.setdefault(n, [0, 0.0])
            a[0] += 1
            a[1] += (en - st) / 1e3
    per = sorted(((n, c / last, t / last) for n, (c, t) in agg.items()), key=lambda r: -r[2])
    return sum(r[2] for r in per), sum(r[1] for r in per), per


def pmc_means(db):
    """{(kernel name, counter): (dispatches, mean value per dispatch)}."""
    out = {}
    for n, cn, cnt, avg in _rows(db, 'select name, counter_name, count(*), avg(counter_value) from pmc_events '
                                     'group by name, counter_name'):
        out[(n, cn)] = (int(cnt), float(avg))
    return out


def _pick(means, counter, substr):
    hits = [(k, v) for k, v in means.items() if k[1] == counter and substr in k[0]]
    if len(hits) != 1:
        raise SystemExit(f'{counter}: expected one kernel matching {substr!r}, found {[k[0] for k, _ in hits]}')
    return hits[0][1][1]


def short(name, width=72):
    return name if len(name) <= width else name[:width - 3] + '...'


def cmd_stats(a):
    if a.last:
        print(f'| kernel | calls | total us | mean us | % | min us | median us |\n|---|---:|---:|---:|---:|---:|---:|')
        for n, c, t, m, p, lo, md in kernel_stats_last(a.db, a.last):
            print(f'| `{short(n)}` | {c} | {t:.1f} | {m:.2f} | {p:.1f} | {lo:.2f} | {md:.2f} |')
        return
    print(f'| kernel | calls | total us | mean us | % |\n|---|---:|---:|---:|---:|')
    for n, c, t, m, p in kernel_stats(a.db):
        print(f'| `{short(n)}` | {c} | {t:.1f} | {m:.2f} | {p:.1f} |')


def cmd_steps(a):
    tot, launches, per = step_window(a.db, a.marker, a.last)
    print(f'{a.last} steps: {tot:.1f} us of kernel time and {launches:.1f} launches per step\n')
    print('| kernel | launches per step | us per step | % |\n|---|---:|---:|---:|')
    for n, c, t in per:
        print(f'| `{short(n)}` | {c:.2f} | {t:.2f} | {100 * t / tot:.1f} |')


def cmd_pmc(a):
    print('| kernel | counter | dispatches | mean per dispatch |\n|---|---|---:|---:|')
    for (n, cn), (cnt, avg) in sorted(pmc_means(a.db).items()):
        print(f'| `{short(n)}` | {cn} | {cnt} | {avg:.2f} |')


def cmd_traffic(a):
    f_kib = _pick(pmc_means(a.fetch), 'FETCH_SIZE', a.kernel)
    w_kib = _pick(pmc_means(a.write), 'WRITE_SIZE', a.kernel)
    cf_kib = _pick(pmc_means(a.copy_fetch), 'FETCH_SIZE', a.copy_kernel)
    cw_kib = _pick(pmc_means(a.copy_write), 'WRITE_SIZE', a.copy_kernel)
    f_scale = a.copy_bytes / (cf_kib * 1024.0)
    w_scale = a.copy_bytes / (cw_kib * 1024.0)
    rd = f_kib * 1024.0 * f_scale
    wr = w_kib * 1024.0 * w_scale
    print(f'kernel: {a.kernel}')
    from elara_amd.build import source_hash
    print(f'source_hash = {source_hash()}')
    print(f'FETCH_SIZE_KiB_per_dispatch = {f_kib:.2f}')
    print(f'WRITE_SIZE_KiB_per_dispatch = {w_kib:.2f}')
    print(f'copy_bytes = {a.copy_bytes}')
    print(f'copy_FETCH_SIZE_KiB = {cf_kib:.2f}   fetch_scale = {f_scale:.4f}')
    print(f'copy_WRITE_SIZE_KiB = {cw_kib:.2f}   write_scale = {w_scale:.4f}')
    print(f'read_bytes_per_launch = {rd:.0f}')
    print(f'write_bytes_per_launch = {wr:.0f}')
    print(f'bytes_per_launch = {rd + wr:.0f}')


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest='cmd', required=True)
    s = sub.add_parser('stats'); s.add_argument('db'); s.add_argument('--last', type=int, default=0)
    s.set_defaults(fn=cmd_stats)
    w = sub.add_parser('steps'); w.add_argument('db'); w.add_argument('--marker', required=True)
    w.add_argument('--last', type=int, required=True); w.set_defaults(fn=cmd_steps)
    p = sub.add_parser('pmc'); p.add_argument('db'); p.set_defaults(fn=cmd_pmc)
    t = sub.add_parser('traffic')
    t.add_argument('--kernel', required=True)
    t.add_argument('--fetch', required=True)
    t.add_argument('--write', required=True)
    t.add_argument('--copy-fetch', required=True)
    t.add_argument('--copy-write', required=True)
    t.add_argument('--copy-kernel', default='copyBuffer')
    t.add_argument('--copy-bytes', type=int, default=1 << 30)
    t.set_defaults(fn=cmd_traffic)
    a = ap.parse_args(argv)
    a.fn(a)


if __name__ == '__main__':
    sys.exit(main())
