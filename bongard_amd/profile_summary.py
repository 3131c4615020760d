"""Summaries of rocprofv3 result databases (kernel trace and PMC counters).

    python -m bongard_amd.profile_summary trace <results.db>
    python -m bongard_amd.profile_summary pmc <results.db>
    python -m bongard_amd.profile_summary steps <results.db> <first kernel> [skip]

``trace``: per-kernel call count and average / min / max duration (us) from the
kernel-dispatch records, and the average over the kernel's longest run of back-to-back
dispatches (no other kernel between them): a benchmark that times N launches of one
kernel between two events produces exactly such a run, so that figure is the one to set
beside the benchmark's own per-launch average. ``pmc``: per-kernel, per-counter average
value per dispatch. ``steps``: the dispatches cut into steps, each starting at a dispatch
whose name contains ``first kernel`` (the first ``skip`` steps dropped, default 2: clock
ramp), and per position in the step the kernel, its median and minimum duration (us); the
steps must all launch the same kernel sequence.
"""
import sqlite3, sys, re
W = 76  # kernel-name column: wide enough for the GEMM template arguments
def short(n):
    n = n.replace("(anonymous namespace)", "anon")
    depth = 0
    for i, ch in enumerate(n):
        if ch == '<': depth += 1
        elif ch == '>': depth -= 1
        elif ch == '(' and depth == 0:
            n = n[:i]; break
    n = n.replace("void ", "").replace("bf8::anon::", "")
    return n[:W]
def kernel_stats(path):
    db = sqlite3.connect(path); cur = db.cursor()
    rows = cur.execute("select name, start, end from kernels").fetchall()
    agg = {}
    for name, s, e in rows:
        d = (e - s) / 1e3
        a = agg.setdefault(short(name), [0, 0.0, 1e18, 0])
        a[0] += 1; a[1] += d; a[2] = min(a[2], d); a[3] = max(a[3], d)
    # longest run of consecutive dispatches of one kernel, in dispatch-start order
    runs, prev, cur = {}, None, []
    for name, s, e in sorted(rows, key=lambda r: r[1]) + [(None, 0, 0)]:
        k = short(name) if name is not None else None
        if k != prev and cur:
            if len(cur) > len(runs.get(prev, [])):
                runs[prev] = cur
            cur = []
        if k is not None:
            cur.append((e - s) / 1e3)
        prev = k
    tot = sum(v[1] for v in agg.values())
    out = [f"{'kernel':{W}s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'time%':>7s}"
           f" {'run':>4s} {'run_avg_us':>10s}"]
    for k, v in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        r = runs.get(k, [])
        out.append(f"{k:{W}s} {v[0]:6d} {v[1]/v[0]:9.2f} {v[2]:9.2f} {v[3]:9.2f} {100*v[1]/tot:7.2f}"
                   f" {len(r):4d} {sum(r) / max(len(r), 1):10.2f}")
    return "\n".join(out)
def pmc(path):
    db = sqlite3.connect(path); cur = db.cursor()
    rows = cur.execute("select kernel_name, counter_name, value, grid_size from counters_collection").fetchall()
    agg = {}
    for name, c, v, g in rows:
        a = agg.setdefault((short(name), c, g), [0, 0.0])
        a[0] += 1; a[1] += v
    return {k: v[1] / v[0] for k, v in agg.items()}
def step_table(path, first, skip=2):
    db = sqlite3.connect(path); cur = db.cursor()
    rows = sorted(cur.execute("select name, start, end from kernels").fetchall(), key=lambda r: r[1])
    steps = []
    for name, s, e in rows:
        if first in name:
            steps.append([])
        if steps:
            steps[-1].append((short(name), (e - s) / 1e3))
    steps = steps[skip:]
    if not steps or any([k for k, _ in st] != [k for k, _ in steps[0]] for st in steps):
        raise SystemExit("steps: no steps found, or the steps launch different kernel sequences")
    out = [f"{'kernel':{W}s} {'median_us':>10s} {'min_us':>9s}"]
    med_sum = min_sum = 0.0
    for i, (k, _) in enumerate(steps[0]):
        d = sorted(st[i][1] for st in steps)
        med = d[len(d) // 2] if len(d) % 2 else 0.5 * (d[len(d) // 2 - 1] + d[len(d) // 2])
        med_sum += med; min_sum += d[0]
        out.append(f"{k:{W}s} {med:10.2f} {d[0]:9.2f}")
    out.append(f"{'sum (' + str(len(steps)) + ' steps)':{W}s} {med_sum:10.2f} {min_sum:9.2f}")
    return "\n".join(out)
if __name__ == "__main__":
    if sys.argv[1] == "trace":
        print(kernel_stats(sys.argv[2]))
    elif sys.argv[1] == "steps":
        print(step_table(sys.argv[2], sys.argv[3], int(sys.argv[4]) if len(sys.argv) > 4 else 2))
    else:
        for k, v in sorted(pmc(sys.argv[2]).items()):
            print(f"{k[0]:{W}s} {k[1]:22s} grid={k[2]:<10d} {v:16.1f} per dispatch")
