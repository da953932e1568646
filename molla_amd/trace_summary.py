"""Per-kernel summary of a rocprofv3 kernel trace (the SQLite file that
`rocprofv3 --kernel-trace -d DIR -o NAME` writes as DIR/NAME_results.db).

    python -m molla_amd.trace_summary DB            # every kernel of the run
    python -m molla_amd.trace_summary DB --steps N  # the last N decode steps
    python -m molla_amd.trace_summary DB --first N  # each kernel's first N dispatches
    python -m molla_amd.trace_summary DB --steps N --cycle 'KERNEL=wo,down'
        # the same, the dispatches of KERNEL in each step labelled in turn
    python -m molla_amd.trace_summary DB --calls prefill_x_kernel --per 23
        # calls that start at each dispatch of the named kernel, in runs of
        # 23 calls (one bench shape each): median duration per kernel

A decode step starts at an embed_kernel dispatch (DeviceSession.step), so
--steps N keeps the dispatches from the N-th last embed_kernel on and reports
per-step counts and times, the wall span per step, the median embed-to-embed
step and the kernel-busy time per step.  Used for the tables under profiles/.
"""

from __future__ import annotations

import argparse
import collections
import re
import sqlite3


def short(name: str) -> str:
    n = name.replace("void ", "").replace("mi::", "").replace("(anonymous namespace)::", "")
    return re.sub(r"\((float|int|unsigned|__half|mi|const|long|void|signed|RowSegs|at::).*", "", n)[:64]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--steps", type=int, default=0)
    ap.add_argument("--top", type=int, default=20)
    ap.add_argument("--calls", default="")
    ap.add_argument("--per", type=int, default=1)
    ap.add_argument("--first", type=int, default=0,
                    help="each kernel's first N dispatches only, with their median duration")
    ap.add_argument("--cycle", action="append", default=[],
                    help="NAME=a,b: label the dispatches of kernel NAME in each step a, b, a, b, ... in order")
    a = ap.parse_args()
    cycles = {}
    for c in a.cycle:
        name, labels = c.split("=", 1)
        cycles[name] = labels.split(",")
    rows = sqlite3.connect(a.db).execute("select name, start, end from kernels order by start").fetchall()
    if a.calls:
        calls = []
        for name, st, en in rows:
            if a.calls in name:
                calls.append([])
            if calls:
                calls[-1].append((short(name), (en - st) / 1e3))
        # the calls of one run share the kernels of the first; stop a call at
        # any kernel the run's first call does not have
        for r0 in range(0, len(calls) - a.per + 1, a.per):
            run = calls[r0:r0 + a.per]
            names = list(dict.fromkeys(n for n, _ in run[0]))
            per = collections.defaultdict(list)
            for c in run:
                for n, d in c:
                    if n in names:
                        per[n].append(d)
            cells = "; ".join(f"`{n}` {sorted(per[n])[len(per[n]) // 2]:.1f}" for n in names)
            print(f"| run {r0 // a.per} | {cells} |")
        return
    if a.first:
        per = collections.defaultdict(list)
        for name, st, en in rows:
            if len(per[short(name)]) < a.first:
                per[short(name)].append((en - st) / 1e3)
        print("| kernel | calls | avg us | median us |")
        print("|---|---|---|---|")
        for k, d in sorted(per.items(), key=lambda kv: -sum(kv[1]))[: a.top]:
            print(f"| `{k}` | {len(d)} | {sum(d) / len(d):.2f} | {sorted(d)[len(d) // 2]:.2f} |")
        return
    n = 1
    if a.steps:
        emb = [r[1] for r in rows if "embed_kernel" in r[0]]
        t0 = emb[-a.steps]
        rows = [r for r in rows if r[1] >= t0]
        n = a.steps
        span = (max(r[2] for r in rows) - t0) / 1e3
    agg = collections.defaultdict(lambda: [0, 0.0])
    seen = collections.Counter()
    for name, s, e in rows:
        kn = short(name)
        if "embed_kernel" in name:
            seen.clear()
        if kn in cycles:
            labels = cycles[kn]
            seen[kn] += 1
            kn = f"{kn} [{labels[(seen[kn] - 1) % len(labels)]}]"
        x = agg[kn]
        x[0] += 1
        x[1] += (e - s) / 1e3
    busy = sum(v[1] for v in agg.values())
    if a.steps:
        gaps = sorted((b - a_) / 1e3 for a_, b in zip(emb[-a.steps:], emb[-a.steps + 1:]))
        med = gaps[len(gaps) // 2] if gaps else span
        print(f"last {n} steps: {len(rows)} dispatches, span {span / n:.1f} us/step, "
              f"kernel-busy {busy / n:.1f} us/step, median step {med:.1f} us")
    unit = "per step" if a.steps else "calls"
    print(f"| kernel | {unit} | avg us | us{'/step' if a.steps else ' total'} | share |")
    print("|---|---|---|---|---|")
    for k, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1])[: a.top]:
        print(f"| `{k}` | {c / n:g} | {t / c:.2f} | {t / n:.1f} | {100 * t / busy:.1f}% |")


if __name__ == "__main__":
    main()
