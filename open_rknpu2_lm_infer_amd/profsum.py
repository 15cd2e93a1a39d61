"""Summaries of rocprofv3 result databases (SQLite, the default rocprofv3 output).

    python -m open_rknpu2_lm_infer_amd.profsum stats  RESULTS.db [--match REGEX] [--md]
    python -m open_rknpu2_lm_infer_amd.profsum pmc    RESULTS.db [--match REGEX]
    python -m open_rknpu2_lm_infer_amd.profsum traffic --fetch F.db --write W.db \
        --copy-fetch CF.db --copy-write CW.db --copy-bytes B --match REGEX

`stats` prints per-kernel dispatch count and average / min / max duration;
`pmc` prints the per-dispatch average of every collected counter; `traffic` turns
FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the matched kernel into bytes per
launch, each scaled by what the same counter reads for a plain copy of known size.
"""
from __future__ import annotations

import argparse
import re
import sqlite3
import sys


def _con(path):
    return sqlite3.connect(f"file:{path}?mode=ro", uri=True)


def kernel_stats(path, match=None):
    rows = _con(path).execute(
        "select name, count(*), avg(duration), min(duration), max(duration), grid_x, workgroup_x, "
        "vgpr_count, accum_vgpr_count, lds_size from kernels group by name, grid_x order by sum(duration) desc"
    ).fetchall()
    out = []
    for name, n, avg, mn, mx, gx, wx, vgpr, agpr, lds in rows:
        if match and not re.search(match, name):
            continue
        out.append(dict(name=name, dispatches=n, avg_us=avg / 1e3, min_us=mn / 1e3, max_us=mx / 1e3,
                        workgroups=gx // max(wx, 1), wg_size=wx, vgpr=vgpr, agpr=agpr, lds=lds))
    return out


def pmc_means(path, match=None, chunk=0):
    """{kernel name [grid]: {counter: mean value per dispatch}} (values summed over
    instances), one entry per kernel and grid size.  chunk > 0 splits each entry into
    consecutive runs of that many dispatches (in dispatch order), labelled #0, #1, ...:
    a program that launches the same kernel and grid for different shapes one shape
    after another gets one entry per shape."""
    con = _con(path)
    rows = con.execute(
        "select P.name, K.grid_x / max(K.workgroup_x, 1), P.dispatch_id, P.counter_name, sum(P.counter_value) "
        "from pmc_events P join kernels K on K.dispatch_id = P.dispatch_id "
        "group by P.name, K.grid_x, P.dispatch_id, P.counter_name order by P.dispatch_id").fetchall()
    order = {}
    for name, wgs, disp, _, _ in rows:
        ids = order.setdefault((name, wgs), [])
        if not ids or ids[-1] != disp:
            ids.append(disp)
    rank = {(k, d): i for k, ids in order.items() for i, d in enumerate(ids)}
    acc = {}
    for name, wgs, disp, cn, v in rows:
        if match and not re.search(match, name):
            continue
        key = f"{name} [{wgs} workgroups]"
        if chunk:
            key += f" #{rank[((name, wgs), disp)] // chunk}"
        d = acc.setdefault(key, {}).setdefault(cn, [0.0, 0])
        d[0] += v
        d[1] += 1
    return {k: {c: s / n for c, (s, n) in v.items()} for k, v in acc.items()}


def _one(path, counter, match):
    m = pmc_means(path, match)
    vals = [v[counter] for v in m.values() if counter in v]
    if not vals:
        raise SystemExit(f"no {counter} for /{match}/ in {path}")
    return sum(vals) / len(vals)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=["stats", "pmc", "traffic"])
    ap.add_argument("db", nargs="?")
    ap.add_argument("--match", default=None)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-match", default="copyBuffer")
    ap.add_argument("--copy-bytes", type=float)
    ap.add_argument("--md", action="store_true", help="stats as a markdown table with each kernel's share")
    ap.add_argument("--chunk", type=int, default=0,
                    help="pmc / traffic: split each kernel and grid into runs of N dispatches (traffic: one line each)")
    a = ap.parse_args(argv)
    if a.what == "stats" and a.md:
        rows = kernel_stats(a.db, a.match)
        total = sum(r["avg_us"] * r["dispatches"] for r in rows) or 1.0
        print("| kernel | grid (workgroups x size) | calls | avg us | min us | max us | share of listed time |")
        print("|---|---|---:|---:|---:|---:|---:|")
        for r in rows:
            share = 100.0 * r["avg_us"] * r["dispatches"] / total
            print(f"| `{r['name'][:100]}` | {r['workgroups']}x{r['wg_size']} | {r['dispatches']} | {r['avg_us']:.2f} | "
                  f"{r['min_us']:.2f} | {r['max_us']:.2f} | {share:.1f}% |")
        return 0
    if a.what == "stats":
        for r in kernel_stats(a.db, a.match):
            print(f"{r['avg_us']:9.2f} us avg  {r['min_us']:8.2f} min  {r['max_us']:8.2f} max  n={r['dispatches']:6d}  "
                  f"wg={r['workgroups']}x{r['wg_size']} vgpr={r['vgpr']} lds={r['lds']}  {r['name'][:110]}")
    elif a.what == "pmc":
        for name, d in pmc_means(a.db, a.match, a.chunk).items():
            print(name[:120])
            for c, v in sorted(d.items()):
                print(f"    {c:32s} {v:16.2f}")
    else:
        f_c = _one(a.copy_fetch, "FETCH_SIZE", a.copy_match)
        w_c = _one(a.copy_write, "WRITE_SIZE", a.copy_match)
        kib = a.copy_bytes / 1024.0
        f_scale, w_scale = kib / f_c, kib / w_c
        print(f"copy of {a.copy_bytes:.0f} B: FETCH_SIZE {f_c:.1f} KiB (scale {f_scale:.4f}), "
              f"WRITE_SIZE {w_c:.1f} KiB (scale {w_scale:.4f})")
        if a.chunk:
            # every matched kernel and grid, split into runs of --chunk dispatches
            fm, wm = pmc_means(a.fetch, a.match, a.chunk), pmc_means(a.write, a.match, a.chunk)
            for name in fm:
                if "FETCH_SIZE" not in fm[name] or "WRITE_SIZE" not in wm.get(name, {}):
                    continue
                fb = fm[name]["FETCH_SIZE"] * f_scale * 1024.0
                wb = wm[name]["WRITE_SIZE"] * w_scale * 1024.0
                print(f"{name[:110]}: fetch {fb:.0f} B, write {wb:.0f} B, traffic {fb + wb:.0f} B")
            return 0
        f_k = _one(a.fetch, "FETCH_SIZE", a.match)
        w_k = _one(a.write, "WRITE_SIZE", a.match)
        fetch_b = f_k * f_scale * 1024.0
        write_b = w_k * w_scale * 1024.0
        print(f"kernel /{a.match}/: FETCH_SIZE {f_k:.1f} KiB -> {fetch_b:.0f} B, WRITE_SIZE {w_k:.1f} KiB -> {write_b:.0f} B")
        print(f"traffic_bytes_per_launch: {fetch_b + write_b:.0f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
