"""Summarise a rocprofv3 results database (rocpd SQLite) as short text.

    python -m ggnpu_amd.profile_summary stats <results.db> [name-filter]
    python -m ggnpu_amd.profile_summary pmc   <results.db> [name-filter]
    python -m ggnpu_amd.profile_summary traffic <fetch.db> <write.db> <copy_fetch.db>
            <copy_write.db> <steps> <copy_bytes> <algorithmic_bytes_per_step> <out.json> [name-filter]

`stats`: per kernel (and grid size): dispatches, mean / min / max duration.
`pmc`:   per kernel (and grid size): mean counter value per dispatch for
         every collected counter (FETCH_SIZE / WRITE_SIZE are in KiB).
`traffic`: HBM bytes per step of a profiled run of `steps` steps: the sum of
         FETCH_SIZE and of WRITE_SIZE over the matching kernels' dispatches,
         each scaled by the factor that makes the same counter read the known
         size of a device copy (copy_bytes read and written per copy), divided
         by `steps`.  Prints the tables and the derivation, and writes the one
         figure (with its inputs) to out.json.
"""
import json
import sqlite3
import sys


def stats(db, pat):
    c = sqlite3.connect(db)
    q = ("select name, grid_x / workgroup_x, count(*), avg(duration), min(duration), max(duration), "
         "sum(duration), max(vgpr_count), max(lds_size) from kernels where name like ? "
         "group by name, grid_x order by sum(duration) desc")
    print("%-64s %7s %6s %9s %9s %9s %11s %5s %6s" % ("kernel", "wgs", "calls", "avg_us", "min_us", "max_us",
                                                    "total_us", "vgpr", "lds"))
    for name, wgs, n, avg, mn, mx, tot, vg, lds in c.execute(q, (pat,)):
        print("%-64s %7d %6d %9.2f %9.2f %9.2f %11.1f %5d %6d" % (name[:64], wgs, n, avg / 1e3, mn / 1e3, mx / 1e3,
                                                                tot / 1e3, vg or 0, lds or 0))


def pmc(db, pat):
    c = sqlite3.connect(db)
    q = ("select p.name, k.grid_x / k.workgroup_x, p.counter_name, count(distinct p.dispatch_id), "
         "sum(p.counter_value) / count(distinct p.dispatch_id), avg(p.duration) "
         "from pmc_events p join kernels k on k.dispatch_id = p.dispatch_id where p.name like ? "
         "group by p.name, k.grid_x, p.counter_name order by p.name")
    try:
        rows = list(c.execute(q, (pat,)))
    except sqlite3.OperationalError:
        q = ("select name, 0, counter_name, count(distinct dispatch_id), sum(counter_value) / "
             "count(distinct dispatch_id), avg(duration) from pmc_events where name like ? "
             "group by name, counter_name order by name")
        rows = list(c.execute(q, (pat,)))
    print("%-64s %7s %-14s %6s %14s" % ("kernel", "wgs", "counter", "calls", "per_dispatch"))
    for name, wgs, cn, n, v, _ in rows:
        print("%-64s %7d %-14s %6d %14.1f" % (name[:64], wgs, cn, n, v))


def _counter_sum(db, counter, pat):
    """(sum of counter over all matching dispatches in KiB, dispatches)."""
    c = sqlite3.connect(db)
    row = c.execute("select sum(counter_value), count(distinct dispatch_id) from pmc_events "
                    "where name like ? and counter_name = ?", (pat, counter)).fetchone()
    return float(row[0] or 0.0), int(row[1] or 0)


def traffic(fdb, wdb, cfdb, cwdb, steps, copy_bytes, alg_bytes, out_json, pat="%ggq%"):
    steps, copy_bytes, alg_bytes = int(steps), int(copy_bytes), int(alg_bytes)
    copy_kib = copy_bytes / 1024
    cf, nf = _counter_sum(cfdb, "FETCH_SIZE", "%copyBuffer%")
    cw, nw = _counter_sum(cwdb, "WRITE_SIZE", "%copyBuffer%")
    fscale = copy_kib / (cf / nf)
    wscale = copy_kib / (cw / nw)
    f, df = _counter_sum(fdb, "FETCH_SIZE", pat)
    w, dw = _counter_sum(wdb, "WRITE_SIZE", pat)
    fetch = f * fscale / steps * 1024
    write = w * wscale / steps * 1024
    tot = round(fetch + write)
    print("# per kernel, FETCH_SIZE run:")
    pmc(fdb, pat)
    print("# per kernel, WRITE_SIZE run:")
    pmc(wdb, pat)
    print(f"# calibration copy ({copy_kib:.0f} KiB read + written): FETCH_SIZE {cf / nf:.1f} KiB -> x {fscale:.3f}, "
          f"WRITE_SIZE {cw / nw:.1f} KiB -> x {wscale:.3f}")
    print(f"# {df} / {dw} matching dispatches over {steps} steps")
    print(f"# per step: fetch {f / steps:.1f} KiB raw x {fscale:.3f} = {fetch / 1e6:.1f} MB; "
          f"write {w / steps:.1f} KiB raw x {wscale:.3f} = {write / 1e6:.2f} MB")
    print(f"# traffic = {tot} bytes per step vs {alg_bytes} algorithmic ({tot / alg_bytes:.3f}x)")
    with open(out_json, "w") as fh:
        json.dump({"source": "ggnpu_amd/profile_summary.py traffic over the FETCH_SIZE / WRITE_SIZE runs",
                   "traffic_bytes_per_step": tot, "algorithmic_bytes_per_step": alg_bytes,
                   "fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4),
                   "fetch_kib_per_step_raw": round(f / steps, 1), "write_kib_per_step_raw": round(w / steps, 1),
                   "steps_profiled": steps}, fh)
        fh.write("\n")


if __name__ == "__main__":
    mode = sys.argv[1]
    if mode == "traffic":
        traffic(*sys.argv[2:])
    else:
        db = sys.argv[2]
        pat = sys.argv[3] if len(sys.argv) > 3 else "%"
        {"stats": stats, "pmc": pmc}[mode](db, pat)
