"""Summarise a rocprofv3 results database (rocpd SQLite) as short text.

    python -m ggnpu_amd.profile_summary stats <results.db> [name-filter]
    python -m ggnpu_amd.profile_summary pmc   <results.db> [name-filter]

`stats`: per kernel (and grid size): dispatches, mean / min / max duration.
`pmc`:   per kernel (and grid size): mean counter value per dispatch for
         every collected counter (FETCH_SIZE / WRITE_SIZE are in KiB).
"""
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


if __name__ == "__main__":
    mode, db = sys.argv[1], sys.argv[2]
    pat = sys.argv[3] if len(sys.argv) > 3 else "%"
    {"stats": stats, "pmc": pmc}[mode](db, pat)
