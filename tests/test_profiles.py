"""The committed profile summaries agree with what bench.py reports from them."""
import json
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_decode_traffic_single_source():
    """roofline.traffic comes from profiles/decode_step_traffic.json, written
    by the same computation that printed the summary text: one figure."""
    with open(os.path.join(ROOT, "profiles", "decode_step_traffic.json")) as f:
        t = json.load(f)
    with open(os.path.join(ROOT, "profiles", "decode_step_gemv_hbm_traffic.txt")) as f:
        txt = f.read()
    m = re.search(r"traffic = (\d+) bytes per step vs (\d+) algorithmic", txt)
    assert m, "summary line missing"
    assert int(m.group(1)) == t["traffic_bytes_per_step"]
    assert int(m.group(2)) == t["algorithmic_bytes_per_step"]
    raw = t["fetch_kib_per_step_raw"] * t["fetch_scale"] + t["write_kib_per_step_raw"] * t["write_scale"]
    assert abs(raw * 1024 - t["traffic_bytes_per_step"]) < 1e-3 * t["traffic_bytes_per_step"]
