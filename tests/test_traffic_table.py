"""The committed HBM traffic table (profiles/traffic.json) that bench.py's roofline objects read: every entry's bytes
follow from its counters and the copy-kernel calibration, sit within a few percent above the algorithmic bytes of its
workload, and were measured on the kernel sources in the tree (otherwise the bench reports traffic as null)."""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

_omp = {k: os.environ.get(k) for k in ("GOMP_SPINCOUNT", "OMP_PROC_BIND")}
import bench  # noqa: E402  (sets the OpenMP variables above for its own CPU baseline)

for _k, _v in _omp.items():                         # leave this process's environment as it was
    if _v is None:
        os.environ.pop(_k, None)
    else:
        os.environ[_k] = _v

# algorithmic bytes per launch of each measured workload (bench.py's formulas: the expert body's four experts of
# gate_up + down at batch 1; the attention block's weights plus the K / V rows of 128 ring slots or ~4096 positions)
BLOCK_W = 2 * (5120 * 2880 + 5120 + 2880 * 4096 + 2880 + 128 * 2880 + 128 + 2 * 2880 + 64)
ALGO = {
    ("k_moe_one_t950", "t950"): 4 * bench.SLOT_ALGO_BYTES,
    ("k_attn_block", "sliding"): BLOCK_W + 2 * 2 * 8 * 64 * 128,
    ("k_attn_block", "full"): BLOCK_W + 2 * 2 * 8 * 64 * 4097,
}


def table():
    with open(bench.TRAFFIC_FILE) as fh:
        return json.load(fh)


def test_entries_follow_from_counters_and_calibration():
    tab = table()
    cal = tab["calibration"]
    ff, wf = cal["bytes"] / 1024 / cal["fetch_kib"], cal["bytes"] / 1024 / cal["write_kib"]
    assert abs(ff - cal["fetch_factor"]) < 1e-3 and abs(wf - cal["write_factor"]) < 1e-3
    assert tab["entries"], "no measured workload"
    for e in tab["entries"]:
        hbm = (e["fetch_kib"] * ff + e["write_kib"] * wf) * 1024
        assert abs(hbm - e["hbm_bytes_per_launch"]) <= 1e-6 * hbm + 1, e["kernel"]


@pytest.mark.parametrize("key", sorted(ALGO))
def test_traffic_close_to_algorithmic_bytes(key):
    e = next((e for e in table()["entries"] if (e["kernel"], e["layout"]) == key), None)
    assert e is not None, f"{key} not measured"
    ratio = e["hbm_bytes_per_launch"] / ALGO[key]
    assert 1.0 <= ratio < 1.06, (key, ratio)      # every byte read about once, a little metadata and output on top


def test_entries_measured_on_current_sources():
    for e in table()["entries"]:
        files = tuple(e.get("sources", bench.KERNEL_SOURCES))
        assert e["sources_sha256"] == bench.sources_sha256(files), (
            f"{e['kernel']} ({e['layout']}) was profiled on other sources: re-measure it (FETCH_SIZE / WRITE_SIZE "
            "passes) or the bench reports its traffic as null")
    assert bench.measured_traffic("k_moe_one_t950", "t950", 1, 4)[1] == "ok"
    assert bench.attn_block_entry("sliding") is not None and bench.attn_block_entry("full") is not None
