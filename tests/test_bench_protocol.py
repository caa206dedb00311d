"""The bench's CPU-baseline protocol (``bench.cpu_timed``) on the CPU: one probe call of
the first item prices the work per unit of weight, the sample is the longest prefix of
items whose call fits the budget split over the warm-ups and timed calls, the warm-ups
and timed calls all run that sample, and the reported value is the median timed call
scaled to the whole call by weight. A fake workload whose time is proportional to its
weight stands in for the oracle."""

import time

import pytest
import torch

import bench


@pytest.fixture(autouse=True)
def _threads():
    """cpu_timed sets torch's thread count; the tests that follow keep theirs."""
    n = torch.get_num_threads()
    yield
    torch.set_num_threads(n)


def _fake(per_weight_s, weights, log):
    def run(n):
        log.append(n)
        time.sleep(per_weight_s * sum(weights[:n]))

    return run


def test_sample_prefix_and_call_order():
    weights = [10, 20, 30, 80]  # prefixes 10, 30, 60 fit 100 ms per call; 140 does not
    log = []
    rec = bench.cpu_timed(_fake(1e-3, weights, log), weights, "us/call", "items", budget_s=0.7, threads=1)
    assert log == [1] + [3] * 7  # the probe, 2 warm-ups, 5 timed calls
    assert rec["sample"].startswith("first 3 of 4 items (60 of 140 by weight): median of 5 calls after 2 warm-ups")
    assert rec["cores"] == 1 and rec["kind"] == "port" and rec["unit"] == "us/call"


def test_value_scaled_to_the_whole_call():
    weights = [5, 5, 5, 5, 5, 5, 5, 5]
    log = []
    rec = bench.cpu_timed(_fake(2e-3, weights, log), weights, "us/call", "items", budget_s=0.18, threads=1,
                          warmups=1, calls=3)  # 45 ms per call: about 4 of the 8 items
    n = log[1]
    assert 1 <= n < len(weights) and log == [1] + [n] * 4
    # a call of the whole batch would sleep 80 ms; the sample's median, scaled by weight, says so
    # (sleeps never end early; a loaded host may add to them)
    assert 80e3 <= rec["value"] <= 80e3 * 1.6


def test_the_first_item_alone_when_even_it_exceeds_the_budget():
    weights = [100, 1, 1]
    log = []
    rec = bench.cpu_timed(_fake(1e-4, weights, log), weights, "us/call", "items", budget_s=0.007, threads=1)
    assert log == [1] * 8  # the sample never drops below one item
    assert "first 1 of 3 items" in rec["sample"]


def test_more_than_one_gpu_is_refused():
    """``bench.py --gpus N`` for N above 1 exits with status 2 and says why, before it
    touches a GPU (one GPU is what is measured)."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    p = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=root)
    assert p.returncode == 2
    assert "GPU" in p.stderr + p.stdout


def test_committed_traffic_records_are_consistent():
    """Each committed calibrated-traffic record: the copy calibration gives the factors (a
    1 GiB copy reads and writes 1 GiB), and the record's bytes per launch are the kernel's
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by them; its commands name the
    counter runs they came from."""
    import json
    from pathlib import Path

    recs = sorted((Path(__file__).resolve().parents[1] / "profiles").glob("*.traffic.json"))
    assert recs
    for f in recs:
        r = json.loads(f.read_text())
        ff = r["copy_bytes"] / (r["copy_fetch_kib"] * 1024)
        wf = r["copy_bytes"] / (r["copy_write_kib"] * 1024)
        assert abs(ff - r["fetch_factor"]) < 1e-4 and abs(wf - r["write_factor"]) < 1e-4, f.name
        want = r["fetch_kib_per_dispatch"] * 1024 * ff + r["write_kib_per_dispatch"] * 1024 * wf
        assert abs(r["traffic_bytes"] - want) / want < 1e-6, f.name
        assert any("--pmc FETCH_SIZE" in c and r["workload"] in c for c in r["commands"]), f.name
        assert any("--pmc WRITE_SIZE" in c and r["workload"] in c for c in r["commands"]), f.name


def test_committed_mfma_records_are_consistent():
    """Each committed MFMA record: its utilisation is SQ_VALU_MFMA_BUSY_CYCLES over the
    SIMDs' cycles (1024 SIMDs, SQ_CYCLES counted per 32 shader engines), its MFMA work
    (MOPS x 512 flop) is the workload's algorithmic 4 K Hq D sum(L) to within 1 % (no
    MFMA work is wasted beyond the padding of a unit's rows), and its TFLOP/s is that work
    over the counted dispatches' mean duration."""
    import json
    import re
    from pathlib import Path

    algorithmic = {"c3-qwen3-8b-paged-b64": 4 * 16 * 32 * 128 * 245380,
                   "c3-qwen3-8b-paged-b64-fp8": 4 * 16 * 32 * 128 * 245380,
                   "c5-27b-gqa5-b32": 4 * 16 * 40 * 128 * 172058}
    recs = sorted((Path(__file__).resolve().parents[1] / "profiles").glob("*.mfma.json"))
    assert recs
    for f in recs:
        r = json.loads(f.read_text())
        c = r["counters"]
        util = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (r["simds"] * c["SQ_CYCLES"] / r["shader_engines"])
        assert abs(util - r["util"]) < 1e-3, f.name
        flop = (c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] + c["SQ_INSTS_VALU_MFMA_MOPS_F8"]) * 512
        assert 1.0 <= flop / algorithmic[r["workload"]] < 1.01, f.name
        tflops = float(re.search(r"([0-9.]+) TFLOP/s", r["derivation"]).group(1))
        assert abs(tflops - flop / (r["mean_duration_us"] * 1e-6) / 1e12) < 0.1, f.name
