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
    assert 80e3 <= rec["value"] <= 80e3 * 1.3


def test_the_first_item_alone_when_even_it_exceeds_the_budget():
    weights = [100, 1, 1]
    log = []
    rec = bench.cpu_timed(_fake(1e-4, weights, log), weights, "us/call", "items", budget_s=0.007, threads=1)
    assert log == [1] * 8  # the sample never drops below one item
    assert "first 1 of 3 items" in rec["sample"]
