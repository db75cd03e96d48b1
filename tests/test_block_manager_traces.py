"""BlockManager against golden traces recorded from the reference
implementation (tests/golden/make_block_manager_trace.py): seeded random
allocate / append / preempt / free / probe / clear / LRU-toggle sequences on
pools of 12 to 40 blocks with 2 to 10 host offload slots.  Every op's return
values, block tables, metrics, free-list head, host slots in use and the
executor calls it made (put / get / release, with arguments, in order) must
match."""
import gzip
import json
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import bm_trace_driver as drv  # noqa: E402

from nanovllm_amd.engine.block_manager import BlockManager  # noqa: E402
from nanovllm_amd.engine.sequence import Sequence  # noqa: E402

with gzip.open(os.path.join(HERE, "golden", "block_manager_trace.json.gz"), "rt") as f:
    TRACES = json.load(f)["traces"]


@pytest.mark.parametrize("trace", TRACES,
                         ids=[f"seed{t['seed']}-{t['num_blocks']}blk-{t['host_slots']}slots"
                              for t in TRACES])
def test_replay_matches_reference_trace(trace):
    got = drv.run(trace["ops"], BlockManager, Sequence, num_blocks=trace["num_blocks"],
                  host_slots=trace["host_slots"], log_calls=True)
    assert len(got) == len(trace["records"])
    for i, (g, want) in enumerate(zip(got, trace["records"])):
        assert g == want, f"op {i} ({trace['ops'][i]['op']}): {g} != {want}"


def test_traces_exercise_offload_paths():
    last = [t["records"][-1]["metrics"] for t in TRACES]
    keys = drv.METRIC_KEYS
    col = lambda k: sum(m[keys.index(k)] for m in last)
    assert col("kv_offload_puts_total") > 0 and col("kv_offload_revives_total") > 0
    assert col("kv_offload_drops_total") > 0 and col("kv_lru_evictions_total") > 0
