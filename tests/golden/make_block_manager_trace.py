"""Writes tests/golden/block_manager_trace.json.gz: seeded BlockManager traces
recorded from the reference implementation (nanovllm/engine/block_manager.py,
loaded from /root/reference by file path with a stub package so the device
tree is not imported).  Run in the development container only:

    python tests/golden/make_block_manager_trace.py
"""
import gzip
import importlib.util
import json
import os
import sys
import types

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
sys.path.insert(0, HERE)
import bm_trace_driver as drv  # noqa: E402


def load(name, rel):
    spec = importlib.util.spec_from_file_location(name, os.path.join(REF, rel))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def main():
    pkg = types.ModuleType("nanovllm")
    pkg.__path__ = [os.path.join(REF, "nanovllm")]
    sys.modules["nanovllm"] = pkg
    eng = types.ModuleType("nanovllm.engine")
    eng.__path__ = [os.path.join(REF, "nanovllm", "engine")]
    sys.modules["nanovllm.engine"] = eng
    sp = load("nanovllm.sampling_params", "nanovllm/sampling_params.py")
    sq = load("nanovllm.engine.sequence", "nanovllm/engine/sequence.py")
    bm = load("nanovllm.engine.block_manager", "nanovllm/engine/block_manager.py")
    traces = []
    # (seed, ops, pool blocks, host slots): the first three are the original
    # 24-block / 5-slot traces; the others squeeze the pool and the host
    # slots (more drops and revive-into-evicted-block cases) or widen them.
    for seed, n_ops, blocks, slots in ((1, 400, 24, 5), (2, 400, 24, 5), (3, 400, 24, 5),
                                       (4, 600, 12, 2), (5, 600, 40, 10), (6, 800, 16, 3)):
        ops = drv.make_ops(seed, n_ops=n_ops)
        recs = drv.run(ops, bm.BlockManager, sq.Sequence, num_blocks=blocks, host_slots=slots,
                       make_seq=lambda toks: sq.Sequence(toks, sp.SamplingParams(max_tokens=1)),
                       log_calls=True)
        traces.append({"seed": seed, "num_blocks": blocks, "host_slots": slots, "ops": ops,
                       "records": recs})
    out = os.path.join(HERE, "block_manager_trace.json.gz")
    with gzip.open(out, "wt") as f:
        json.dump({"source": "nanovllm/engine/block_manager.py (reference), pages of 256; "
                             "each record holds the op's executor calls",
                   "traces": traces}, f, separators=(",", ":"))
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
