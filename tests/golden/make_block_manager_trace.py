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
    for seed in (1, 2, 3):
        ops = drv.make_ops(seed)
        recs = drv.run(ops, bm.BlockManager, sq.Sequence,
                       make_seq=lambda toks: sq.Sequence(toks, sp.SamplingParams(max_tokens=1)))
        traces.append({"seed": seed, "ops": ops, "records": recs})
    out = os.path.join(HERE, "block_manager_trace.json.gz")
    with gzip.open(out, "wt") as f:
        json.dump({"source": "nanovllm/engine/block_manager.py (reference), 24 blocks x 256, "
                             "5 host slots", "traces": traces}, f, separators=(",", ":"))
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
