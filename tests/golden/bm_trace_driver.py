"""Seeded BlockManager operation traces (shared by the fixture generator and
the replay test).

An op list is generated from a seed, then executed against a BlockManager
class and a Sequence class with a slot-accounting executor (LIFO host slots,
-1 when full).  The record of every op — return values, block tables,
metrics, host slots in use — is what the fixture stores.
"""
import random


class SlotExecutor:
    """Host slot accounting of the offload executor protocol (no bytes)."""

    def __init__(self, capacity):
        self.free = list(range(capacity - 1, -1, -1))
        self.in_use = {}
        self.log = []

    def call(self, name, *args):
        self.log.append([name, *args])
        if name == "offload_put":
            if not self.free:
                return -1
            slot = self.free.pop()
            self.in_use[slot] = args[0]
            return slot
        if name == "offload_get":
            self.in_use[args[0]] = args[1]
            return None
        if name == "offload_release":
            del self.in_use[args[0]]
            self.free.append(args[0])
            return None
        raise AssertionError(name)


def make_ops(seed, n_ops=400, n_docs=4, block_size=256):
    rng = random.Random(seed)
    ops, live, next_id, uniq = [], [], 0, 10**6
    for _ in range(n_ops):
        r = rng.random()
        if live and r < 0.30:
            ops.append({"op": "free", "id": live.pop(rng.randrange(len(live)))})
        elif live and r < 0.55:
            ops.append({"op": "append", "id": rng.choice(live), "n": rng.choice([1, 3, 17, 255])})
        elif r < 0.62:
            doc = rng.randrange(n_docs)
            ops.append({"op": "probe", "doc": doc, "len": rng.randrange(1, 4 * block_size)})
        elif r < 0.64:
            ops.append({"op": "clear"})
        elif r < 0.66:
            ops.append({"op": "lru", "on": rng.random() < 0.7})
        else:
            doc = rng.randrange(n_docs)
            plen = rng.randrange(block_size, 5 * block_size)
            tail = rng.randrange(0, 300)
            ops.append({"op": "new", "id": next_id, "doc": doc, "plen": plen, "tail": [uniq, tail]})
            uniq += tail
            live.append(next_id)
            next_id += 1
    return ops


METRIC_KEYS = (
    "kv_blocks_used", "kv_prefix_hit_tokens_total", "kv_block_allocations_total",
    "kv_block_reclaims_total", "kv_lru_size", "kv_lru_evictions_total", "kv_lru_enabled",
    "kv_offload_host_entries", "kv_offload_puts_total", "kv_offload_revives_total",
    "kv_offload_drops_total")


def op_tokens(op):
    if op["op"] == "probe":
        return [op["doc"] * 100000 + i for i in range(op["len"])]
    start, n = op["tail"]
    return [op["doc"] * 100000 + i for i in range(op["plen"])] + list(range(start, start + n))


def run(ops, manager_cls, sequence_cls, num_blocks=24, block_size=256, host_slots=5,
        make_seq=None, log_calls=False):
    """Execute `ops`; with log_calls every record also carries the executor
    calls the op made, in order, with their arguments."""
    logged = 0
    mgr = manager_cls(num_blocks, block_size)
    mgr.lru_enabled = True
    ex = SlotExecutor(host_slots)
    mgr.set_offload_executor(ex)
    seqs = {}
    records = []
    make_seq = make_seq or (lambda toks: sequence_cls(toks))
    for op in ops:
        kind = op["op"]
        rec = {"op": kind}
        if kind == "new":
            s = make_seq(op_tokens(op))
            c = mgr.can_allocate(s)
            rec["cached"] = c
            if c != -1:
                mgr.allocate(s, c)
                mgr.hash_blocks(s, len(s) - s.num_cached_tokens)
                s.num_cached_tokens = len(s)
                seqs[op["id"]] = s
                rec["table"] = list(s.block_table)
        elif kind == "free":
            s = seqs.pop(op["id"], None)
            if s is not None:
                mgr.deallocate(s)
        elif kind == "append":
            s = seqs.get(op["id"])
            if s is not None:
                ok = 0
                for k in range(op["n"]):
                    s.append_token(7 * len(s) + k)
                    if not mgr.can_append(s):
                        # no block for the new token: the scheduler preempts
                        mgr.deallocate(s)
                        del seqs[op["id"]]
                        rec["preempted"] = True
                        break
                    mgr.may_append(s)
                    mgr.hash_blocks(s, 1)
                    s.num_cached_tokens = len(s)
                    ok += 1
                rec["appended"] = ok
                rec["table"] = list(s.block_table)
        elif kind == "probe":
            rec["cached"] = mgr.can_allocate(make_seq(op_tokens(op)), touch=False)
        elif kind == "clear":
            mgr.clear_prefix_cache()
        elif kind == "lru":
            mgr.lru_enabled = op["on"]
        m = mgr.metrics()
        rec["metrics"] = [m[k] for k in METRIC_KEYS]
        rec["free_head"] = list(mgr.free_block_ids)[:8]
        rec["host_in_use"] = sorted(ex.in_use)
        rec["exec_calls"] = len(ex.log)
        if log_calls:
            rec["exec_log"] = ex.log[logged:]
            logged = len(ex.log)
        records.append(rec)
    return records
