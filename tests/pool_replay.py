"""Replay the golden KvPool traces (tests/golden/pool_traces.json, produced by
the reference's own code/graph/kv_pool.h) against any implementation exposing
the PoolAPI surface of oracle/oracle_py.py, comparing every return value and
the full pool state after every op."""
from __future__ import annotations

import json
from pathlib import Path

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_traces():
    return json.loads((GOLDEN / "pool_traces.json").read_text())


def state(api, h, live):
    return {
        "free_list": api.free_list_arr(h),
        "refcnt": api.refcnt_arr(h),
        "tables": {str(s): api.table_arr(h, s) for s in sorted(live)},
        "n_past": {str(s): api.n_past(h, s) for s in sorted(live)},
        "need_copy": {str(s): list(api.need_copy_pair(h, s)) for s in sorted(live)},
        "cow_count": api.cow_count(h),
        "free_blocks": api.free_blocks(h),
        "used": api.used(h),
        "free_slices": api.free_slices(h),
    }


def replay(api, trace):
    h = api.new(trace["n_slices"], trace["ctx"])
    live = []
    try:
        for k, op in enumerate(trace["ops"]):
            kind = op["op"]
            if kind == "acquire":
                r = api.acquire(h)
                if r >= 0:
                    live.append(r)
            elif kind == "alloc":
                r = api.alloc_block(h)
            elif kind == "free":
                api.free_block(h, op["b"]); r = None
            elif kind == "ref":
                api.ref_block(h, op["b"]); r = None
            elif kind == "attach":
                api.attach(h, op["dst"], op["src"], op["k"]); r = None
            elif kind == "attach_prefix":
                api.attach_prefix(h, op["dst"], op["src"], op["n"]); r = None
            elif kind == "cow":
                r = api.cow_slice(h, op["s"], op["pos"])
            elif kind == "release":
                api.release(h, op["s"]); live.remove(op["s"]); r = None
            else:
                raise AssertionError(kind)
            assert r == op["ret"], (trace["seed"], k, kind, r, op["ret"])
            got = state(api, h, live)
            assert got == op["state"], (trace["seed"], k, kind,
                                        {key: (got[key], op["state"][key]) for key in got
                                         if got[key] != op["state"][key]})
    finally:
        api.delete(h)


def replay_probe(api, probe):
    h = api.new(3, 64)
    try:
        a, b = api.acquire(h), api.acquire(h)
        api.attach_prefix(h, b, a, 20)
        nb = api.cow_slice(h, b, 20)
        assert (a, b, nb) == (probe["A"], probe["B"], probe["cow_ret"])
        assert api.free_blocks(h) == probe["free_blocks"] == 3
        assert api.refcnt(h, api.table_arr(h, a)[1]) == probe["refcnt_A_table1"] == 1
        assert api.refcnt(h, nb) == probe["refcnt_new"] == 1
        assert state(api, h, [a, b]) == probe["state"]
    finally:
        api.delete(h)


def replay_fork(api, f):
    import numpy as np
    rng = np.random.default_rng(f["seed"])
    n_roots, per_root, prefix, ctx = f["n_roots"], f["per_root"], f["prefix"], f["ctx"]
    h = api.new(n_roots + n_roots * per_root + f["spare"], ctx)
    try:
        roots = [api.acquire(h) for _ in range(n_roots)]
        kids = [api.acquire(h) for _ in range(n_roots * per_root)]
        for c, k in enumerate(kids):
            api.attach_prefix(h, k, roots[c % n_roots], prefix)
        pos = {k: prefix for k in kids}
        rets = []
        for _ in range(ctx - prefix):
            for k in kids:
                if rng.random() < 0.7 and pos[k] < ctx:
                    rets.append(api.cow_slice(h, k, pos[k]))
                    pos[k] += 1
        assert rets == f["cow_rets"]
        assert state(api, h, roots + kids) == f["state"]
        # COW exactly once per child of an unaligned fork (tests/cow_e2e_demo.cpp:87-88)
        assert sum(1 for r in rets if r >= 0) == n_roots * per_root
    finally:
        api.delete(h)
