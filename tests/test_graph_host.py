"""The product's host paging layer (conflux-nova_amd/code/graph, through the
C ABI of include/nova_graph.h) against the reference's golden traces and the
pinned oracle.  Host-only: nothing here touches a GPU."""
import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

from pool_replay import load_traces, replay, replay_fork, replay_probe

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(autouse=True, params=["host", pytest.param("gpu_box", marks=pytest.mark.gpu)])
def where(request):
    """every test here runs in the CPU suite and again, marked gpu, in the GPU
    box's run, so the product's host paging layer is part of that record"""
    return request.param


@pytest.fixture(scope="module")
def prod_pool(nova7):
    from oracle_py import PoolAPI
    return PoolAPI(nova7.lib, "nova_kvpool_", True)


def test_pool_fork_cow_probe(prod_pool):
    replay_probe(prod_pool, load_traces()["fork_cow_probe"])


@pytest.mark.parametrize("k", range(5))
def test_pool_golden_traces(prod_pool, k):
    replay(prod_pool, load_traces()["traces"][k])


def test_pool_fork_scenario(prod_pool):
    replay_fork(prod_pool, load_traces()["fork"])


@pytest.mark.parametrize("seed", range(8))
def test_pool_fuzz_vs_oracle(prod_pool, oracle, seed):
    """random op sequences recorded on the oracle, replayed on the product"""
    from golden.make_golden import random_trace
    trace = random_trace(oracle.pool, 5000 + seed, 2 + seed % 5, 20 + 29 * seed, 150)
    replay(prod_pool, trace)


def test_pool_large_acquire_matches_oracle(prod_pool, oracle):
    """acquire order and free-list contents at a size where the one-pass removal
    matters (the reference does one std::find per page)"""
    n, ctx = 40, 4096
    a, b = prod_pool.new(n, ctx), oracle.pool.new(n, ctx)
    try:
        for _ in range(n):
            assert prod_pool.acquire(a) == oracle.pool.acquire(b)
            # exercise a few frees / allocs in between
            prod_pool.free_block(a, 3)
            oracle.pool.free_block(b, 3)
        assert prod_pool.free_list_arr(a) == oracle.pool.free_list_arr(b)
        assert prod_pool.refcnt_arr(a) == oracle.pool.refcnt_arr(b)
        assert prod_pool.acquire(a) == oracle.pool.acquire(b) == -1
    finally:
        prod_pool.delete(a)
        oracle.pool.delete(b)


def test_pool_exhaustion_returns_minus_two(prod_pool):
    """cow_slice reports a full pool with -2 (kv_pool.h:160); cow_guard turns
    that into an abort (model.cpp:173, tested on the device-backed layer)"""
    h = prod_pool.new(2, 32)
    try:
        a, b = prod_pool.acquire(h), prod_pool.acquire(h)
        prod_pool.attach_prefix(h, b, a, 20)
        assert prod_pool.free_blocks(h) == 0
        assert prod_pool.cow_slice(h, b, 20) == -2
        assert prod_pool.cow_count(h) == 0
    finally:
        prod_pool.delete(h)


def _nova_hash(nova, ids):
    a = np.ascontiguousarray(ids, dtype=np.int32)
    return nova.nova_kv_hash_ids(a.ctypes.data_as(C.POINTER(C.c_int)), len(a))


def test_kv_block_ids(nova7, oracle):
    g = json.loads((GOLDEN / "kv_hash.json").read_text())
    for c in g["ids"]:
        assert _nova_hash(nova7, c["ids"]) == c["hash"]
    for c in g["texts"]:
        t = c["text"].encode()
        assert nova7.nova_kv_hash_text(t, len(t)) == c["hash"]
    for c in g["block_ids"]:
        out = C.create_string_buffer(40)
        nova7.nova_kv_block_id(c["prefix"], c["suffix"], out)
        assert out.value.decode() == c["id"]
    rng = np.random.default_rng(3)
    for n in range(0, 300, 7):
        ids = rng.integers(-1000, 151936, n)
        assert _nova_hash(nova7, ids) == oracle.kv_hash_ids(ids.tolist())


def test_registry(nova7):
    for case in json.loads((GOLDEN / "registry.json").read_text()):
        h = nova7.nova_registry_new()
        if case["capacity"] != 64:
            nova7.nova_registry_set_capacity(h, case["capacity"])
        for op in case["ops"]:
            if op["op"] == "put":
                nova7.nova_registry_put(h, *op["args"])
                assert (nova7.nova_registry_live(h), nova7.nova_registry_total(h)) == (op["live"], op["total"])
            else:
                s, t, a, b = C.c_int(), C.c_int(), C.c_int64(), C.c_int64()
                ok = nova7.nova_registry_find(h, *op["args"], C.byref(s), C.byref(t), C.byref(a), C.byref(b))
                got = [s.value, t.value, a.value, b.value] if ok else None
                assert got == op["ret"]
        nova7.nova_registry_delete(h)


def test_geometry(nova7, nova15, nova14):
    for nova, want in ((nova7, (28, 4, 128, 28)), (nova15, (12, 2, 128, 28)), (nova14, (40, 8, 128, 48))):
        assert (nova.nh, nova.nkv, nova.hd, nova.n_layers, nova.kb) == want + (16,)
