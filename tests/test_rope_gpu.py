"""Parity of the gfx950 RoPE and the fused RoPE + paged append against the CPU
oracle (or_rope_table / or_rope_apply / or_rope_kv_store_paged, restating
src/kernel/rope.cu:9-58 and RopeKvOp, code/graph/dense.h:75-83).

Bit-exact throughout: the table is the reference recipe with correctly
rounded steps on both sides; the rotation is x0*c - x1*s / x0*s + x1*c without
contraction on both sides; the append rounds to fp16 to nearest even.
"""
import numpy as np
import pytest

from helpers import PagedFixture

pytestmark = pytest.mark.gpu
LAYER = 3
MODELS = ["qwen25_7b", "qwen25_1p5b", "qwen25_14b"]


def _table(nova, rows=None):
    half = nova.hd // 2
    n = 4096 if rows is None else rows
    cs, sn = nova.alloc(n * half * 4), nova.alloc(n * half * 4)
    if rows is None:
        nova.launch_rope_table(cs.ptr, sn.ptr, None)
    else:
        nova.launch_rope_table_rows(cs.ptr, sn.ptr, rows, None)
    nova.dev_sync()
    return cs, sn, cs.numpy((n, half), np.float32), sn.numpy((n, half), np.float32)


@pytest.mark.parametrize("rows", [None, 40000])
def test_rope_table(rows, nova7, oracle):
    print(f"[case] rope table rows={rows}", flush=True)
    _, _, cs, sn = _table(nova7, rows)
    rcs, rsn = oracle.rope_table(cs.shape[0], 64, 1e6)
    assert np.array_equal(cs, rcs) and np.array_equal(sn, rsn)


@pytest.mark.parametrize("model", MODELS)
def test_rope_batch_in_place(model, oracle):
    import nova_amd
    nova = nova_amd.load(model)
    print(f"[case] rope batch model={model}", flush=True)
    dcs, dsn, cs, sn = _table(nova)
    rng = np.random.default_rng(5)
    for n, pos0 in ((1, 0), (1, 4095), (37, 100), (300, 3000)):
        q = rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
        k = rng.standard_normal((n, nova.nkv, nova.hd)).astype(np.float32)
        dq, dk = nova.upload(q), nova.upload(k)
        if n == 1:
            nova.launch_rope(dq.ptr, dk.ptr, pos0, dcs.ptr, dsn.ptr, None)
        else:
            nova.launch_rope_batch(dq.ptr, dk.ptr, n, pos0, dcs.ptr, dsn.ptr, None)
        nova.dev_sync()
        rq, rk = oracle.rope_apply(model, q, k, pos0, cs, sn)
        assert np.array_equal(dq.numpy(q.shape, np.float32), rq), (n, pos0)
        assert np.array_equal(dk.numpy(k.shape, np.float32), rk), (n, pos0)


@pytest.mark.parametrize("model,n,pos0", [("qwen25_7b", 1, 17), ("qwen25_7b", 45, 13),
                                          ("qwen25_1p5b", 64, 0), ("qwen25_14b", 19, 250)])
def test_rope_kv_store_paged(model, n, pos0, oracle):
    import nova_amd
    nova = nova_amd.load(model)
    print(f"[case] rope+append model={model} n={n} pos0={pos0}", flush=True)
    dcs, dsn, cs, sn = _table(nova)
    pages = (pos0 + n + 15) // 16
    fx = PagedFixture(nova, nb=pages + 3, layer=LAYER, seed=n + pos0)
    table = fx.tables(1, pages)[0]
    rng = np.random.default_rng(n)
    q = rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
    k = rng.standard_normal((n, nova.nkv, nova.hd)).astype(np.float32)
    v = rng.standard_normal((n, nova.nkv, nova.hd)).astype(np.float32)
    dq, dk, dv, dt = nova.upload(q), nova.upload(k), nova.upload(v), nova.upload(table)
    nova.launch_rope_kv_store_paged(dq.ptr, dk.ptr, dv.ptr, dcs.ptr, dsn.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, LAYER,
                                    fx.nb, n, pos0, None)
    nova.dev_sync()
    hk, hv = fx.hk.copy(), fx.hv.copy()
    rq = oracle.rope_kv_store_paged(model, q, k, v, cs, sn, hk, hv, table, 0, fx.nb, pos0)
    gk, gv = fx.pull()
    assert np.array_equal(dq.numpy(q.shape, np.float32), rq)
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv)       # appended rows and every other slot
    assert np.array_equal(dk.numpy(k.shape, np.float32), k)        # k's buffer is not rotated


@pytest.mark.parametrize("n", [1, 33])
def test_rope_kv_store_paged_batch(n, nova7, oracle):
    """A decode step (n = 1) and a prefill chunk (n = 33) for 5 ragged sessions."""
    nova = nova7
    print(f"[case] rope+append batch n={n}", flush=True)
    dcs, dsn, cs, sn = _table(nova)
    n_past = np.array([0, 15, 16, 777, 40], np.int32)
    pages = int((n_past.max() + n + 15) // 16)
    fx = PagedFixture(nova, nb=5 * pages + 2, layer=LAYER, seed=90 + n)
    tables = fx.tables(5, pages)
    rng = np.random.default_rng(77)
    q = rng.standard_normal((5, n, nova.nh, nova.hd)).astype(np.float32)
    k = rng.standard_normal((5, n, nova.nkv, nova.hd)).astype(np.float32)
    v = rng.standard_normal((5, n, nova.nkv, nova.hd)).astype(np.float32)
    dq, dk, dv = nova.upload(q), nova.upload(k), nova.upload(v)
    dt, dn = nova.upload(tables), nova.upload(n_past)
    nova.launch_rope_kv_store_paged_batch(dq.ptr, dk.ptr, dv.ptr, dcs.ptr, dsn.ptr, fx.k.ptr, fx.v.ptr, dt.ptr,
                                          pages, dn.ptr, 5, n, LAYER, fx.nb, None)
    nova.dev_sync()
    hk, hv = fx.hk.copy(), fx.hv.copy()
    got_q = dq.numpy(q.shape, np.float32)
    for i in range(5):
        rq = oracle.rope_kv_store_paged("qwen25_7b", q[i], k[i], v[i], cs, sn, hk, hv,
                                        np.ascontiguousarray(tables[i]), 0, fx.nb, int(n_past[i]))
        assert np.array_equal(got_q[i], rq), i
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv)
