"""Bit-exact parity of the page movers (append, COW copy, clears, table patch)
and of the device-backed session layer against the CPU oracle."""
import ctypes as C

import numpy as np
import pytest

from helpers import PagedFixture, f16

pytestmark = pytest.mark.gpu
LAYER = 2


@pytest.mark.parametrize("n,pos0", [(1, 0), (1, 15), (1, 16), (5, 13), (37, 100), (512, 48)])
def test_kv_store_bit_exact(nova7, oracle, n, pos0):
    nova = nova7
    print(f"[case] kv_store n={n} pos0={pos0}", flush=True)
    pages = (pos0 + n + 15) // 16
    fx = PagedFixture(nova, nb=pages + 3, layer=LAYER, seed=n + pos0)
    table = fx.tables(1, pages)[0]
    k = f16(fx.rng, (n, nova.nkv, nova.hd))
    v = f16(fx.rng, (n, nova.nkv, nova.hd))
    dt, dk, dv = nova.upload(table), nova.upload(k), nova.upload(v)
    nova.launch_kv_store_paged(fx.k.ptr, fx.v.ptr, dt.ptr, LAYER, fx.nb, n, pos0, dk.ptr, dv.ptr, None)
    nova.dev_sync()
    hk, hv = fx.hk.copy(), fx.hv.copy()
    oracle.kv_store_paged("qwen25_7b", hk, hv, table, 0, fx.nb, n, pos0, k, v)
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv)
    # gather through the table returns exactly the appended rows
    got = oracle.kv_gather_paged("qwen25_7b", gk, table, 0, fx.nb, pos0 + n)[pos0:]
    assert np.array_equal(got, k)


def _full_pool(nova, nb, seed):
    """device pool with every layer filled by the seeded testkit generator"""
    per = nova.n_layers * nb * nova.kb * nova.kvw
    k, v = nova.alloc(per * 2), nova.alloc(per * 2)
    nova.testkit_fill_normal_f16(k.ptr, per, seed, 1.0, None)
    nova.testkit_fill_normal_f16(v.ptr, per, seed + 1, 1.0, None)
    nova.dev_sync()
    shape = (nova.n_layers, nb, nova.kb, nova.nkv, nova.hd)
    return k, v, shape


def test_cow_apply_and_zero_pages(nova7, oracle):
    nova = nova7
    nb = 40
    k, v, shape = _full_pool(nova, nb, 77)
    hk, hv = nova.download(k, shape, np.uint16), nova.download(v, shape, np.uint16)
    tables = nova.upload(np.arange(4 * 10, dtype=np.int32))
    ops = [(3, 20, 5), (7, 21, 17), (3, 22, 30)]          # (src, dst, table index)
    arr = (nova_cow_op_t(nova) * len(ops))(*[nova_cow_op_t(nova)(s, d, t) for s, d, t in ops])
    nova.launch_kv_cow_apply(k.ptr, v.ptr, nb, tables.ptr, arr, len(ops), None)
    pages = nova.upload(np.array([9, 11], np.int32))
    nova.launch_kv_zero_pages(k.ptr, v.ptr, nb, pages.ptr, 2, None)
    nova.dev_sync()
    flat_k = hk.reshape(nova.n_layers * nb * nova.kb * nova.kvw)
    flat_v = hv.reshape(flat_k.shape)
    for s, d, _ in ops:
        oracle.cow_copy("qwen25_7b", flat_k, flat_v, nova.n_layers, nb, s, d)
    hk[:, [9, 11]] = 0
    hv[:, [9, 11]] = 0
    assert np.array_equal(nova.download(k, shape, np.uint16), hk)
    assert np.array_equal(nova.download(v, shape, np.uint16), hv)
    t = nova.download(tables, (40,), np.int32)
    want = np.arange(40, dtype=np.int32)
    for s, d, ti in ops:
        want[ti] = d
    assert np.array_equal(t, want)


def nova_cow_op_t(nova):
    import nova_amd
    return nova_amd.CowOp


def test_session_layer_cow_fork(nova7, oracle):
    """Fork at an unaligned prefix (tests/cow_e2e_demo.cpp:39-40): the first
    append of each child copies the shared tail page once, donors are left
    untouched (tests/reuse_demo.cpp:74-75), tables / refcounts / free list match
    the oracle pool driven with the same calls."""
    nova = nova7
    ctx = 256
    h = nova.nova_paged_new(6, ctx)
    try:
        pool = nova.nova_paged_pool(h)
        o = oracle.pool
        oh = o.new(6, ctx)
        nb = nova.nova_paged_nb(h)
        kp, vp = nova.nova_paged_pool_k(h), nova.nova_paged_pool_v(h)
        per = nova.n_layers * nb * nova.kb * nova.kvw
        sess = [nova.nova_paged_create_session(h, 1) for _ in range(3)]
        osess = [o.acquire(oh) for _ in range(3)]
        assert sess == osess
        # a freshly created session's pages are cleared
        shape = (nova.n_layers, nb, nova.kb, nova.nkv, nova.hd)
        assert not nova.download(kp, shape, np.uint16)[:, :3 * (ctx // 16)].any()
        nova.testkit_fill_normal_f16(kp, per, 5, 1.0, None)
        nova.testkit_fill_normal_f16(vp, per, 6, 1.0, None)
        nova.dev_sync()
        before_k = nova.download(kp, shape, np.uint16)
        before_v = nova.download(vp, shape, np.uint16)
        P = 45   # unaligned shared prefix: pages 0..2, tail page 2 half full
        for child in (1, 2):
            nova.nova_paged_attach_prefix(h, child, 0, P)
            o.attach_prefix(oh, child, 0, P)
        st = nova.nova_paged_stream(h)
        ids = (C.c_int * 2)(1, 2)
        pos = (C.c_int64 * 2)(P, P)
        ns = (C.c_int * 2)(3, 3)
        copies = nova.nova_paged_cow_batch(h, ids, pos, ns, 2, st)
        for child in (1, 2):
            o.cow_slice(oh, child, P)
        nova.dev_stream_sync(st)
        assert copies == 2 and nova.nova_kvpool_cow_count(pool) == o.cow_count(oh) == 2
        for s in (0, 1, 2):
            assert table_of(nova, pool, s) == o.table_arr(oh, s)
            dev = nova.download(nova.nova_paged_table_dev(h, s), (ctx // 16,), np.int32)
            assert dev.tolist() == o.table_arr(oh, s)
        assert free_of(nova, pool) == o.free_list_arr(oh)
        assert [nova.nova_kvpool_refcnt(pool, b) for b in range(nb)] == o.refcnt_arr(oh)
        # the copied tails equal the donor's tail in every layer; the donor is untouched
        after_k = nova.download(kp, shape, np.uint16)
        after_v = nova.download(vp, shape, np.uint16)
        donor_tail = o.table_arr(oh, 0)[2]
        for child in (1, 2):
            new = o.table_arr(oh, child)[2]
            assert new != donor_tail
            assert np.array_equal(after_k[:, new], before_k[:, donor_tail])
            assert np.array_equal(after_v[:, new], before_v[:, donor_tail])
        changed = [o.table_arr(oh, c)[2] for c in (1, 2)]
        mask = np.ones(nb, bool)
        mask[changed] = False
        assert np.array_equal(after_k[:, mask], before_k[:, mask])
        assert nova.nova_kvpool_refcnt(pool, donor_tail) == 1
        # a second append into the now-private page copies nothing
        assert nova.nova_paged_cow_batch(h, ids, pos, ns, 2, st) == 0
    finally:
        nova.nova_paged_delete(h)


def table_of(nova, pool, s):
    n = nova.nova_kvpool_table(pool, s, None, 0)
    buf = (C.c_int32 * n)()
    nova.nova_kvpool_table(pool, s, buf, n)
    return list(buf)


def free_of(nova, pool):
    n = nova.nova_kvpool_free_list(pool, None, 0)
    buf = (C.c_int * max(n, 1))()
    nova.nova_kvpool_free_list(pool, buf, n)
    return list(buf[:n])


def test_batched_session_manager(nova7, oracle):
    """create_sessions / push_tables: the ids serial creates would give (oracle
    pool driven with the same acquire/release sequence), exhaustion reported
    as -1, every created session's pages cleared and no other page touched,
    device tables equal to the host tables after host-side attaches pushed in
    one call."""
    nova = nova7
    print("[case] batched session manager", flush=True)
    ctx = 64
    h = nova.nova_paged_new(8, ctx)
    try:
        pool = nova.nova_paged_pool(h)
        o = oracle.pool
        oh = o.new(8, ctx)
        nb = nova.nova_paged_nb(h)
        kp, vp = nova.nova_paged_pool_k(h), nova.nova_paged_pool_v(h)
        shape = (nova.n_layers, nb, nova.kb, nova.nkv, nova.hd)
        per = nova.n_layers * nb * nova.kb * nova.kvw
        first = [nova.nova_paged_create_session(h, 0) for _ in range(3)]
        assert first == [o.acquire(oh) for _ in range(3)]
        nova.nova_paged_destroy_session(h, first[1])
        o.release(oh, first[1])
        nova.testkit_fill_normal_f16(kp, per, 11, 1.0, None)
        nova.testkit_fill_normal_f16(vp, per, 12, 1.0, None)
        nova.dev_sync()
        before_k = nova.download(kp, shape, np.uint16)
        ids = (C.c_int * 7)()
        made = nova.nova_paged_create_sessions(h, 7, 1, ids)
        want = [o.acquire(oh) for _ in range(7)]
        assert made == 6 and list(ids) == [w if w >= 0 else -1 for w in want] and ids[6] == -1
        after_k = nova.download(kp, shape, np.uint16)
        after_v = nova.download(vp, shape, np.uint16)
        cleared = np.zeros(nb, bool)
        for s in list(ids)[:made]:
            cleared[table_of(nova, pool, s)] = True
        assert not after_k[:, cleared].any() and not after_v[:, cleared].any()
        assert np.array_equal(after_k[:, ~cleared], before_k[:, ~cleared])
        live = [first[0], first[2]] + list(ids)[:made]
        for s in live:
            dev = nova.download(nova.nova_paged_table_dev(h, s), (ctx // 16,), np.int32)
            assert dev.tolist() == table_of(nova, pool, s) == o.table_arr(oh, s)
        # host-only attaches (KvPool), then one batched push
        kpool = nova.nova_paged_pool(h)
        targets = list(ids)[:3]
        for t, n_tok in zip(targets, (17, 33, 64)):
            nova.nova_kvpool_attach_prefix(kpool, t, first[0], n_tok)
            o.attach_prefix(oh, t, first[0], n_tok)
        stale = nova.download(nova.nova_paged_table_dev(h, targets[0]), (ctx // 16,), np.int32).tolist()
        assert stale != table_of(nova, pool, targets[0])
        arr = (C.c_int * 3)(targets[2], targets[0], targets[1])
        nova.nova_paged_push_tables(h, arr, 3)
        for s in live:
            dev = nova.download(nova.nova_paged_table_dev(h, s), (ctx // 16,), np.int32)
            assert dev.tolist() == o.table_arr(oh, s)
        o.delete(oh)
    finally:
        nova.nova_paged_delete(h)
