"""Config 3 at full size: copy-on-write prefix sharing through the device-backed
session layer (include/nova_graph.h), checked bit-exact against the C oracle's
KvPool (oracle/nova_oracle.c, restating code/graph/kv_pool.h:56-199) driven
with the same calls, and against the end-to-end invariants of the reference's
tests/cow_e2e_demo.cpp:36-107: exactly one COW per child on its first append
into the unaligned shared tail page, none on any later append, and the donor's
tail page back at refcount 1 once every child has its own copy.

4 roots x 2048 seeded token ids (vocab 151936), 16 children per root forked at
2047 tokens (attach_prefix), suffixes U[0, 1024] appended token by token in
every layer (nova_paged_cow_batch before each step, then
launch_kv_store_paged_batch); kv_block IDs: prefix = kv_hash_ids(root ids up
to the fork), suffix = kv_hash_ids(child ids) ^ 1 (code/graph/kv_block.h:21-64,
the ID convention of INPUT_TOKENIZR.h:69-71 with the child's suffix in place of
the user text).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

VOCAB, ROOT_LEN, FORK = 151936, 2048, 2047
N_ROOTS, PER_ROOT = 4, 16


def _table(nova, pool, s):
    n = nova.nova_kvpool_table(pool, s, None, 0)
    buf = (C.c_int32 * n)()
    nova.nova_kvpool_table(pool, s, buf, n)
    return list(buf)


def _free(nova, pool):
    n = nova.nova_kvpool_free_list(pool, None, 0)
    buf = (C.c_int * max(n, 1))()
    nova.nova_kvpool_free_list(pool, buf, n)
    return list(buf[:n])


def _hash(nova, ids):
    a = np.ascontiguousarray(ids, dtype=np.int32)
    return nova.nova_kv_hash_ids(a.ctypes.data_as(C.POINTER(C.c_int)), len(a))


def test_config3_cow_forks_full_size(nova7, oracle):
    import nova_amd
    nova, orc = nova7, oracle
    rng = np.random.default_rng(3)
    n_child = N_ROOTS * PER_ROOT
    suffix = rng.integers(0, 1025, n_child)
    order = np.argsort(-suffix, kind="stable")      # longest suffix first: the active children are a prefix
    suffix = suffix[order]
    ctx = ROOT_LEN + 1024
    n_slices = N_ROOTS + n_child + 4                # spare slices feed alloc_block
    print(f"[case] config3 cow: {n_child} children, suffix tokens {int(suffix.sum())}", flush=True)
    h = nova.nova_paged_new(n_slices, ctx)
    oh = orc.pool.new(n_slices, ctx)
    try:
        pool = nova.nova_paged_pool(h)
        nb = nova.nova_paged_nb(h)
        nblocks = nova.nova_kvpool_nblocks(pool)
        st = nova.nova_paged_stream(h)
        kp, vp = nova.nova_paged_pool_k(h), nova.nova_paged_pool_v(h)
        sess = [nova.nova_paged_create_session(h, 1) for _ in range(N_ROOTS + n_child)]
        assert sess == [orc.pool.acquire(oh) for _ in range(N_ROOTS + n_child)]
        per_pool = nova.n_layers * nb * nova.kb * nova.kvw
        nova.testkit_fill_normal_f16(kp, per_pool, 31, 1.0, st)
        nova.testkit_fill_normal_f16(vp, per_pool, 32, 1.0, st)
        nova.dev_stream_sync(st)

        # kv_block IDs and the registry
        root_ids = rng.integers(0, VOCAB, (N_ROOTS, ROOT_LEN)).astype(np.int32)
        child_ids = [rng.integers(0, VOCAB, int(n)).astype(np.int32) for n in suffix]
        reg, oreg = nova.nova_registry_new(), orc.registry.new()
        for c in range(n_child):
            root = c % N_ROOTS
            p = _hash(nova, root_ids[root][:FORK])
            assert p == orc.kv_hash_ids(root_ids[root][:FORK].tolist())
            s = _hash(nova, child_ids[c]) ^ 1
            assert s == orc.kv_hash_ids(child_ids[c].tolist()) ^ 1
            out = C.create_string_buffer(40)
            nova.nova_kv_block_id(p, s, out)
            assert out.value.decode() == orc.kv_block_id(p, s)
            args = (p, s, N_ROOTS + c, 1, FORK, FORK + int(suffix[c]))
            nova.nova_registry_put(reg, *args)
            orc.registry.put(oreg, *args)
            assert nova.nova_registry_live(reg) == orc.registry.live(oreg)
            assert nova.nova_registry_total(reg) == orc.registry.total(oreg)
        for c in (0, 17, n_child - 1):
            p = _hash(nova, root_ids[c % N_ROOTS][:FORK])
            s = _hash(nova, child_ids[c]) ^ 1
            a, b, x, y = C.c_int(), C.c_int(), C.c_int64(), C.c_int64()
            ok = nova.nova_registry_find(reg, p, s, C.byref(a), C.byref(b), C.byref(x), C.byref(y))
            want = orc.registry.find_tuple(oreg, p, s)
            assert ((a.value, b.value, x.value, y.value) if ok else None) == want
        nova.nova_registry_delete(reg)
        orc.registry.delete(oreg)

        # fork at the unaligned point: every child shares its root's 128 pages,
        # the last one half full
        layer0 = (nb, nova.kb, nova.nkv, nova.hd)
        before_k = nova.download(kp, layer0, np.uint16)
        before_v = nova.download(vp, layer0, np.uint16)
        for c in range(n_child):
            nova.nova_paged_attach_prefix(h, N_ROOTS + c, c % N_ROOTS, FORK)
            orc.pool.attach_prefix(oh, N_ROOTS + c, c % N_ROOTS, FORK)
        lb = FORK >> 4
        tails = [orc.pool.table_arr(oh, r)[lb] for r in range(N_ROOTS)]
        assert [nova.nova_kvpool_refcnt(pool, t) for t in tails] == [1 + PER_ROOT] * N_ROOTS
        cow0 = nova.nova_kvpool_cow_count(pool)

        # the suffixes, token by token, in every layer
        maxL = int(suffix.max())
        kvn = nova.alloc(nova.n_layers * maxL * n_child * nova.kvw * 2 * 2)
        nova.testkit_fill_normal_f16(kvn.ptr, nova.n_layers * maxL * n_child * nova.kvw * 2, 33, 1.0, st)
        posbuf = nova.upload(np.full(n_child, FORK, np.int32))
        tables_child = nova.nova_paged_tables(h) + N_ROOTS * nblocks * 4
        cow_seq = []
        for step in range(maxL):
            active = int((suffix > step).sum())
            act = (C.c_int * active)(*range(N_ROOTS, N_ROOTS + active))
            ps = (C.c_int64 * active)(*([FORK + step] * active))
            ns = (C.c_int * active)(*([1] * active))
            copies = nova.nova_paged_cow_batch(h, act, ps, ns, active, st)
            for c in range(active):
                orc.pool.cow_slice(oh, N_ROOTS + c, FORK + step)
            assert copies == (active if step == 0 else 0)
            cow_seq.append(nova.nova_kvpool_cow_count(pool))
            pv = np.full(active, FORK + step, np.int32)
            nova.dev_upload_async(posbuf.ptr, pv.ctypes.data, pv.nbytes, st)
            nova.dev_stream_sync(st)
            for layer in range(nova.n_layers):
                base = kvn.ptr + ((layer * maxL + step) * n_child) * nova.kvw * 2 * 2
                nova.launch_kv_store_paged_batch(kp, vp, tables_child, nblocks, posbuf.ptr, active, layer, nb, 1,
                                                 base, base + n_child * nova.kvw * 2, st)
        nova.dev_stream_sync(st)

        # cow_e2e_demo invariants: one COW per child (all on the first append), none later
        first_cow = int((suffix > 0).sum())
        assert cow_seq[0] - cow0 == first_cow
        assert all(v == cow_seq[0] for v in cow_seq)
        assert nova.nova_kvpool_cow_count(pool) == orc.pool.cow_count(oh) == first_cow
        # the donors' tail pages: shared by the children that never appended
        for r in range(N_ROOTS):
            still = sum(1 for c in range(n_child) if c % N_ROOTS == r and suffix[c] == 0)
            assert nova.nova_kvpool_refcnt(pool, tails[r]) == 1 + still
        # tables (host and device), refcounts and free list bit-exact vs the oracle pool
        for s in sess:
            assert _table(nova, pool, s) == orc.pool.table_arr(oh, s)
        dev_tables = nova.download(nova.nova_paged_tables(h), (n_slices, nblocks), np.int32)
        for s in sess:
            assert dev_tables[s].tolist() == orc.pool.table_arr(oh, s)
        assert [nova.nova_kvpool_refcnt(pool, b) for b in range(nb)] == orc.pool.refcnt_arr(oh)
        assert _free(nova, pool) == orc.pool.free_list_arr(oh)

        # data: a child sees its root's prefix, then its own suffix, in every layer
        # checked (0 and the last); the donors' pages are untouched
        kv_all = nova.download(kvn, (nova.n_layers, maxL, 2, n_child, nova.nkv, nova.hd), np.uint16)
        for layer in (0, nova.n_layers - 1):
            off = layer * nb * nova.kb * nova.kvw * 2
            ak = nova.download(kp, layer0, np.uint16, off)
            av = nova.download(vp, layer0, np.uint16, off)
            if layer == 0:
                bk, bv = before_k, before_v
            else:
                bk = bv = None
            for c in range(n_child):
                child, root = N_ROOTS + c, c % N_ROOTS
                n_tok = FORK + int(suffix[c])
                tab = np.asarray(orc.pool.table_arr(oh, child), np.int32)
                gk = orc.kv_gather_paged("qwen25_7b", ak, tab, 0, nb, n_tok)
                gv = orc.kv_gather_paged("qwen25_7b", av, tab, 0, nb, n_tok)
                rtab = np.asarray(orc.pool.table_arr(oh, root), np.int32)
                assert np.array_equal(gk[:FORK], orc.kv_gather_paged("qwen25_7b", ak, rtab, 0, nb, FORK))
                assert np.array_equal(gv[:FORK], orc.kv_gather_paged("qwen25_7b", av, rtab, 0, nb, FORK))
                if suffix[c]:
                    assert np.array_equal(gk[FORK:], kv_all[layer, :suffix[c], 0, c])
                    assert np.array_equal(gv[FORK:], kv_all[layer, :suffix[c], 1, c])
            if bk is not None:
                for r in range(N_ROOTS):
                    for p in orc.pool.table_arr(oh, r):
                        assert np.array_equal(ak[p], bk[p]) and np.array_equal(av[p], bv[p])
    finally:
        nova.nova_paged_delete(h)
        orc.pool.delete(oh)
