"""Entry points checked against the reference's own known answers and the
oracle's page movers:

* the attention fixtures tests/golden/attn_<model>.npz -- decode at n_past 9
  and prefill of 3 queries at n_past 5, computed by the reference's own SYCL
  attention (src/kernel/sycl/attn.cpp, the cases of tests/sycl_bench.cpp:889-985)
  -- fed straight to launch_attn_decode_paged, the batched decode and
  launch_attn_prefill_paged[_batch];
* launch_kv_store_paged_batch vs or_kv_store_paged (src/kernel/elem.cu:59-98),
  launch_kv_cow_copy vs or_cow_copy and launch_table_patch vs the H2D patch
  of Engine::cow_guard (src/model.cpp:178-190), bit-exact;
* copy-on-write then chunked prefill through the shared tail, the order of
  engine_host.cpp:139 / tests/cow_e2e_demo.cpp:67 (session_cow over the chunk's
  range, append, attend): the chunk's attention matches the oracle and the
  donor's pages and attention are untouched.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from helpers import PagedFixture, assert_close, causal_f64, decode_f64, f16

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
LAYER = 2


def _golden_fixture(nova, g):
    """the fixture's contiguous 32-token cache as pages 1 and 3 of a pool"""
    fx = PagedFixture(nova, nb=5, layer=LAYER, seed=9)
    table = np.array([3, 1], np.int32)
    k = g["k16"].reshape(2, 16, nova.nkv, nova.hd)
    v = g["v16"].reshape(2, 16, nova.nkv, nova.hd)
    fx.hk[table], fx.hv[table] = k, v
    fx.push()
    return fx, table


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b"])
def test_golden_decode_through_hip(model):
    import nova_amd
    nova = nova_amd.load(model)
    g = np.load(GOLDEN / f"attn_{model}.npz")
    fx, table = _golden_fixture(nova, g)
    n_keys = int(g["decode_n_past"]) + 1
    q = np.ascontiguousarray(g["q"])
    dq, dt = nova.upload(q), nova.upload(table)
    scratch = nova.alloc(nova.nh * 32 * (nova.hd + 2) * 4)
    do = nova.alloc(q.nbytes)
    nova.launch_attn_decode_paged(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, LAYER, fx.nb, n_keys, do.ptr, scratch.ptr,
                                  None)
    nova.dev_sync()
    err = assert_close(do.numpy(q.shape, np.float32), g["decode_out"], what=f"{model} golden decode")
    # batched form: the same session twice
    q2 = np.stack([q, q])
    tables = np.stack([table, table])
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(2))
    dq2, dt2, dn = nova.upload(q2), nova.upload(tables), nova.upload(np.array([n_keys, n_keys], np.int32))
    do2 = nova.alloc(q2.nbytes)
    nova.launch_attn_decode_paged_batch(dq2.ptr, fx.k.ptr, fx.v.ptr, dt2.ptr, 2, dn.ptr, 2, LAYER, fx.nb, None,
                                        None, do2.ptr, ws.ptr, None)
    nova.dev_sync()
    got2 = do2.numpy(q2.shape, np.float32)
    for i in range(2):
        assert_close(got2[i], g["decode_out"], what=f"{model} golden batched decode")
    print(f"  {model} max|gpu-golden|={err:.3e}")


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b"])
def test_golden_prefill_through_hip(model):
    import nova_amd
    nova = nova_amd.load(model)
    g = np.load(GOLDEN / f"attn_{model}.npz")
    fx, table = _golden_fixture(nova, g)
    n_q, n_past = int(g["prefill_n_q"]), int(g["prefill_n_past"])
    q = np.ascontiguousarray(g["q_prefill"])
    dq, dt, do = nova.upload(q), nova.upload(table), nova.alloc(q.nbytes)
    nova.launch_attn_prefill_paged(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, LAYER, fx.nb, n_q, n_past, do.ptr, None)
    nova.dev_sync()
    err = assert_close(do.numpy(q.shape, np.float32), g["prefill_out"], what=f"{model} golden prefill")
    dn = nova.upload(np.array([n_past], np.int32))
    do2 = nova.upload(np.full(q.shape, np.nan, np.float32))
    nova.launch_attn_prefill_paged_batch(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, 2, dn.ptr, 1, n_q, LAYER, fx.nb,
                                         do2.ptr, None)
    nova.dev_sync()
    assert_close(do2.numpy(q.shape, np.float32), g["prefill_out"], what=f"{model} golden batched prefill")
    print(f"  {model} max|gpu-golden|={err:.3e}")


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_14b"])
@pytest.mark.parametrize("n", [1, 16, 37, 512])
def test_kv_store_batch_bit_exact(model, n, oracle):
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(n)
    n_sess = 5
    pos0 = rng.integers(0, 300, n_sess).astype(np.int32)
    pos0[0], pos0[1] = 0, 15                      # page-aligned and page-crossing starts
    pages = (pos0 + n + 15) // 16
    print(f"[case] kv_store batch {model} n={n} pos0={pos0.tolist()}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * int(pages.max()) + 4, layer=LAYER, seed=n + 1)
    tables = fx.tables(n_sess, int(pages.max()))
    k = f16(rng, (n_sess, n, nova.nkv, nova.hd))
    v = f16(rng, (n_sess, n, nova.nkv, nova.hd))
    dt, dp, dk, dv = nova.upload(tables), nova.upload(pos0), nova.upload(k), nova.upload(v)
    nova.launch_kv_store_paged_batch(fx.k.ptr, fx.v.ptr, dt.ptr, tables.shape[1], dp.ptr, n_sess, LAYER, fx.nb, n,
                                     dk.ptr, dv.ptr, None)
    nova.dev_sync()
    hk, hv = fx.hk.copy(), fx.hv.copy()
    for i in range(n_sess):
        oracle.kv_store_paged(model, hk, hv, tables[i], 0, fx.nb, n, int(pos0[i]), np.ascontiguousarray(k[i]),
                              np.ascontiguousarray(v[i]))
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv)


def _full_pool(nova, nb, seed):
    per = nova.n_layers * nb * nova.kb * nova.kvw
    k, v = nova.alloc(per * 2), nova.alloc(per * 2)
    nova.testkit_fill_normal_f16(k.ptr, per, seed, 1.0, None)
    nova.testkit_fill_normal_f16(v.ptr, per, seed + 1, 1.0, None)
    nova.dev_sync()
    return k, v, (nova.n_layers, nb, nova.kb, nova.nkv, nova.hd)


@pytest.mark.parametrize("n_pairs", [1, 3, 64, 200])
def test_kv_cow_copy_bit_exact(nova7, oracle, n_pairs):
    nova = nova7
    nb = 2 * n_pairs + 6
    rng = np.random.default_rng(n_pairs)
    k, v, shape = _full_pool(nova, nb, 100 + n_pairs)
    hk, hv = nova.download(k, shape, np.uint16), nova.download(v, shape, np.uint16)
    perm = rng.permutation(nb).astype(np.int32)
    src = np.sort(perm[:n_pairs])[::-1].copy()      # donors need not be ordered
    dst = perm[n_pairs:2 * n_pairs].copy()
    if n_pairs >= 3:
        src[1] = src[2]                               # one donor copied twice (several children of a root)
    ds, dd = nova.upload(src), nova.upload(dst)
    nova.launch_kv_cow_copy(k.ptr, v.ptr, nb, ds.ptr, dd.ptr, n_pairs, None)
    nova.dev_sync()
    fk = hk.reshape(-1)
    fv = hv.reshape(-1)
    for s, d in zip(src, dst):
        oracle.cow_copy("qwen25_7b", fk, fv, nova.n_layers, nb, int(s), int(d))
    assert np.array_equal(nova.download(k, shape, np.uint16), hk)
    assert np.array_equal(nova.download(v, shape, np.uint16), hv)


@pytest.mark.parametrize("n", [1, 5, 300])
def test_table_patch(nova7, n):
    nova = nova7
    rng = np.random.default_rng(n)
    tab = rng.integers(0, 1 << 20, 4 * 512).astype(np.int32)
    idx = rng.choice(tab.size, n, replace=False).astype(np.int32)
    val = rng.integers(0, 1 << 20, n).astype(np.int32)
    dtab, di, dv = nova.upload(tab), nova.upload(idx), nova.upload(val)
    nova.launch_table_patch(dtab.ptr, di.ptr, dv.ptr, n, None)
    nova.dev_sync()
    want = tab.copy()
    want[idx] = val
    assert np.array_equal(dtab.numpy(tab.shape, np.int32), want)


@pytest.mark.parametrize("prefix,n_q", [(45, 40), (2047, 24), (31, 1)])
def test_cow_then_prefill_through_shared_tail(nova7, oracle, prefix, n_q):
    """A child forked at an unaligned prefix runs session_cow over its chunk's
    range, appends the chunk and attends it causally: the output matches the
    oracle over (donor prefix + chunk); the donor's pages and its own decode
    are unchanged; the session layer's tables match the oracle pool."""
    nova = nova7
    model = "qwen25_7b"
    ctx = ((prefix + n_q + 15) // 16 + 1) * 16
    print(f"[case] cow then prefill prefix={prefix} n_q={n_q}", flush=True)
    h = nova.nova_paged_new(4, ctx)
    o = oracle.pool
    oh = o.new(4, ctx)
    try:
        pool = nova.nova_paged_pool(h)
        nb = nova.nova_paged_nb(h)
        kp, vp = nova.nova_paged_pool_k(h), nova.nova_paged_pool_v(h)
        st = nova.nova_paged_stream(h)
        donor = nova.nova_paged_create_session(h, 1)
        child = nova.nova_paged_create_session(h, 1)
        assert [donor, child] == [o.acquire(oh), o.acquire(oh)]
        per = nova.n_layers * nb * nova.kb * nova.kvw
        nova.testkit_fill_normal_f16(kp, per, 61, 1.0, st)
        nova.testkit_fill_normal_f16(vp, per, 62, 1.0, st)
        nova.dev_stream_sync(st)
        shape = (nova.n_layers, nb, nova.kb, nova.nkv, nova.hd)
        before_k, before_v = nova.download(kp, shape, np.uint16), nova.download(vp, shape, np.uint16)
        nova.nova_paged_attach_prefix(h, child, donor, prefix)
        o.attach_prefix(oh, child, donor, prefix)
        # session_cow over [prefix, prefix + n_q): the shared, partly filled tail page is copied once
        nova.nova_paged_session_cow(h, child, prefix, n_q, st)
        for pos in range(prefix, prefix + n_q):
            o.cow_slice(oh, child, pos)
        nova.dev_stream_sync(st)
        assert nova.nova_kvpool_cow_count(pool) == o.cow_count(oh) == 1
        ctab = np.asarray(o.table_arr(oh, child), np.int32)
        dtab_child = nova.nova_paged_table_dev(h, child)
        assert nova.download(dtab_child, (len(ctab),), np.int32).tolist() == ctab.tolist()
        # append the chunk in this layer, then attend it
        rng = np.random.default_rng(prefix + n_q)
        k = f16(rng, (n_q, nova.nkv, nova.hd))
        v = f16(rng, (n_q, nova.nkv, nova.hd))
        dk, dv = nova.upload(k), nova.upload(v)
        nova.launch_kv_store_paged(kp, vp, dtab_child, LAYER, nb, n_q, prefix, dk.ptr, dv.ptr, st)
        q = rng.standard_normal((n_q, nova.nh, nova.hd)).astype(np.float32)
        dq, do = nova.upload(q), nova.alloc(q.nbytes)
        nova.launch_attn_prefill_paged(dq.ptr, kp, vp, dtab_child, LAYER, nb, n_q, prefix, do.ptr, st)
        nova.dev_stream_sync(st)
        got = do.numpy(q.shape, np.float32)
        # expected: the oracle pool image of this layer after COW copy + append
        hk = before_k[LAYER].copy()
        hv = before_v[LAYER].copy()
        lb = (prefix - 1) >> 4 if prefix % 16 else None
        if lb is not None:
            dtab = o.table_arr(oh, donor)
            assert ctab[lb] != dtab[lb]
            hk[ctab[lb]], hv[ctab[lb]] = hk[dtab[lb]], hv[dtab[lb]]
        oracle.kv_store_paged(model, hk, hv, ctab, 0, nb, n_q, prefix, k, v)
        layer_k = nova.download(kp, shape[1:], np.uint16, LAYER * nb * nova.kb * nova.kvw * 2)
        layer_v = nova.download(vp, shape[1:], np.uint16, LAYER * nb * nova.kvw * nova.kb * 2)
        assert np.array_equal(layer_k, hk) and np.array_equal(layer_v, hv)
        ref = oracle.attn_prefill_paged(model, q, hk, hv, ctab, 0, nb, n_q, prefix)
        err = assert_close(got, ref, what="chunk over the copied tail vs oracle")
        assert_close(got, causal_f64(q, hk, hv, ctab, n_q, prefix, nova.group), what="vs f64")
        # the donor: pages untouched in every layer, its decode over its prefix unchanged
        after_k, after_v = nova.download(kp, shape, np.uint16), nova.download(vp, shape, np.uint16)
        dtab = np.asarray(o.table_arr(oh, donor), np.int32)
        assert np.array_equal(after_k[:, dtab], before_k[:, dtab])
        assert np.array_equal(after_v[:, dtab], before_v[:, dtab])
        assert nova.nova_kvpool_refcnt(pool, int(dtab[(prefix - 1) >> 4])) == 1
        qd = rng.standard_normal((nova.nh, nova.hd)).astype(np.float32)
        scratch = nova.alloc(nova.nh * 32 * (nova.hd + 2) * 4)
        dqd, dod = nova.upload(qd), nova.alloc(qd.nbytes)
        nova.launch_attn_decode_paged(dqd.ptr, kp, vp, nova.nova_paged_table_dev(h, donor), LAYER, nb, prefix,
                                      dod.ptr, scratch.ptr, st)
        nova.dev_stream_sync(st)
        assert_close(dod.numpy(qd.shape, np.float32),
                     decode_f64(qd, before_k[LAYER], before_v[LAYER], dtab, prefix, nova.group), what="donor decode")
        # a later append into the now-private tail copies nothing
        nova.nova_paged_session_cow(h, child, prefix + n_q, 1, st)
        assert nova.nova_kvpool_cow_count(pool) == 1
        print(f"  max|gpu-oracle|={err:.3e}")
    finally:
        nova.nova_paged_delete(h)
        o.delete(oh)
