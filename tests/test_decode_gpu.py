"""Parity of the gfx950 split-K paged decode against the CPU oracle.

Oracle: oracle/nova_oracle.c or_attn_decode_paged (restating
src/kernel/attn.cu:163-289,498-512) and its f64 textbook softmax.  Tolerance:
max-abs 2e-3 / rel 1e-2 (task statement); the measured error is printed.
"""
import numpy as np
import pytest

from helpers import PagedFixture, assert_close, f16

pytestmark = pytest.mark.gpu
LAYER = 3


def _decode_single(nova, fx, q, table, n_keys):
    scratch = nova.alloc(nova.nh * 32 * (nova.hd + 2) * 4)
    dq = nova.upload(q)
    dt = nova.upload(table)
    do = nova.alloc(q.nbytes)
    nova.launch_attn_decode_paged(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, LAYER, fx.nb, n_keys, do.ptr,
                                  scratch.ptr, None)
    nova.dev_sync()
    return do.numpy(q.shape, np.float32)


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b", "qwen25_14b"])
@pytest.mark.parametrize("n_keys", [1, 2, 15, 16, 17, 33, 100, 1025, 4000])
def test_decode_single_matches_oracle(model, n_keys, oracle):
    import nova_amd
    nova = nova_amd.load(model)
    print(f"[case] decode single model={model} n_keys={n_keys}", flush=True)
    max_pages = (n_keys + 15) // 16
    fx = PagedFixture(nova, nb=max(max_pages + 3, 8), layer=LAYER, seed=n_keys)
    table = fx.tables(1, max_pages)[0]
    q = fx.rng.standard_normal((nova.nh, nova.hd)).astype(np.float32)
    got = _decode_single(nova, fx, q, table, n_keys)
    ref = oracle.attn_decode_paged(model, q, fx.hk, fx.hv, table, 0, fx.nb, n_keys)
    err = assert_close(got, ref, what=f"{model} n_keys={n_keys}")
    ref64 = oracle.attn_decode_paged(model, q, fx.hk, fx.hv, table, 0, fx.nb, n_keys, f64=True)
    err64 = float(np.abs(got - ref64).max())
    print(f"  max|gpu-oracle|={err:.3e} max|gpu-f64|={err64:.3e}")
    assert err64 < 1e-4   # fp32-grade: the hi/lo fp16 splits keep ~2^-22 per operand


def test_decode_single_key_is_v(nova7, oracle):
    """n_keys == 1 => O[h] == V[kvh] exactly up to rounding (tests/gpu_misc.cu:41-65)."""
    nova = nova7
    fx = PagedFixture(nova, nb=4, layer=LAYER, seed=7)
    table = np.array([2], np.int32)
    q = np.full((nova.nh, nova.hd), 0.5, np.float32)
    got = _decode_single(nova, fx, q, table, 1)
    v = fx.hv[2, 0].view(np.float16).astype(np.float32)    # [NKV][HD]
    want = np.repeat(v, nova.group, axis=0)
    assert np.abs(got - want).max() <= 1e-6


def _batch(nova, fx, q, tables, n_keys, k_new=None, v_new=None):
    n = len(n_keys)
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n))
    nova.dev_zero(ws.ptr, ws.nbytes, None)
    dq, dt, dn = nova.upload(q), nova.upload(tables), nova.upload(np.asarray(n_keys, np.int32))
    do = nova.alloc(q.nbytes)
    dk = nova.upload(k_new) if k_new is not None else None
    dv = nova.upload(v_new) if v_new is not None else None
    outs = []
    for _ in range(2):   # a repeated call must give the same bits
        nova.launch_attn_decode_paged_batch(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, tables.shape[1], dn.ptr, n,
                                            LAYER, fx.nb, dk.ptr if dk else None, dv.ptr if dv else None,
                                            do.ptr, ws.ptr, None)
        nova.dev_sync()
        outs.append(do.numpy(q.shape, np.float32))
        assert nova.attn_decode_batch_status(ws.ptr, n) == 0   # no exchange gave up
    assert np.array_equal(outs[0], outs[1])
    return outs[0]


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b", "qwen25_14b"])
def test_decode_batch_ragged_fused_append(model, oracle):
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(11)
    n_sess = 16
    n_keys = rng.integers(1, 700, n_sess).astype(np.int32)
    n_keys[3] = 1
    n_keys[5] = 16
    n_keys[6] = 17
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] decode batch fused model={model} n_keys={n_keys.tolist()}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * max_pages + 5, layer=LAYER, seed=5)
    tables = fx.tables(n_sess, max_pages)
    q = rng.standard_normal((n_sess, nova.nh, nova.hd)).astype(np.float32)
    k_new = f16(rng, (n_sess, nova.nkv, nova.hd))
    v_new = f16(rng, (n_sess, nova.nkv, nova.hd))
    got = _batch(nova, fx, q, tables, n_keys, k_new, v_new)
    # oracle: append (kv_store_paged at pos n_keys-1), then decode each session
    hk, hv = fx.hk.copy(), fx.hv.copy()
    for i in range(n_sess):
        oracle.kv_store_paged(model, hk, hv, tables[i], 0, fx.nb, 1, int(n_keys[i]) - 1,
                              np.ascontiguousarray(k_new[i]), np.ascontiguousarray(v_new[i]))
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv), "fused append not bit-exact"
    worst = 0.0
    for i in range(n_sess):
        ref = oracle.attn_decode_paged(model, np.ascontiguousarray(q[i]), hk, hv, tables[i], 0, fx.nb,
                                       int(n_keys[i]))
        worst = max(worst, assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}"))
    print(f"  worst max|gpu-oracle|={worst:.3e}")


def test_decode_batch_skewed_xcd_homes(nova7, oracle):
    """One long session and 39 one-page sessions: the split workgroups fill
    XCDs in logical order, so most sessions share two XCDs and their combine
    blocks overflow onto the other XCDs' free blocks."""
    nova = nova7
    rng = np.random.default_rng(41)
    n_keys = np.concatenate([[3000], rng.integers(1, 17, 39)]).astype(np.int32)
    n_sess = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] decode batch skewed homes n_sess={n_sess}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * max_pages + 3, layer=LAYER, seed=41)
    tables = fx.tables(n_sess, max_pages)
    q = rng.standard_normal((n_sess, nova.nh, nova.hd)).astype(np.float32)
    got = _batch(nova, fx, q, tables, n_keys)
    worst = 0.0
    for i in range(n_sess):
        ref = oracle.attn_decode_paged("qwen25_7b", np.ascontiguousarray(q[i]), fx.hk, fx.hv, tables[i], 0,
                                       fx.nb, int(n_keys[i]))
        worst = max(worst, assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}"))
    print(f"  worst max|gpu-oracle|={worst:.3e}")


def test_decode_batch_empty_session_and_no_append(nova7, oracle):
    nova = nova7
    n_keys = np.array([40, 0, 1, 0, 300], np.int32)
    fx = PagedFixture(nova, nb=5 * 19 + 2, layer=LAYER, seed=9)
    tables = fx.tables(5, 19)
    q = fx.rng.standard_normal((5, nova.nh, nova.hd)).astype(np.float32)
    got = _batch(nova, fx, q, tables, n_keys)
    for i in range(5):
        if n_keys[i] == 0:
            assert (got[i] == 0).all()
        else:
            ref = oracle.attn_decode_paged("qwen25_7b", np.ascontiguousarray(q[i]), fx.hk, fx.hv, tables[i],
                                           0, fx.nb, int(n_keys[i]))
            assert_close(got[i], ref)


def test_decode_plan_reused_across_layers(nova7, oracle):
    """one plan per step, planned calls for several layers (bench.py's step)"""
    nova = nova7
    n_keys = np.array([700, 33, 1, 2048, 15, 300], np.int32)
    n = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    nb = n * max_pages + 4
    rng = np.random.default_rng(12)
    per_pool = nova.n_layers * nb * nova.kb * nova.kvw
    k, v = nova.alloc(per_pool * 2), nova.alloc(per_pool * 2)
    nova.testkit_fill_normal_f16(k.ptr, per_pool, 91, 1.0, None)
    nova.testkit_fill_normal_f16(v.ptr, per_pool, 92, 1.0, None)
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.ascontiguousarray(perm[: n * max_pages].reshape(n, max_pages))
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n))
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    nova.launch_attn_decode_plan(dt.ptr, max_pages, dn.ptr, n, ws.ptr, None)
    shape = (nb, nova.kb, nova.nkv, nova.hd)
    for layer in (0, 7, 27):
        q = rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
        dq, do = nova.upload(q), nova.alloc(q.nbytes)
        nova.launch_attn_decode_paged_planned(dq.ptr, k.ptr, v.ptr, dt.ptr, max_pages, n, layer, nb, None, None,
                                              do.ptr, ws.ptr, None)
        nova.dev_sync()
        got = do.numpy(q.shape, np.float32)
        off = layer * nb * nova.kb * nova.kvw * 2
        hk = nova.download(k.ptr + off, shape, np.uint16)
        hv = nova.download(v.ptr + off, shape, np.uint16)
        for i in range(n):
            ref = oracle.attn_decode_paged("qwen25_7b", np.ascontiguousarray(q[i]), hk, hv, tables[i], 0, nb,
                                           int(n_keys[i]))
            assert_close(got[i], ref, what=f"layer {layer} session {i}")


def test_decode_batch_many_sessions(nova7, oracle):
    """300 ragged sessions (some empty): more sessions than one wave's 64-lane
    passes over the batch and than the 256-workgroup grid base."""
    nova = nova7
    rng = np.random.default_rng(31)
    n_sess = 300
    n_keys = rng.integers(0, 300, n_sess).astype(np.int32)
    n_keys[::37] = 0
    n_keys[5] = 1
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] decode batch n_sess={n_sess}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * max_pages + 3, layer=LAYER, seed=31)
    tables = fx.tables(n_sess, max_pages)
    q = rng.standard_normal((n_sess, nova.nh, nova.hd)).astype(np.float32)
    got = _batch(nova, fx, q, tables, n_keys)
    worst = 0.0
    for i in range(n_sess):
        if n_keys[i] == 0:
            assert (got[i] == 0).all(), i
            continue
        ref = oracle.attn_decode_paged("qwen25_7b", np.ascontiguousarray(q[i]), fx.hk, fx.hv, tables[i], 0, fx.nb,
                                       int(n_keys[i]))
        worst = max(worst, assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}"))
    print(f"  worst max|gpu-oracle|={worst:.3e}")


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b", "qwen25_14b"])
def test_decode_batch_rope_fused(model, oracle):
    """launch_attn_decode_paged_rope_batch = RopeKvOp (rope of q and k at
    n_keys-1, fp16 append of k and v) + the batched decode: appended rows
    bit-exact against or_rope_kv_store_paged, the output within tolerance of
    the oracle's decode over the rotated q, the caller's q untouched, and the
    rotation really applied (the unrotated result differs)."""
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(23)
    n_sess = 16
    n_keys = rng.integers(1, 900, n_sess).astype(np.int32)
    n_keys[2], n_keys[7], n_keys[9] = 1, 16, 17
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] decode batch rope fused model={model} n_keys={n_keys.tolist()}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * max_pages + 5, layer=LAYER, seed=8)
    tables = fx.tables(n_sess, max_pages)
    half = nova.hd // 2
    dcs, dsn = nova.alloc(4096 * half * 4), nova.alloc(4096 * half * 4)
    nova.launch_rope_table(dcs.ptr, dsn.ptr, None)
    nova.dev_sync()
    cs, sn = dcs.numpy((4096, half), np.float32), dsn.numpy((4096, half), np.float32)
    q = rng.standard_normal((n_sess, nova.nh, nova.hd)).astype(np.float32)
    k = rng.standard_normal((n_sess, nova.nkv, nova.hd)).astype(np.float32)
    v = rng.standard_normal((n_sess, nova.nkv, nova.hd)).astype(np.float32)
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n_sess))
    dq, dk, dv = nova.upload(q), nova.upload(k), nova.upload(v)
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    do = nova.alloc(q.nbytes)
    nova.launch_attn_decode_paged_rope_batch(dq.ptr, dk.ptr, dv.ptr, dcs.ptr, dsn.ptr, fx.k.ptr, fx.v.ptr, dt.ptr,
                                             max_pages, dn.ptr, n_sess, LAYER, fx.nb, do.ptr, ws.ptr, None)
    nova.dev_sync()
    got = do.numpy(q.shape, np.float32)
    assert np.array_equal(dq.numpy(q.shape, np.float32), q), "caller's q modified"
    hk, hv = fx.hk.copy(), fx.hv.copy()
    rqs = []
    for i in range(n_sess):
        rqs.append(oracle.rope_kv_store_paged(model, q[i][None], k[i][None], v[i][None], cs, sn, hk, hv,
                                              np.ascontiguousarray(tables[i]), 0, fx.nb, int(n_keys[i]) - 1)[0])
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv), "fused rope + append not bit-exact"
    worst = 0.0
    for i in range(n_sess):
        ref = oracle.attn_decode_paged(model, np.ascontiguousarray(rqs[i]), hk, hv, tables[i], 0, fx.nb,
                                       int(n_keys[i]))
        worst = max(worst, assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}"))
        if n_keys[i] > 1:
            plain = oracle.attn_decode_paged(model, np.ascontiguousarray(q[i]), hk, hv, tables[i], 0, fx.nb,
                                             int(n_keys[i]))
            assert np.abs(plain - ref).max() > 1e-3, "rotation had no effect"
    print(f"  worst max|gpu-oracle|={worst:.3e}")


def _decode_f64(q, hk, hv, table, n_keys, group):
    """Textbook softmax attention in float64 for one session (the reference the
    C oracle is pinned to), vectorised for very long contexts."""
    pos = np.arange(n_keys)
    k = hk[table[pos >> 4], pos & 15].view(np.float16).astype(np.float64)   # [n_keys][NKV][HD]
    v = hv[table[pos >> 4], pos & 15].view(np.float16).astype(np.float64)
    qh = q.astype(np.float64).reshape(k.shape[1], group, q.shape[-1])          # [NKV][G][HD]
    s = np.einsum("ngd,knd->ngk", qh, k) / np.sqrt(q.shape[-1])
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("ngk,knd->ngd", p, v).reshape(q.shape)


def test_decode_long_ranges():
    """Split workgroups that own more than 64 pages reload their block-table
    slice while they stream: the single-session entry point from ~32K keys
    (at most 31 splits), the batched one once the batch exceeds 256 x 64
    pages (share > 64)."""
    import nova_amd
    nova = nova_amd.load("qwen25_1p5b")
    n_keys = np.array([140000, 130001], np.int32)
    pages = (n_keys + 15) // 16
    print(f"[case] decode long ranges n_keys={n_keys.tolist()} pages={int(pages.sum())}", flush=True)
    assert int(pages.sum()) > 256 * 64
    fx = PagedFixture(nova, nb=2 * int(pages.max()) + 4, layer=LAYER, seed=41)
    tables = fx.tables(2, int(pages.max()))
    q = fx.rng.standard_normal((2, nova.nh, nova.hd)).astype(np.float32)
    ref = [_decode_f64(q[i], fx.hk, fx.hv, tables[i], int(n_keys[i]), nova.group) for i in range(2)]
    got = _batch(nova, fx, q, tables, n_keys)
    for i in range(2):
        assert_close(got[i], ref[i], what=f"batched session {i}")
    one = _decode_single(nova, fx, np.ascontiguousarray(q[1]), np.ascontiguousarray(tables[1]), 40000)
    assert_close(one, _decode_f64(q[1], fx.hk, fx.hv, tables[1], 40000, nova.group), what="single 40000 keys")


def test_stream_floor_reads_the_planned_pairs(nova7):
    """testkit_decode_stream_floor (the bench's HBM floor of the planned split)
    reads, in every workgroup slot of the plan and every wave, exactly the page
    pairs that wave of the split kernel reads: with pools of fp16 words 0x0001
    each thread's sink word is 64 * 0x00010001 per pair it loaded."""
    nova = nova7
    n_keys = np.array([700, 33, 1, 2048, 15, 300, 4100, 0, 129], np.int32)
    n = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    nb = n * max_pages + 4
    rng = np.random.default_rng(31)
    page = nova.kb * nova.kvw
    ones = np.ones(nb * page, np.uint16)
    k, v = nova.upload(ones), nova.upload(ones)       # layer 0 only
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.ascontiguousarray(perm[: n * max_pages].reshape(n, max_pages))
    ws_bytes = nova.attn_decode_batch_workspace_bytes(n)
    ws = nova.alloc(ws_bytes)
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    nova.launch_attn_decode_plan(dt.ptr, max_pages, dn.ptr, n, ws.ptr, None)
    nova.testkit_decode_stream_floor(k.ptr, v.ptr, dt.ptr, max_pages, n, 0, nb, ws.ptr, None)
    nova.dev_sync()
    # workspace = plan (session table, combine map, slot records, status
    # word; rounded to 256 B) + slots * R * NH * PW floats, PW = HD + 4
    R, PW, rec = 8 // nova.nkv, nova.hd + 4, 72
    rec_off = n * 4 + n * nova.nh * 4
    slots = [s for s in range(1, 4096)
             if -(-(rec_off + s * rec + 1) * 4 // 256) * 256 + s * R * nova.nh * PW * 4 == ws_bytes]
    assert len(slots) == 1, slots
    slots = slots[0]
    plan_b = ws_bytes - slots * R * nova.nh * PW * 4
    plan = nova.download(ws, (plan_b // 4,), np.int32)
    sink = nova.download(ws, (slots, 512), np.uint32, plan_b)
    per_pair = 64 * 0x00010001
    covered = [np.zeros(int((nk + 15) // 16), np.int32) for nk in n_keys]
    for w in range(slots):
        r0 = rec_off + w * rec
        sess, pa, pb = plan[r0 + 64], plan[r0 + 65], plan[r0 + 66]
        if sess < 0:          # idle slot
            continue
        assert (plan[r0:r0 + min(64, pb - pa)] == tables[sess, pa:pb][:64]).all()
        covered[sess][pa:pb] += 1
        npairs = (pb - pa + 1) // 2
        for wave in range(8):
            r = wave // nova.nkv
            want = len(range(r, npairs, R)) * per_pair
            assert (sink[w, 64 * wave:64 * wave + 64] == want).all(), (w, wave)
    for i in range(n):
        assert (covered[i] == 1).all(), i


def test_decode_exchange_give_up_is_reported(nova7, oracle):
    """The bounded LDS wait of the one-slot partial exchange (7B: two waves per
    kv head) never gives up silently.  The test kit's copy of the planned call
    sets the bound to 0 polls, so every exchange gives up (forced from the
    host; every kernel still exits normally): the status word reads 1 and the
    outputs are NaN.  The next plan clears the word, and the product call is
    then correct with status 0."""
    nova = nova7
    assert nova.testkit is not None, "test kit library not built"
    n_keys = np.array([300, 40, 1000], np.int32)
    n = len(n_keys)
    pages = (n_keys + 15) // 16
    fx = PagedFixture(nova, nb=n * int(pages.max()) + 4, layer=LAYER, seed=91)
    tables = fx.tables(n, int(pages.max()))
    q = fx.rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n))
    dq, dt, dn = nova.upload(q), nova.upload(tables), nova.upload(n_keys)
    do = nova.alloc(q.nbytes)
    print("[case] decode exchange give-up forced (spin 0), 7B, 3 sessions", flush=True)
    nova.launch_attn_decode_plan(dt.ptr, tables.shape[1], dn.ptr, n, ws.ptr, None)
    nova.testkit_attn_decode_planned_spin(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, tables.shape[1], n, LAYER, fx.nb,
                                          None, None, do.ptr, ws.ptr, 0, None)
    nova.dev_sync()
    assert nova.attn_decode_batch_status(ws.ptr, n) == 1
    assert np.isnan(do.numpy(q.shape, np.float32)).all()
    print("[case] decode after a give-up: plan clears the status", flush=True)
    nova.launch_attn_decode_plan(dt.ptr, tables.shape[1], dn.ptr, n, ws.ptr, None)
    assert nova.attn_decode_batch_status(ws.ptr, n) == 0
    nova.testkit_attn_decode_planned_spin(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, tables.shape[1], n, LAYER, fx.nb,
                                          None, None, do.ptr, ws.ptr, 1 << 22, None)
    nova.dev_sync()
    assert nova.attn_decode_batch_status(ws.ptr, n) == 0
    got = do.numpy(q.shape, np.float32)
    for i in range(n):
        ref = oracle.attn_decode_paged("qwen25_7b", q[i], fx.hk, fx.hv, tables[i], 0, fx.nb, int(n_keys[i]))
        assert_close(got[i], ref, what=f"session {i} after give-up")


@pytest.mark.parametrize("n_keys", [[1000], [1009, 77], [4001, 33, 250]])
def test_decode_batch_uneven_ranges_1p5b(n_keys, oracle):
    """1.5B (four waves per kv head, a partial slot per wave row): the combine
    reads only the rows that can hold a page pair, ceil(ceil(P/k)/2) per split
    workgroup.  Page counts that k does not divide give ranges of unequal
    length (e.g. 63 pages over 16 workgroups); every one of them must be
    read."""
    import nova_amd
    nova = nova_amd.load("qwen25_1p5b")
    n_keys = np.asarray(n_keys, np.int32)
    n = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] decode batch uneven ranges 1.5B n_keys={n_keys.tolist()}", flush=True)
    fx = PagedFixture(nova, nb=n * max_pages + 3, layer=LAYER, seed=int(n_keys.sum()))
    tables = fx.tables(n, max_pages)
    q = fx.rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
    got = _batch(nova, fx, q, tables, n_keys)
    for i in range(n):
        ref = oracle.attn_decode_paged("qwen25_1p5b", np.ascontiguousarray(q[i]), fx.hk, fx.hv, tables[i], 0,
                                       fx.nb, int(n_keys[i]))
        assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}")


@pytest.mark.parametrize("model", ["qwen25_1p5b", "qwen25_7b", "qwen25_14b"])
@pytest.mark.parametrize("n_keys", [1, 17, 1025, 3000])
def test_decode_batch_one_session(model, n_keys, oracle):
    """A batched call with one session takes the single-session split kernel
    (query and new-token rows loaded beside the plan record): fused append
    bit-exact, output against the oracle and f64, repeated calls identical."""
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(n_keys)
    pages = (n_keys + 15) // 16
    print(f"[case] decode one session model={model} n_keys={n_keys}", flush=True)
    fx = PagedFixture(nova, nb=pages + 4, layer=LAYER, seed=n_keys + 3)
    tables = fx.tables(1, pages)
    q = rng.standard_normal((1, nova.nh, nova.hd)).astype(np.float32)
    k_new = f16(rng, (1, nova.nkv, nova.hd))
    v_new = f16(rng, (1, nova.nkv, nova.hd))
    got = _batch(nova, fx, q, tables, np.array([n_keys], np.int32), k_new, v_new)
    hk, hv = fx.hk.copy(), fx.hv.copy()
    oracle.kv_store_paged(model, hk, hv, tables[0], 0, fx.nb, 1, n_keys - 1, np.ascontiguousarray(k_new[0]),
                          np.ascontiguousarray(v_new[0]))
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv), "fused append not bit-exact"
    ref = oracle.attn_decode_paged(model, np.ascontiguousarray(q[0]), hk, hv, tables[0], 0, fx.nb, n_keys)
    err = assert_close(got[0], ref, what=f"{model} one session n_keys={n_keys}")
    err64 = float(np.abs(got[0] - _decode_f64(q[0], hk, hv, tables[0], n_keys, nova.group)).max())
    print(f"  max|gpu-oracle|={err:.3e} max|gpu-f64|={err64:.3e}")
    assert err64 < 1e-4


@pytest.mark.parametrize("model", ["qwen25_1p5b", "qwen25_7b"])
def test_decode_rope_one_session(model, oracle):
    """launch_attn_decode_paged_rope_batch with one session (the single-session
    split kernel with RoPE fused): rows bit-exact, output within tolerance."""
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(31)
    n_keys = np.array([777], np.int32)
    pages = int((n_keys[0] + 15) // 16)
    fx = PagedFixture(nova, nb=pages + 4, layer=LAYER, seed=12)
    tables = fx.tables(1, pages)
    half = nova.hd // 2
    dcs, dsn = nova.alloc(4096 * half * 4), nova.alloc(4096 * half * 4)
    nova.launch_rope_table(dcs.ptr, dsn.ptr, None)
    nova.dev_sync()
    cs, sn = dcs.numpy((4096, half), np.float32), dsn.numpy((4096, half), np.float32)
    q = rng.standard_normal((1, nova.nh, nova.hd)).astype(np.float32)
    k = rng.standard_normal((1, nova.nkv, nova.hd)).astype(np.float32)
    v = rng.standard_normal((1, nova.nkv, nova.hd)).astype(np.float32)
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(1))
    dq, dk, dv, dt, dn = nova.upload(q), nova.upload(k), nova.upload(v), nova.upload(tables), nova.upload(n_keys)
    do = nova.alloc(q.nbytes)
    nova.launch_attn_decode_paged_rope_batch(dq.ptr, dk.ptr, dv.ptr, dcs.ptr, dsn.ptr, fx.k.ptr, fx.v.ptr, dt.ptr,
                                             pages, dn.ptr, 1, LAYER, fx.nb, do.ptr, ws.ptr, None)
    nova.dev_sync()
    got = do.numpy(q.shape, np.float32)
    hk, hv = fx.hk.copy(), fx.hv.copy()
    rq = oracle.rope_kv_store_paged(model, q, k, v, cs, sn, hk, hv, np.ascontiguousarray(tables[0]), 0, fx.nb,
                                    int(n_keys[0]) - 1)[0]
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv), "fused rope + append not bit-exact"
    ref = oracle.attn_decode_paged(model, np.ascontiguousarray(rq), hk, hv, tables[0], 0, fx.nb, int(n_keys[0]))
    assert_close(got[0], ref, what=f"{model} rope one session")
