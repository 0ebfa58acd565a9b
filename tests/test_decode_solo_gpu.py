"""Parity of the one-launch ("solo") decode against the CPU oracle.

launch_attn_decode_paged_solo / _rope_solo run one workgroup per (kv head,
session) that streams the session's pages for its head, merges its waves in
LDS and writes the output rows itself (no partials, no combine launch).
Oracle: oracle/nova_oracle.c or_kv_store_paged / or_rope_kv_store_paged
(appended rows bit-exact) and or_attn_decode_paged (restating
src/kernel/attn.cu:163-289,498-512), tolerance max-abs 2e-3 / rel 1e-2; an
f64 textbook softmax bounds the error to fp32 grade as for the split path.
"""
import numpy as np
import pytest

from helpers import PagedFixture, assert_close, f16

pytestmark = pytest.mark.gpu
LAYER = 2


def _solo(nova, fx, q, tables, n_keys, k_new=None, v_new=None):
    n = len(n_keys)
    dq, dt, dn = nova.upload(q), nova.upload(tables), nova.upload(np.asarray(n_keys, np.int32))
    do = nova.alloc(q.nbytes)
    dk = nova.upload(k_new) if k_new is not None else None
    dv = nova.upload(v_new) if v_new is not None else None
    outs = []
    for _ in range(2):   # a repeated call gives the same bits (the append rewrites the same rows)
        nova.dev_zero(do.ptr, do.nbytes, None)
        nova.launch_attn_decode_paged_solo(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, tables.shape[1], dn.ptr, n, LAYER,
                                           fx.nb, dk.ptr if dk else None, dv.ptr if dv else None, do.ptr, None)
        nova.dev_sync()
        outs.append(do.numpy(q.shape, np.float32))
    assert np.array_equal(outs[0], outs[1])
    return outs[0]


def _f64(q, hk, hv, table, n_keys, group):
    pos = np.arange(n_keys)
    k = hk[table[pos >> 4], pos & 15].view(np.float16).astype(np.float64)
    v = hv[table[pos >> 4], pos & 15].view(np.float16).astype(np.float64)
    qh = q.astype(np.float64).reshape(k.shape[1], group, q.shape[-1])
    s = np.einsum("ngd,knd->ngk", qh, k) / np.sqrt(q.shape[-1])
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("ngk,knd->ngd", p, v).reshape(q.shape)


@pytest.mark.parametrize("model", ["qwen25_1p5b", "qwen25_7b", "qwen25_14b"])
def test_solo_fused_append_matches_oracle(model, oracle):
    """Ragged short sessions with the fused append, including page-edge
    lengths (1, 16, 17), config 1's 1025 keys (65 pages: the 65th page lies
    past the 64 table entries read up front) and a session far longer than
    the solo path is meant for (still exact, only slow)."""
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(71)
    n_keys = np.array([1, 16, 17, 1025, 300, 33, 2500, 1536, 1537], np.int32)
    n_sess = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] solo fused model={model} n_keys={n_keys.tolist()}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * max_pages + 5, layer=LAYER, seed=13)
    tables = fx.tables(n_sess, max_pages)
    q = rng.standard_normal((n_sess, nova.nh, nova.hd)).astype(np.float32)
    k_new = f16(rng, (n_sess, nova.nkv, nova.hd))
    v_new = f16(rng, (n_sess, nova.nkv, nova.hd))
    got = _solo(nova, fx, q, tables, n_keys, k_new, v_new)
    hk, hv = fx.hk.copy(), fx.hv.copy()
    for i in range(n_sess):
        oracle.kv_store_paged(model, hk, hv, tables[i], 0, fx.nb, 1, int(n_keys[i]) - 1,
                              np.ascontiguousarray(k_new[i]), np.ascontiguousarray(v_new[i]))
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv), "solo fused append not bit-exact"
    worst = worst64 = 0.0
    for i in range(n_sess):
        ref = oracle.attn_decode_paged(model, np.ascontiguousarray(q[i]), hk, hv, tables[i], 0, fx.nb,
                                       int(n_keys[i]))
        worst = max(worst, assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}"))
        worst64 = max(worst64, float(np.abs(got[i] - _f64(q[i], hk, hv, tables[i], int(n_keys[i]), nova.group)).max()))
    print(f"  worst max|gpu-oracle|={worst:.3e} max|gpu-f64|={worst64:.3e}")
    assert worst64 < 1e-4


def test_solo_empty_session_and_no_append(nova7, oracle):
    """n_keys == 0 gives a zero row; without k_new/v_new the pool is untouched."""
    nova = nova7
    rng = np.random.default_rng(3)
    n_keys = np.array([40, 0, 1, 129], np.int32)
    max_pages = 9
    fx = PagedFixture(nova, nb=4 * max_pages + 2, layer=LAYER, seed=21)
    tables = fx.tables(4, max_pages)
    q = rng.standard_normal((4, nova.nh, nova.hd)).astype(np.float32)
    got = _solo(nova, fx, q, tables, n_keys)
    gk, gv = fx.pull()
    assert np.array_equal(gk, fx.hk) and np.array_equal(gv, fx.hv)
    assert np.all(got[1] == 0.0)
    for i in (0, 2, 3):
        ref = oracle.attn_decode_paged("qwen25_7b", np.ascontiguousarray(q[i]), fx.hk, fx.hv, tables[i], 0,
                                       fx.nb, int(n_keys[i]))
        assert_close(got[i], ref, what=f"session {i}")


def test_solo_matches_split_path(nova7):
    """The solo and the split + combine paths agree on the same step to
    fp32 grade (different summation orders, the same math)."""
    nova = nova7
    rng = np.random.default_rng(5)
    n_keys = rng.integers(1, 1600, 12).astype(np.int32)
    max_pages = int((n_keys.max() + 15) // 16)
    fx = PagedFixture(nova, nb=12 * max_pages + 3, layer=LAYER, seed=9)
    tables = fx.tables(12, max_pages)
    q = rng.standard_normal((12, nova.nh, nova.hd)).astype(np.float32)
    solo = _solo(nova, fx, q, tables, n_keys)
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(12))
    dq, dt, dn = nova.upload(q), nova.upload(tables), nova.upload(n_keys)
    do = nova.alloc(q.nbytes)
    nova.launch_attn_decode_paged_batch(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, max_pages, dn.ptr, 12, LAYER, fx.nb,
                                        None, None, do.ptr, ws.ptr, None)
    nova.dev_sync()
    split = do.numpy(q.shape, np.float32)
    assert float(np.abs(solo - split).max()) < 1e-5


@pytest.mark.parametrize("model", ["qwen25_1p5b", "qwen25_7b"])
def test_solo_rope_fused(model, oracle):
    """launch_attn_decode_paged_rope_solo: RoPE of q and k at n_keys-1, fp16
    append of k and v (bit-exact against or_rope_kv_store_paged) and the
    attention over the rotated q, in one launch."""
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(29)
    n_keys = np.array([1, 17, 1025, 700, 64], np.int32)
    n_sess = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    print(f"[case] solo rope model={model} n_keys={n_keys.tolist()}", flush=True)
    fx = PagedFixture(nova, nb=n_sess * max_pages + 5, layer=LAYER, seed=17)
    tables = fx.tables(n_sess, max_pages)
    half = nova.hd // 2
    dcs, dsn = nova.alloc(4096 * half * 4), nova.alloc(4096 * half * 4)
    nova.launch_rope_table(dcs.ptr, dsn.ptr, None)
    nova.dev_sync()
    cs, sn = dcs.numpy((4096, half), np.float32), dsn.numpy((4096, half), np.float32)
    q = rng.standard_normal((n_sess, nova.nh, nova.hd)).astype(np.float32)
    k = rng.standard_normal((n_sess, nova.nkv, nova.hd)).astype(np.float32)
    v = rng.standard_normal((n_sess, nova.nkv, nova.hd)).astype(np.float32)
    dq, dk, dv = nova.upload(q), nova.upload(k), nova.upload(v)
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    do = nova.alloc(q.nbytes)
    nova.launch_attn_decode_paged_rope_solo(dq.ptr, dk.ptr, dv.ptr, dcs.ptr, dsn.ptr, fx.k.ptr, fx.v.ptr, dt.ptr,
                                            max_pages, dn.ptr, n_sess, LAYER, fx.nb, do.ptr, None)
    nova.dev_sync()
    got = do.numpy(q.shape, np.float32)
    assert np.array_equal(dq.numpy(q.shape, np.float32), q), "caller's q modified"
    hk, hv = fx.hk.copy(), fx.hv.copy()
    rqs = []
    for i in range(n_sess):
        rqs.append(oracle.rope_kv_store_paged(model, q[i][None], k[i][None], v[i][None], cs, sn, hk, hv,
                                              np.ascontiguousarray(tables[i]), 0, fx.nb, int(n_keys[i]) - 1)[0])
    gk, gv = fx.pull()
    assert np.array_equal(gk, hk) and np.array_equal(gv, hv), "solo rope + append not bit-exact"
    worst = 0.0
    for i in range(n_sess):
        ref = oracle.attn_decode_paged(model, np.ascontiguousarray(rqs[i]), hk, hv, tables[i], 0, fx.nb,
                                       int(n_keys[i]))
        worst = max(worst, assert_close(got[i], ref, what=f"session {i} n_keys={n_keys[i]}"))
    print(f"  worst max|gpu-oracle|={worst:.3e}")
