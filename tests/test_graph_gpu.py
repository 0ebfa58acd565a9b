"""HIP-graph replays of the hot path equal its eager run.

The benchmark replays whole decode steps, prefill layers and GEMV layers from
HIP graphs.  A captured graph must hold no memset node (only fill kernels), so
replays after the first see the same state; each test captures a step, replays
it several times with unrelated eager work and synchronisations in between,
and requires every replay to reproduce the eager outputs bit for bit (the
appends rewrite the same slots with the same bits, so a step is idempotent).
"""
import ctypes as C

import numpy as np
import pytest

from helpers import PagedFixture, f16

pytestmark = pytest.mark.gpu
LAYERS = (0, 3, 7)


def _replays(nova, s, run, read, n=4):
    """eager run, then n graph replays of the same launches; returns outputs"""
    run()
    nova.dev_stream_sync(s)
    eager = read()
    nova.dev_graph_begin(s)
    run()
    g = nova.dev_graph_end(s)
    junk = nova.alloc(1 << 20)
    outs = []
    try:
        for r in range(n):
            nova.dev_zero(junk.ptr, junk.nbytes, s)          # unrelated eager work between replays
            nova.dev_stream_sync(s)
            nova.dev_graph_launch(g, s)
            nova.dev_stream_sync(s)
            outs.append(read())
    finally:
        nova.dev_graph_destroy(g)
    return eager, outs


def _fill_layers(fx, layers):
    """seeded fp16 pages in every layer a test reads (the fixture fills one)"""
    for layer in layers:
        off = layer * fx.nb * fx.page_halves * 2
        fx.nova.dev_upload(fx.k.ptr + off, fx.hk.ctypes.data, fx.hk.nbytes)
        fx.nova.dev_upload(fx.v.ptr + off, fx.hv.ctypes.data, fx.hv.nbytes)


def test_decode_step_graph(nova7):
    """plan + fused-append decode of three layers for 6 ragged sessions"""
    nova = nova7
    print("[case] graph decode step", flush=True)
    n_keys = np.array([700, 1, 33, 2048, 16, 300], np.int32)
    n = len(n_keys)
    pages = int((n_keys.max() + 15) // 16)
    fx = PagedFixture(nova, nb=n * pages + 3, layer=LAYERS[0], seed=12)
    tables = fx.tables(n, pages)
    rng = np.random.default_rng(5)
    q = nova.upload(rng.standard_normal((len(LAYERS), n, nova.nh, nova.hd)).astype(np.float32))
    kn = nova.upload(f16(rng, (len(LAYERS), n, nova.nkv, nova.hd)))
    vn = nova.upload(f16(rng, (len(LAYERS), n, nova.nkv, nova.hd)))
    o = nova.upload(np.full((len(LAYERS), n, nova.nh, nova.hd), np.nan, np.float32))
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n))
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    s = nova.dev_stream_create()
    qs, kvs = n * nova.nh * nova.hd, n * nova.kvw

    def run():
        nova.launch_attn_decode_plan(dt.ptr, pages, dn.ptr, n, ws.ptr, s)
        for i, layer in enumerate(LAYERS):
            nova.launch_attn_decode_paged_planned(q.ptr + i * qs * 4, fx.k.ptr, fx.v.ptr, dt.ptr, pages, n, layer,
                                                  fx.nb, kn.ptr + i * kvs * 2, vn.ptr + i * kvs * 2,
                                                  o.ptr + i * qs * 4, ws.ptr, s)

    eager, outs = _replays(nova, s, run, lambda: o.numpy((len(LAYERS), n, nova.nh, nova.hd), np.float32))
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"


def test_decode_rope_step_graph(nova7):
    """the fused RoPE + append + decode step"""
    nova = nova7
    print("[case] graph decode rope step", flush=True)
    n_keys = np.array([90, 1, 4000, 17], np.int32)
    n = len(n_keys)
    pages = int((n_keys.max() + 15) // 16)
    fx = PagedFixture(nova, nb=n * pages + 3, layer=LAYERS[0], seed=13)
    tables = fx.tables(n, pages)
    half = nova.hd // 2
    cs, sn = nova.alloc(4096 * half * 4), nova.alloc(4096 * half * 4)
    nova.launch_rope_table(cs.ptr, sn.ptr, None)
    rng = np.random.default_rng(6)
    q = nova.upload(rng.standard_normal((len(LAYERS), n, nova.nh, nova.hd)).astype(np.float32))
    k = nova.upload(rng.standard_normal((len(LAYERS), n, nova.nkv, nova.hd)).astype(np.float32))
    v = nova.upload(rng.standard_normal((len(LAYERS), n, nova.nkv, nova.hd)).astype(np.float32))
    o = nova.alloc(len(LAYERS) * n * nova.nh * nova.hd * 4)
    ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n))
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    s = nova.dev_stream_create()
    qs, kvs = n * nova.nh * nova.hd, n * nova.kvw
    nova.dev_sync()

    def run():
        nova.launch_attn_decode_plan(dt.ptr, pages, dn.ptr, n, ws.ptr, s)
        for i, layer in enumerate(LAYERS):
            nova.launch_attn_decode_paged_rope_planned(q.ptr + i * qs * 4, k.ptr + i * kvs * 4, v.ptr + i * kvs * 4,
                                                       cs.ptr, sn.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, pages, n, layer,
                                                       fx.nb, o.ptr + i * qs * 4, ws.ptr, s)

    eager, outs = _replays(nova, s, run, lambda: o.numpy((len(LAYERS), n, nova.nh, nova.hd), np.float32))
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"


def test_prefill_layer_graph(nova7):
    """batched append + causal prefill, 4 sessions"""
    nova = nova7
    print("[case] graph prefill", flush=True)
    n_past = np.array([0, 300, 1000, 47], np.int32)
    n, n_q = len(n_past), 96
    pages = int((n_past.max() + n_q + 15) // 16)
    fx = PagedFixture(nova, nb=n * pages + 3, layer=LAYERS[1], seed=14)
    tables = fx.tables(n, pages)
    rng = np.random.default_rng(7)
    q = nova.upload(rng.standard_normal((n, n_q, nova.nh, nova.hd)).astype(np.float32))
    kc = nova.upload(f16(rng, (n, n_q, nova.nkv, nova.hd)))
    vc = nova.upload(f16(rng, (n, n_q, nova.nkv, nova.hd)))
    o = nova.alloc(n * n_q * nova.nh * nova.hd * 4)
    dt, dp = nova.upload(tables), nova.upload(n_past)
    s = nova.dev_stream_create()

    def run():
        nova.launch_kv_store_paged_batch(fx.k.ptr, fx.v.ptr, dt.ptr, pages, dp.ptr, n, LAYERS[1], fx.nb, n_q,
                                         kc.ptr, vc.ptr, s)
        nova.launch_attn_prefill_paged_batch(q.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, pages, dp.ptr, n, n_q, LAYERS[1],
                                             fx.nb, o.ptr, s)

    eager, outs = _replays(nova, s, run, lambda: o.numpy((n, n_q, nova.nh, nova.hd), np.float32))
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"


def test_prefill_single_session_graph(nova7):
    """the reference's per-session prefill calls (launch_kv_store_paged, then
    launch_attn_prefill_paged: the 64-column, two-key-group kernel) for three
    sessions, one of them with no prefix"""
    nova = nova7
    print("[case] graph single-session prefill", flush=True)
    n_past = [0, 500, 1700]
    n, n_q = len(n_past), 130
    pages = (max(n_past) + n_q + 15) // 16
    fx = PagedFixture(nova, nb=n * pages + 3, layer=LAYERS[1], seed=15)
    tables = fx.tables(n, pages)
    rng = np.random.default_rng(8)
    q = nova.upload(rng.standard_normal((n, n_q, nova.nh, nova.hd)).astype(np.float32))
    kc = nova.upload(f16(rng, (n, n_q, nova.nkv, nova.hd)))
    vc = nova.upload(f16(rng, (n, n_q, nova.nkv, nova.hd)))
    o = nova.upload(np.full((n, n_q, nova.nh, nova.hd), np.nan, np.float32))
    dts = [nova.upload(np.ascontiguousarray(tables[i])) for i in range(n)]
    s = nova.dev_stream_create()
    qrows, kvrows = n_q * nova.nh * nova.hd, n_q * nova.kvw

    def run():
        for i in range(n):
            nova.launch_kv_store_paged(fx.k.ptr, fx.v.ptr, dts[i].ptr, LAYERS[1], fx.nb, n_q, n_past[i],
                                       kc.ptr + i * kvrows * 2, vc.ptr + i * kvrows * 2, s)
            nova.launch_attn_prefill_paged(q.ptr + i * qrows * 4, fx.k.ptr, fx.v.ptr, dts[i].ptr, LAYERS[1], fx.nb,
                                           n_q, n_past[i], o.ptr + i * qrows * 4, s)

    eager, outs = _replays(nova, s, run, lambda: o.numpy((n, n_q, nova.nh, nova.hd), np.float32))
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"

def test_gemv_fused_graph(nova7):
    """quantise-in-launch GEMV over three matrices, and the four-token GEMV"""
    nova = nova7
    print("[case] graph gemv", flush=True)
    rng = np.random.default_rng(8)
    cols, rows = 3584, (512, 64, 300)
    ws = []
    for r in rows:
        b = rng.integers(0, 256, (r, cols // 256, 144), dtype=np.uint8)
        b[..., 0:2] = rng.uniform(2e-4, 4e-3, (r, cols // 256, 1)).astype(np.float16).view(np.uint8)
        b[..., 2:4] = rng.uniform(1e-4, 2e-3, (r, cols // 256, 1)).astype(np.float16).view(np.uint8)
        ws.append(nova.upload(b))
    x = nova.upload(rng.standard_normal(cols).astype(np.float32))
    x4 = nova.upload(rng.standard_normal((4, cols)).astype(np.float32))
    outs = [nova.alloc(r * 4) for r in rows]
    out4 = nova.alloc(4 * rows[0] * 4)
    qs, dd, sm = nova.alloc(4 * cols), nova.alloc(4 * cols // 8), nova.alloc(4 * cols // 4)
    s = nova.dev_stream_create()
    bl = (C.c_void_p * 3)(*[w.ptr for w in ws])
    rw = (C.c_int64 * 3)(*rows)
    ou = (C.c_void_p * 3)(*[o.ptr for o in outs])

    def run():
        nova.launch_gemv_q4k_f32(bl, rw, ou, 3, cols, x.ptr, s)
        nova.launch_quant_q8(qs.ptr, dd.ptr, sm.ptr, x4.ptr, 4, cols, s)
        nova.launch_gemv4_q4k(ws[0].ptr, rows[0], cols, qs.ptr, dd.ptr, sm.ptr, out4.ptr, s)

    def read():
        return np.concatenate([o.numpy((r,), np.float32) for o, r in zip(outs, rows)] +
                              [out4.numpy((4 * rows[0],), np.float32)])

    eager, reps = _replays(nova, s, run, read)
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(reps):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"


def test_gemv4_mfma_graph(nova7):
    """the four-token GEMV on its matrix-core path (32M weights and up), ragged 16-row blocks"""
    nova = nova7
    print("[case] graph gemv4 mfma", flush=True)
    rng = np.random.default_rng(9)
    rows, cols = 2051, 16384
    b = rng.integers(0, 256, (rows, cols // 256, 144), dtype=np.uint8)
    b[..., 0:2] = rng.uniform(2e-4, 4e-3, (rows, cols // 256, 1)).astype(np.float16).view(np.uint8)
    b[..., 2:4] = rng.uniform(1e-4, 2e-3, (rows, cols // 256, 1)).astype(np.float16).view(np.uint8)
    w = nova.upload(b)
    x4 = nova.upload(rng.standard_normal((4, cols)).astype(np.float32))
    qs, dd, sm = nova.alloc(4 * cols), nova.alloc(4 * cols // 8), nova.alloc(4 * cols // 4)
    out4 = nova.alloc(4 * rows * 4)
    s = nova.dev_stream_create()

    def run():
        nova.launch_quant_q8(qs.ptr, dd.ptr, sm.ptr, x4.ptr, 4, cols, s)
        nova.launch_gemv4_q4k(w.ptr, rows, cols, qs.ptr, dd.ptr, sm.ptr, out4.ptr, s)

    eager, reps = _replays(nova, s, run, lambda: out4.numpy((4 * rows,), np.float32))
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(reps):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"


def test_reference_call_pattern_graph(nova7):
    """the reference's per-session calls (launch_kv_store_paged, then
    launch_attn_decode_paged) for sessions on both sides of the one-launch
    short-context path (<= 40 pages) and the split + combine pair, two layers"""
    nova = nova7
    print("[case] graph reference call pattern", flush=True)
    n_keys = np.array([1, 17, 640, 641, 1500], np.int32)      # 1, 2, 40, 41, 94 pages
    n = len(n_keys)
    pages = int((n_keys.max() + 15) // 16)
    fx = PagedFixture(nova, nb=n * pages + 3, layer=LAYERS[0], seed=21)
    tables = fx.tables(n, pages)
    rng = np.random.default_rng(9)
    layers = LAYERS[:2]
    _fill_layers(fx, layers)
    q = nova.upload(rng.standard_normal((len(layers), n, nova.nh, nova.hd)).astype(np.float32))
    kn = nova.upload(f16(rng, (len(layers), n, nova.nkv, nova.hd)))
    vn = nova.upload(f16(rng, (len(layers), n, nova.nkv, nova.hd)))
    o = nova.upload(np.full((len(layers), n, nova.nh, nova.hd), np.nan, np.float32))
    dts = [nova.upload(np.ascontiguousarray(tables[i])) for i in range(n)]
    scratch = [nova.alloc(nova.nh * 32 * (nova.hd + 2) * 4) for _ in range(n)]
    s = nova.dev_stream_create()
    qrow, kvrow = nova.nh * nova.hd, nova.kvw

    def run():
        for li, layer in enumerate(layers):
            for i in range(n):
                r = li * n + i
                nova.launch_kv_store_paged(fx.k.ptr, fx.v.ptr, dts[i].ptr, layer, fx.nb, 1, int(n_keys[i]) - 1,
                                           kn.ptr + r * kvrow * 2, vn.ptr + r * kvrow * 2, s)
                nova.launch_attn_decode_paged(q.ptr + r * qrow * 4, fx.k.ptr, fx.v.ptr, dts[i].ptr, layer, fx.nb,
                                              int(n_keys[i]), o.ptr + r * qrow * 4, scratch[i].ptr, s)

    eager, outs = _replays(nova, s, run, lambda: o.numpy((len(layers), n, nova.nh, nova.hd), np.float32))
    assert np.all(np.isfinite(eager))
    for r, got in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"


def test_solo_step_graph(nova7):
    """the one-launch decode (fused append, then the RoPE-fused form) of two
    layers for ragged sessions, including an empty one"""
    nova = nova7
    print("[case] graph solo decode step", flush=True)
    n_keys = np.array([300, 0, 1, 129, 33], np.int32)
    n = len(n_keys)
    pages = int((n_keys.max() + 15) // 16)
    fx = PagedFixture(nova, nb=n * pages + 3, layer=LAYERS[0], seed=23)
    tables = fx.tables(n, pages)
    rng = np.random.default_rng(13)
    layers = LAYERS[:2]
    _fill_layers(fx, list(layers) + [layer + 1 for layer in layers])
    q = nova.upload(rng.standard_normal((len(layers), n, nova.nh, nova.hd)).astype(np.float32))
    kn = nova.upload(f16(rng, (len(layers), n, nova.nkv, nova.hd)))
    vn = nova.upload(f16(rng, (len(layers), n, nova.nkv, nova.hd)))
    k32 = nova.upload(rng.standard_normal((len(layers), n, nova.nkv, nova.hd)).astype(np.float32))
    v32 = nova.upload(rng.standard_normal((len(layers), n, nova.nkv, nova.hd)).astype(np.float32))
    cs, sn = nova.alloc(4096 * (nova.hd // 2) * 4), nova.alloc(4096 * (nova.hd // 2) * 4)
    nova.launch_rope_table(cs.ptr, sn.ptr, None)
    o = nova.upload(np.full((2, len(layers), n, nova.nh, nova.hd), np.nan, np.float32))
    dt, dn = nova.upload(tables), nova.upload(n_keys)
    s = nova.dev_stream_create()
    qs, kvs = n * nova.nh * nova.hd, n * nova.kvw
    ostride = len(layers) * qs

    def run():
        for li, layer in enumerate(layers):
            nova.launch_attn_decode_paged_solo(q.ptr + li * qs * 4, fx.k.ptr, fx.v.ptr, dt.ptr, pages, dn.ptr, n,
                                               layer, fx.nb, kn.ptr + li * kvs * 2, vn.ptr + li * kvs * 2,
                                               o.ptr + li * qs * 4, s)
        for li, layer in enumerate(layers):
            nova.launch_attn_decode_paged_rope_solo(q.ptr + li * qs * 4, k32.ptr + li * kvs * 4,
                                                    v32.ptr + li * kvs * 4, cs.ptr, sn.ptr, fx.k.ptr, fx.v.ptr,
                                                    dt.ptr, pages, dn.ptr, n, layer + 1, fx.nb,
                                                    o.ptr + (ostride + li * qs) * 4, s)

    eager, outs = _replays(nova, s, run, lambda: o.numpy((2, len(layers), n, nova.nh, nova.hd), np.float32))
    assert np.all(np.isfinite(eager))
    assert np.all(eager[:, :, 1] == 0), "a session without keys gets zero rows"
    for r, got in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {r}"
