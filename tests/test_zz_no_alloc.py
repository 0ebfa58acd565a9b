"""launch_attn_decode_paged_batch_noalloc (plan and partials in the library's
static device array) against launch_attn_decode_paged_batch with a caller
workspace: two calls in a row, the second smaller, each bit-identical to the
workspace path and within tolerance of the C oracle (or_attn_decode_paged,
restating src/kernel/attn.cu:163-289,498-512)."""
import numpy as np
import pytest

from helpers import PagedFixture, assert_close, f16

pytestmark = pytest.mark.gpu
LAYER = 4


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b", "qwen25_14b"])
def test_noalloc_decode_matches_workspace_path(model, oracle):
    import nova_amd
    nova = nova_amd.load(model)
    rng = np.random.default_rng(17)
    first = rng.integers(200, 3000, 20).astype(np.int32)
    second = rng.integers(1, 400, 5).astype(np.int32)
    max_pages = int((max(first.max(), second.max()) + 15) // 16)
    fx = PagedFixture(nova, nb=len(first) * max_pages + 4, layer=LAYER, seed=17)
    for call, n_keys in enumerate((first, second)):
        n = len(n_keys)
        print(f"[case] noalloc decode {model} call {call} n_sess={n} n_keys max {n_keys.max()}", flush=True)
        tables = fx.tables(n, max_pages)
        q = rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
        k_new = f16(rng, (n, nova.nkv, nova.hd))
        v_new = f16(rng, (n, nova.nkv, nova.hd))
        dq, dt, dn = nova.upload(q), nova.upload(tables), nova.upload(n_keys)
        dk, dv = nova.upload(k_new), nova.upload(v_new)
        o_static = nova.upload(np.full(q.shape, np.nan, np.float32))
        nova.launch_attn_decode_paged_batch_noalloc(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, max_pages, dn.ptr, n, LAYER,
                                                    fx.nb, dk.ptr, dv.ptr, o_static.ptr, None)
        nova.dev_sync()
        got = o_static.numpy(q.shape, np.float32)
        ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(n))
        o_ws = nova.alloc(q.nbytes)
        nova.launch_attn_decode_paged_batch(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, max_pages, dn.ptr, n, LAYER, fx.nb,
                                            dk.ptr, dv.ptr, o_ws.ptr, ws.ptr, None)
        nova.dev_sync()
        assert np.array_equal(got, o_ws.numpy(q.shape, np.float32))
        # the appended token is in the pool (both calls wrote the same bits there)
        hk, hv = fx.pull()
        worst = 0.0
        for i in range(n):
            ref = oracle.attn_decode_paged(model, np.ascontiguousarray(q[i]), hk, hv, tables[i], 0, fx.nb,
                                           int(n_keys[i]))
            worst = max(worst, assert_close(got[i], ref, what=f"call {call} session {i}"))
        print(f"  max|gpu-oracle|={worst:.3e}")


def test_noalloc_decode_under_graph_capture():
    """The callers this entry point is for capture it into HIP graphs: a graph
    of one noalloc call (plan, split and combine launches on the static array)
    replayed three times, with an eager noalloc call of another batch between
    the replays rewriting the static array, gives the eager result of its own
    inputs bit for bit every time."""
    import nova_amd
    nova = nova_amd.load("qwen25_7b")
    rng = np.random.default_rng(23)
    n_keys = rng.integers(100, 2500, 12).astype(np.int32)
    other = rng.integers(1, 900, 7).astype(np.int32)
    max_pages = int((max(n_keys.max(), other.max()) + 15) // 16)
    fx = PagedFixture(nova, nb=(len(n_keys) + len(other)) * max_pages + 4, layer=LAYER, seed=23)
    tabs = fx.tables(len(n_keys) + len(other), max_pages)
    t_main, t_other = np.ascontiguousarray(tabs[: len(n_keys)]), np.ascontiguousarray(tabs[len(n_keys):])

    def inputs(n):
        q = rng.standard_normal((n, nova.nh, nova.hd)).astype(np.float32)
        return (q, nova.upload(q), nova.upload(f16(rng, (n, nova.nkv, nova.hd))),
                nova.upload(f16(rng, (n, nova.nkv, nova.hd))))

    q, dq, dk, dv = inputs(len(n_keys))
    qo, dqo, dko, dvo = inputs(len(other))
    dt, dn = nova.upload(t_main), nova.upload(n_keys)
    dto, dno = nova.upload(t_other), nova.upload(other)
    o_eager, o_graph, o_other = nova.alloc(q.nbytes), nova.alloc(q.nbytes), nova.alloc(qo.nbytes)

    def call(o, s, main=True):
        if main:
            nova.launch_attn_decode_paged_batch_noalloc(dq.ptr, fx.k.ptr, fx.v.ptr, dt.ptr, max_pages, dn.ptr,
                                                        len(n_keys), LAYER, fx.nb, dk.ptr, dv.ptr, o.ptr, s)
        else:
            nova.launch_attn_decode_paged_batch_noalloc(dqo.ptr, fx.k.ptr, fx.v.ptr, dto.ptr, max_pages, dno.ptr,
                                                        len(other), LAYER, fx.nb, dko.ptr, dvo.ptr, o.ptr, s)

    print("[case] noalloc decode under graph capture, 12 sessions, 3 replays", flush=True)
    call(o_eager, None)
    nova.dev_sync()
    want = o_eager.numpy(q.shape, np.float32)
    s = nova.dev_stream_create()
    nova.dev_graph_begin(s)
    call(o_graph, s)
    g = nova.dev_graph_end(s)
    for rep in range(3):
        poison = np.full(q.shape, np.nan, np.float32)
        nova.dev_upload(o_graph.ptr, poison.ctypes.data, poison.nbytes)
        call(o_other, None, main=False)          # rewrites the static array between replays
        nova.dev_sync()
        nova.dev_graph_launch(g, s)
        nova.dev_stream_sync(s)
        got = o_graph.numpy(q.shape, np.float32)
        assert np.array_equal(got, want), f"replay {rep}"
    nova.dev_graph_destroy(g)
    nova.dev_stream_destroy(s)
