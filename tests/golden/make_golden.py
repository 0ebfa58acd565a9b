"""Generate the golden fixtures in tests/golden/ from the reference's own code.

Run in the build container (where /root/reference exists) after
`make -C oracle`: it drives oracle/_ref/ -- the reference's paging headers
(code/graph/kv_pool.h, kv_block.h, kv_registry.h) and its SYCL attention
kernels (src/kernel/sycl/attn.cpp through tests/host_sycl/sycl/sycl.hpp),
compiled unchanged -- and stores inputs and outputs only:

  kv_hash.json        id sequences / texts -> 64-bit IDs and block-id strings
  pool_traces.json    random KvPool op sequences with every return value and
                      the full state (free list, refcounts, tables, n_past,
                      cow_count) after each op
  registry.json       BlockRegistry put/find sequences
  q4k.npz             Q4_K blocks -> dequantised floats through the reference's
                      own dequant_block (include/nova/quant/q4_k.h): the
                      known-answer block of tests/selftest_q4k.cpp:31-38 and
                      seeded random blocks (incl. subnormal / zero scales)
  attn_<model>.npz    decode (n_past = 9) and prefill (n_q = 3, n_past = 5)
                      outputs for the inputs of tests/sycl_bench.cpp:889-985
                      (xorshift Rng seed 0x9E3779B97F4A7C15, Q in [-1,1),
                      K/V * 0.7), K/V rounded to fp16 as the build stores them

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))

from oracle_py import GEOMS, Reference  # noqa: E402


class XorShift:
    """The Rng of tests/sycl_bench.cpp:212-220 (xorshift64, top 32 bits -> [-1, 1))."""

    def __init__(self, seed=0x9E3779B97F4A7C15):
        self.s = seed

    def next(self) -> float:
        m = (1 << 64) - 1
        s = self.s
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        self.s = s
        u = s >> 32
        return float(np.float32(np.float32(u) / np.float32(2147483648.0)) - np.float32(1.0))

    def array(self, n, scale=1.0):
        out = np.empty(n, np.float32)
        for i in range(n):
            v = self.next()
            out[i] = np.float32(v) * np.float32(scale) if scale != 1.0 else v
        return out


def hash_fixture(ref: Reference):
    rng = np.random.default_rng(1234)
    cases = [[151644, 8948, 198, 2610], [151644, 8948, 198, 2611], [], [0], [7], [-1, 12], [2147483647]]
    for n in (1, 2, 3, 5, 8, 17, 100, 333, 2047, 2048):
        cases.append(rng.integers(0, 151936, n).tolist())
    ids = [{"ids": c, "hash": ref.kv_hash_ids(c)} for c in cases]
    texts = ["", "a", "hello", "什么是导数？", "The quick brown fox jumps over the lazy dog" * 3]
    tx = [{"text": t, "hash": ref.kv_hash_text(t.encode())} for t in texts]
    blocks = [{"prefix": p, "suffix": s, "id": ref.kv_block_id(p, s)}
              for p, s in ((0, 0), (ids[0]["hash"], ids[1]["hash"]), (2 ** 64 - 1, 1))]
    return {"ids": ids, "texts": tx, "block_ids": blocks}


def snapshot(api, h, live):
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


def random_trace(api, seed, n_slices, ctx, n_ops):
    rng = np.random.default_rng(seed)
    h = api.new(n_slices, ctx)
    nbl = api.nblocks(h)
    live, ops = [], []
    for _ in range(n_ops):
        kind = rng.choice(["acquire", "alloc", "free", "ref", "attach", "attach_prefix", "cow", "release"],
                          p=[.18, .08, .08, .06, .12, .18, .22, .08])
        op = {"op": str(kind)}
        if kind == "acquire":
            r = api.acquire(h)
            if r >= 0:
                live.append(r)
        elif kind == "alloc":
            r = api.alloc_block(h)
        elif kind in ("free", "ref"):
            b = int(rng.integers(-1, api.nb_total(h) + 1))
            op["b"] = b
            (api.free_block if kind == "free" else api.ref_block)(h, b)
            r = None
        elif kind in ("attach", "attach_prefix", "cow", "release") and not live:
            continue
        elif kind == "attach":
            if len(live) < 2:
                continue
            d, s_ = rng.choice(live, 2, replace=False)
            k = int(rng.integers(0, nbl + 1))
            op.update(dst=int(d), src=int(s_), k=k)
            api.attach(h, int(d), int(s_), k)
            r = None
        elif kind == "attach_prefix":
            if len(live) < 2:
                continue
            d, s_ = rng.choice(live, 2, replace=False)
            n = int(rng.integers(0, ctx + 1))
            op.update(dst=int(d), src=int(s_), n=n)
            api.attach_prefix(h, int(d), int(s_), n)
            r = None
        elif kind == "cow":
            s_ = int(rng.choice(live))
            pos = int(rng.integers(-3, ctx + 20))
            op.update(s=s_, pos=pos)
            r = api.cow_slice(h, s_, pos)
        else:
            s_ = int(rng.choice(live))
            op["s"] = s_
            api.release(h, s_)
            live.remove(s_)
            r = None
        op["ret"] = r
        op["state"] = snapshot(api, h, live)
        ops.append(op)
    api.delete(h)
    return {"seed": seed, "n_slices": n_slices, "ctx": ctx, "ops": ops}


def fork_cow_probe(api):
    """init(3,64); acquire A, B; attach_prefix(B, A, 20); cow_slice(B, 20)"""
    h = api.new(3, 64)
    a, b = api.acquire(h), api.acquire(h)
    api.attach_prefix(h, b, a, 20)
    nb = api.cow_slice(h, b, 20)
    out = {"A": a, "B": b, "cow_ret": nb, "free_blocks": api.free_blocks(h),
           "refcnt_A_table1": api.refcnt(h, api.table_arr(h, a)[1]), "refcnt_new": api.refcnt(h, nb),
           "state": snapshot(api, h, [a, b])}
    api.delete(h)
    return out


def fork_scenario(api, n_roots=2, per_root=6, prefix=47, ctx=128, spare=2, seed=5):
    """Roots forked into children at an unaligned prefix, then token-by-token
    appends with cow_slice before each (tests/cow_e2e_demo.cpp:36-107 shape)."""
    rng = np.random.default_rng(seed)
    h = api.new(n_roots + n_roots * per_root + spare, ctx)
    roots = [api.acquire(h) for _ in range(n_roots)]
    kids = [api.acquire(h) for _ in range(n_roots * per_root)]
    rets = []
    for c, k in enumerate(kids):
        api.attach_prefix(h, k, roots[c % n_roots], prefix)
    pos = {k: prefix for k in kids}          # each child's next write position
    for _ in range(int(ctx - prefix)):
        for k in kids:
            if rng.random() < 0.7 and pos[k] < ctx:
                rets.append(api.cow_slice(h, k, pos[k]))
                pos[k] += 1
    out = {"n_roots": n_roots, "per_root": per_root, "prefix": prefix, "ctx": ctx, "spare": spare,
           "seed": seed, "cow_rets": rets, "state": snapshot(api, h, roots + kids)}
    api.delete(h)
    return out


def registry_fixture(ref: Reference):
    rng = np.random.default_rng(99)
    r = ref.registry
    out = []
    for cap in (64, 3):
        h = r.new()
        if cap != 64:
            r.set_capacity(h, cap)
        ops = []
        keys = [(int(rng.integers(0, 2 ** 63)), int(rng.integers(0, 8))) for _ in range(12)]
        for step in range(80):
            p, s = keys[int(rng.integers(0, len(keys)))]
            if rng.random() < 0.6:
                args = [p, s, int(rng.integers(0, 4)), step, int(rng.integers(0, 100)), int(rng.integers(100, 200))]
                r.put(h, *args)
                ops.append({"op": "put", "args": args, "live": r.live(h), "total": r.total(h)})
            else:
                ops.append({"op": "find", "args": [p, s], "ret": r.find_tuple(h, p, s)})
        out.append({"capacity": cap, "ops": ops})
        r.delete(h)
    return out


def attn_fixture(ref: Reference, model: str):
    nh, nkv, hd, _ = GEOMS[model]
    maxpos = 32
    rng = XorShift()
    q = rng.array(nh * hd)
    kc = rng.array(maxpos * nkv * hd, 0.7)
    vc = rng.array(maxpos * nkv * hd, 0.7)
    # the build stores fp16 K/V: round once, feed the same values to both sides
    kc16 = kc.astype(np.float16)
    vc16 = vc.astype(np.float16)
    k32 = kc16.astype(np.float32).reshape(maxpos, nkv, hd)
    v32 = vc16.astype(np.float32).reshape(maxpos, nkv, hd)
    dec = ref.attn_decode(model, q.reshape(nh, hd), k32, v32, 9)
    qp = rng.array(3 * nh * hd).reshape(3, nh, hd)
    pre = ref.attn_prefill(model, qp, k32, v32, 3, 5)
    return dict(q=q.reshape(nh, hd), k16=kc16.view(np.uint16).reshape(maxpos, nkv, hd),
                v16=vc16.view(np.uint16).reshape(maxpos, nkv, hd), decode_n_past=np.int32(9), decode_out=dec,
                q_prefill=qp, prefill_n_q=np.int32(3), prefill_n_past=np.int32(5), prefill_out=pre)


def q4k_fixture(ref: Reference):
    import ctypes as C
    L = ref.q4k
    st = np.zeros(144, np.uint8)
    L.ref_q4k_selftest_block(st.ctypes.data)
    rng = np.random.default_rng(144)
    blocks = rng.integers(0, 256, (24, 144), dtype=np.uint8)
    ds = rng.uniform(1e-4, 2e-2, (24, 2)).astype(np.float16)
    ds[3] = [np.float16(3e-6), np.float16(0)]       # subnormal scale, zero min scale
    ds[4] = [np.float16(0), np.float16(1e-3)]
    blocks[:, 0:4] = ds.view(np.uint8).reshape(24, 4)
    blocks = np.concatenate([st[None], blocks])
    y = np.empty((len(blocks), 256), np.float32)
    for i, b in enumerate(blocks):
        bb = np.ascontiguousarray(b)
        L.ref_q4k_dequant_block(bb.ctypes.data, y[i].ctypes.data)
    halves = np.array([0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0x2C00, 0x1A00], np.uint16)
    hv = np.array([L.ref_q4k_half(C.c_uint16(int(h))) for h in halves], np.float32)
    return dict(blocks=blocks, y=y, halves=halves, half_values=hv)


def main():
    ref = Reference()
    (HERE / "kv_hash.json").write_text(json.dumps(hash_fixture(ref), indent=1))
    pool = ref.pool
    traces = [random_trace(pool, seed, ns, ctx, 60) for seed, ns, ctx in
              ((1, 3, 64), (2, 4, 80), (3, 5, 48), (4, 2, 100), (5, 6, 33))]
    (HERE / "pool_traces.json").write_text(json.dumps(
        {"fork_cow_probe": fork_cow_probe(pool), "traces": traces, "fork": fork_scenario(pool)}))
    (HERE / "registry.json").write_text(json.dumps(registry_fixture(ref)))
    for model in ("qwen25_7b", "qwen25_1p5b"):
        np.savez_compressed(HERE / f"attn_{model}.npz", **attn_fixture(ref, model))
    np.savez_compressed(HERE / "q4k.npz", **q4k_fixture(ref))
    for p in sorted(HERE.iterdir()):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
