"""Pins the CPU oracle (oracle/nova_oracle.c) to the reference.

  * golden fixtures written by tests/golden/make_golden.py from the reference's
    own code compiled unchanged (oracle/_ref): KvPool traces, kv_block IDs,
    BlockRegistry, SYCL split-K decode / prefill outputs
  * the known answers of tests/kv_block_test.cpp and the pool probe
  * closed forms: n_keys == 1 => O == V (tests/gpu_misc.cu:41-65), equal scores
    => O == mean(V), prefill row == decode at n_past+qi+1, append/gather identity
  * when oracle/_ref is built (this container), a live differential fuzz
"""
import json
from pathlib import Path

import numpy as np
import pytest

from pool_replay import load_traces, replay, replay_fork, replay_probe

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_kv_block_known_answers(oracle):
    # tests/kv_block_test.cpp:7-22 and its printed values
    a = oracle.kv_hash_ids([151644, 8948, 198, 2610])
    b = oracle.kv_hash_ids([151644, 8948, 198, 2611])
    assert a == 0x956D626F6C666E6A and b == 0x966D626F6C666E6A and a != b
    assert oracle.kv_hash_ids([151644, 8948, 198, 2610]) == a
    assert oracle.kv_block_id(a, b) == "{ 956D626F6C666E6A . 966D626F6C666E6A }"
    assert oracle.kv_hash_ids([]) == 0


def test_kv_block_golden(oracle):
    g = json.loads((GOLDEN / "kv_hash.json").read_text())
    for c in g["ids"]:
        assert oracle.kv_hash_ids(c["ids"]) == c["hash"], c["ids"][:8]
    for c in g["texts"]:
        assert oracle.kv_hash_text(c["text"].encode()) == c["hash"]
    for c in g["block_ids"]:
        assert oracle.kv_block_id(c["prefix"], c["suffix"]) == c["id"]


def test_kv_block_fold_by_hand(oracle):
    # "12" -> bytes 0x31 0x32 -> hex "3132" padded right to 16 digits
    assert oracle.kv_hash_ids([12]) == 0x3132000000000000
    # three words fold to w0 + w2 and the middle w1 is carried, then summed
    ids = [1234567, 7654321, 99]          # "1234567" "7654321" "99" -> 32 hex digits + 4 -> 3 words
    hexs = "".join("%02X" % ch for ch in "".join(map(str, ids)).encode())
    hexs += "0" * (-len(hexs) % 16)
    w = [int(hexs[i:i + 16], 16) for i in range(0, len(hexs), 16)]
    while len(w) > 1:
        n = len(w)
        w = [(w[i] + w[n - 1 - i]) % 2 ** 64 for i in range(n // 2)] + ([w[n // 2]] if n % 2 else [])
    assert oracle.kv_hash_ids(ids) == w[0]


def test_pool_fork_cow_probe(oracle):
    replay_probe(oracle.pool, load_traces()["fork_cow_probe"])


@pytest.mark.parametrize("k", range(5))
def test_pool_golden_traces(oracle, k):
    replay(oracle.pool, load_traces()["traces"][k])


def test_pool_fork_scenario(oracle):
    replay_fork(oracle.pool, load_traces()["fork"])


def test_registry_golden(oracle):
    r = oracle.registry
    for case in json.loads((GOLDEN / "registry.json").read_text()):
        h = r.new()
        if case["capacity"] != 64:
            r.set_capacity(h, case["capacity"])
        for op in case["ops"]:
            if op["op"] == "put":
                r.put(h, *op["args"])
                assert (r.live(h), r.total(h)) == (op["live"], op["total"])
            else:
                got = r.find_tuple(h, *op["args"])
                assert (list(got) if got else None) == op["ret"]
        r.delete(h)


def _contiguous_pool(k16, nkv, hd):
    """contiguous [pos][NKV][HD] cache -> one-layer pool with identity table"""
    n = k16.shape[0]
    pages = (n + 15) // 16
    pool = np.zeros((pages * 16, nkv, hd), np.uint16)
    pool[:n] = k16
    return np.ascontiguousarray(pool), np.arange(pages, dtype=np.int32)


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b"])
def test_attention_golden(oracle, model):
    g = np.load(GOLDEN / f"attn_{model}.npz")
    nkv, hd = g["k16"].shape[1], g["k16"].shape[2]
    pk, table = _contiguous_pool(g["k16"], nkv, hd)
    pv, _ = _contiguous_pool(g["v16"], nkv, hd)
    nb = len(table)
    dec = oracle.attn_decode_paged(model, np.ascontiguousarray(g["q"]), pk, pv, table, 0, nb,
                                   int(g["decode_n_past"]) + 1)
    assert np.abs(dec - g["decode_out"]).max() < 1e-6
    pre = oracle.attn_prefill_paged(model, np.ascontiguousarray(g["q_prefill"]), pk, pv, table, 0, nb,
                                    int(g["prefill_n_q"]), int(g["prefill_n_past"]))
    assert np.abs(pre - g["prefill_out"]).max() < 1e-6
    # and the f64 textbook softmax (tests/sycl_bench.cpp:907-935 rel_l2 < 1e-5)
    ref = oracle.attn_decode_paged(model, np.ascontiguousarray(g["q"]), pk, pv, table, 0, nb,
                                   int(g["decode_n_past"]) + 1, f64=True)
    rel = np.sqrt(((dec - ref) ** 2).sum() / (ref ** 2).sum())
    assert rel < 1e-5


def _rand_pool(rng, nb, nkv, hd, scale=1.0):
    return (rng.standard_normal((nb, 16, nkv, hd)) * scale).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_14b"])
def test_decode_closed_forms(oracle, model):
    from oracle_py import GEOMS
    nh, nkv, hd, _ = GEOMS[model]
    rng = np.random.default_rng(3)
    nb = 12
    pk, pv = _rand_pool(rng, nb, nkv, hd), _rand_pool(rng, nb, nkv, hd)
    table = rng.permutation(nb).astype(np.int32)
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    # one key: output is that key's V row (tests/gpu_misc.cu:41-65)
    o1 = oracle.attn_decode_paged(model, q, pk, pv, table, 0, nb, 1)
    v0 = pv[table[0], 0].view(np.float16).astype(np.float32)
    assert np.abs(o1 - np.repeat(v0, nh // nkv, axis=0)).max() <= 1e-6
    # q == 0: all scores equal, output is the mean of V over the keys
    n = 150
    oz = oracle.attn_decode_paged(model, np.zeros_like(q), pk, pv, table, 0, nb, n)
    rows = np.stack([pv[table[p // 16], p % 16] for p in range(n)]).view(np.float16).astype(np.float64)
    mean = rows.mean(axis=0)                       # [nkv][hd]
    assert np.abs(oz - np.repeat(mean, nh // nkv, axis=0)).max() < 1e-5
    # paging is transparent: permuting pages while keeping logical content fixed
    perm = rng.permutation(nb)
    pk2, pv2 = pk.copy(), pv.copy()
    pk2[perm] = pk
    pv2[perm] = pv
    t2 = perm[table].astype(np.int32)
    a = oracle.attn_decode_paged(model, q, pk, pv, table, 0, nb, n)
    b = oracle.attn_decode_paged(model, q, pk2, pv2, t2, 0, nb, n)
    assert np.array_equal(a, b)


def test_prefill_row_is_decode(oracle):
    rng = np.random.default_rng(4)
    nb = 8
    pk, pv = _rand_pool(rng, nb, 4, 128), _rand_pool(rng, nb, 4, 128)
    table = rng.permutation(nb).astype(np.int32)
    q = rng.standard_normal((5, 28, 128)).astype(np.float32)
    pre = oracle.attn_prefill_paged("qwen25_7b", q, pk, pv, table, 0, nb, 5, 40, f64=True)
    for qi in range(5):
        dec = oracle.attn_decode_paged("qwen25_7b", np.ascontiguousarray(q[qi]), pk, pv, table, 0, nb, 41 + qi,
                                       f64=True)
        assert np.abs(pre[qi] - dec).max() < 1e-12


def test_store_gather_identity(oracle):
    rng = np.random.default_rng(6)
    nb = 10
    pk, pv = _rand_pool(rng, nb, 4, 128), _rand_pool(rng, nb, 4, 128)
    table = rng.permutation(nb).astype(np.int32)
    k = rng.integers(0, 65536, (37, 4, 128)).astype(np.uint16)
    v = rng.integers(0, 65536, (37, 4, 128)).astype(np.uint16)
    before_other = pk.copy()
    oracle.kv_store_paged("qwen25_7b", pk, pv, table, 0, nb, 37, 21, k, v)
    assert np.array_equal(oracle.kv_gather_paged("qwen25_7b", pk, table, 0, nb, 58)[21:], k)
    assert np.array_equal(oracle.kv_gather_paged("qwen25_7b", pv, table, 0, nb, 58)[21:], v)
    # positions before 21 untouched; by brute force on page/slot addresses
    for p in range(21):
        assert np.array_equal(pk[table[p // 16], p % 16], before_other[table[p // 16], p % 16])


def test_cow_copy_closed_form(oracle):
    rng = np.random.default_rng(8)
    L, nb = 3, 6
    pk = rng.integers(0, 65536, (L, nb, 16, 4, 128)).astype(np.uint16)
    pv = rng.integers(0, 65536, (L, nb, 16, 4, 128)).astype(np.uint16)
    ek, ev = pk.copy(), pv.copy()
    ek[:, 4] = pk[:, 1]
    ev[:, 4] = pv[:, 1]
    oracle.cow_copy("qwen25_7b", pk, pv, L, nb, 1, 4)
    assert np.array_equal(pk, ek) and np.array_equal(pv, ev)


def test_f16_rounding_matches_numpy(oracle):
    import ctypes as C
    L = oracle.lib
    L.or_f32_to_f16.restype, L.or_f32_to_f16.argtypes = C.c_uint16, [C.c_float]
    L.or_f16_to_f32.restype, L.or_f16_to_f32.argtypes = C.c_float, [C.c_uint16]
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(2000) * 10 ** rng.uniform(-9, 5, 2000),
                         [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.1e-5, 5.96e-8, 2.98e-8]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.or_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    hs = np.arange(0, 65536, 7, dtype=np.uint16)
    back = np.array([L.or_f16_to_f32(int(h)) for h in hs], np.float32)
    ref = hs.view(np.float16).astype(np.float32)
    same = (back == ref) | (np.isnan(back) & np.isnan(ref))
    assert same.all()


# ---------- live differential fuzz against the reference build, where present ----------
ref_mod = pytest.importorskip("oracle_py")
HAVE_REF = ref_mod.Reference.available()


@pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built here")
@pytest.mark.parametrize("seed", range(6))
def test_pool_fuzz_vs_reference(oracle, seed):
    from golden.make_golden import random_trace
    trace = random_trace(ref_mod.Reference().pool, 1000 + seed, 3 + seed % 4, 32 + 17 * seed, 120)
    replay(oracle.pool, trace)


@pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built here")
def test_hash_fuzz_vs_reference(oracle):
    ref = ref_mod.Reference()
    rng = np.random.default_rng(77)
    for n in list(range(0, 40)) + [511, 1000]:
        ids = rng.integers(-5, 10 ** int(rng.integers(1, 10)), n).tolist()
        assert oracle.kv_hash_ids(ids) == ref.kv_hash_ids(ids)


@pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built here")
@pytest.mark.parametrize("n_keys", [2, 31, 33, 64, 257])
def test_decode_fuzz_vs_reference_sycl(oracle, n_keys):
    ref = ref_mod.Reference()
    rng = np.random.default_rng(n_keys)
    model = "qwen25_1p5b"
    nb = (n_keys + 15) // 16 + 2
    pk, pv = _rand_pool(rng, nb, 2, 128), _rand_pool(rng, nb, 2, 128)
    table = rng.permutation(nb).astype(np.int32)
    q = rng.standard_normal((12, 128)).astype(np.float32)
    a = oracle.attn_decode_paged(model, q, pk, pv, table, 0, nb, n_keys)
    kc = np.ascontiguousarray(oracle.kv_gather_paged(model, pk, table, 0, nb, n_keys).view(np.float16).astype(np.float32))
    vc = np.ascontiguousarray(oracle.kv_gather_paged(model, pv, table, 0, nb, n_keys).view(np.float16).astype(np.float32))
    b = ref.attn_decode(model, q, kc, vc, n_keys - 1)
    assert np.abs(a - b).max() < 1e-6
