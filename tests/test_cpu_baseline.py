"""The CPU baseline bench.py times (oracle/cpu_baseline.c) computes the same
attention as the oracle: batched decode and causal prefill against the
oracle's f64 two-pass softmax (attn.cu:163-357 restated), at the attention
tolerance, including a zero-key session, page-boundary lengths, splits of
more than 64 pages and a query block that is not a multiple of 16."""
import numpy as np
import pytest

from helpers import assert_close
from oracle_py import GEOMS, CpuBaseline


@pytest.fixture(scope="module")
def cpub():
    return CpuBaseline()


def _pool(rng, model, nb, layers):
    nh, nkv, hd, _ = GEOMS[model]
    shape = (layers, nb, 16, nkv, hd)
    k = rng.standard_normal(shape).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(shape).astype(np.float16).view(np.uint16)
    return k, v


@pytest.mark.parametrize("model", ["qwen25_7b", "qwen25_1p5b"])
def test_cpu_decode_batch_matches_oracle(cpub, oracle, model):
    rng = np.random.default_rng(41)
    nh, nkv, hd, _ = GEOMS[model]
    n_keys = np.array([1, 15, 16, 17, 700, 0, 2100, 1025], np.int32)
    n = len(n_keys)
    max_pages = int((n_keys.max() + 15) // 16)
    nb, layer = n * max_pages + 3, 1
    pk, pv = _pool(rng, model, nb, layer + 1)
    tables = rng.permutation(nb)[: n * max_pages].astype(np.int32).reshape(n, max_pages)
    q = (rng.standard_normal((n, nh, hd)) * 2.0).astype(np.float32)
    got = cpub.attn_decode_batch(model, q, pk, pv, tables, n_keys, layer, nb, 4)
    for i in range(n):
        if n_keys[i] == 0:
            assert (got[i] == 0).all()
            continue
        ref = oracle.attn_decode_paged(model, np.ascontiguousarray(q[i]), pk, pv,
                                       np.ascontiguousarray(tables[i]), layer, nb, int(n_keys[i]), f64=True)
        err = assert_close(got[i], ref, what=f"session {i}")
        assert err < 1e-5, err


def test_cpu_prefill_batch_matches_oracle(cpub, oracle):
    model = "qwen25_7b"
    rng = np.random.default_rng(43)
    nh, nkv, hd, _ = GEOMS[model]
    n_past = np.array([0, 5, 300], np.int32)
    n_q = 37
    n = len(n_past)
    max_pages = int((n_past.max() + n_q + 15) // 16)
    nb, layer = n * max_pages + 3, 0
    pk, pv = _pool(rng, model, nb, layer + 1)
    tables = rng.permutation(nb)[: n * max_pages].astype(np.int32).reshape(n, max_pages)
    q = rng.standard_normal((n, n_q, nh, hd)).astype(np.float32)
    got = cpub.attn_prefill_batch(model, q, pk, pv, tables, n_past, n_q, layer, nb, 3)
    for i in range(n):
        ref = oracle.attn_prefill_paged(model, np.ascontiguousarray(q[i]), pk, pv,
                                        np.ascontiguousarray(tables[i]), layer, nb, n_q, int(n_past[i]), f64=True)
        err = assert_close(got[i], ref, what=f"session {i}")
        assert err < 1e-5, err
