"""Pins of the CPU oracle's RoPE (or_rope_table / or_rope_apply /
or_rope_kv_store_paged) -- the checker the GPU RoPE tests use.

The reference's RoPE (src/kernel/rope.cu) is CUDA, and its SYCL twin
(src/kernel/sycl/rope.cpp) needs sycl::exp2/log2/cos/sin, which the
reference's host shim (tests/host_sycl/sycl/sycl.hpp) does not provide, so
neither builds here.  The oracle is pinned by the reference's own known
answers (tests/gpu_misc.cu:16-38: cos = 1, sin = 0 at position 0, so RoPE at
position 0 is the identity; cos(1) at position 1, column 0) and by closed
forms that a wrong frequency, sign, pairing or position would break.
"""
import numpy as np
import pytest

THETA = 1e6
HALF = 64


@pytest.fixture(scope="module")
def table(oracle):
    return oracle.rope_table(4096, HALF, THETA)


def test_known_answers_position_zero_and_one(table, oracle):
    cs, sn = table
    assert np.all(cs[0] == 1.0) and np.all(sn[0] == 0.0)          # gpu_misc.cu:16-20
    assert abs(cs[1, 0] - 0.540302) < 5e-7                        # printed "pos1 i=0 cos"
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 28, 128)).astype(np.float32)
    k = rng.standard_normal((1, 4, 128)).astype(np.float32)
    q2, k2 = oracle.rope_apply("qwen25_7b", q, k, 0, cs, sn)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)      # gpu_misc.cu:31-38: identity


def test_column_zero_is_cos_of_position(table):
    cs, sn = table
    pos = np.arange(4096, dtype=np.float64)
    assert np.array_equal(cs[:, 0], np.cos(pos).astype(np.float32))
    assert np.array_equal(sn[:, 0], np.sin(pos).astype(np.float32))


def test_frequencies(table):
    cs, sn = table
    f = THETA ** (-np.arange(HALF) / HALF)                      # theta^(-2i/HD)
    ang = np.arctan2(sn[1].astype(np.float64), cs[1].astype(np.float64))
    assert np.allclose(ang, f, rtol=2e-6, atol=1e-9)
    # a far row: angle = pos * f modulo 2 pi, within the float rounding of pos * f
    p = 3001
    a = np.arctan2(sn[p].astype(np.float64), cs[p].astype(np.float64))
    want = np.angle(np.exp(1j * p * f))
    d = np.angle(np.exp(1j * (a - want)))
    assert np.abs(d).max() < p * f.max() * 2e-7 + 1e-6
    assert np.allclose(cs.astype(np.float64) ** 2 + sn.astype(np.float64) ** 2, 1.0, atol=3e-7)


def test_pairing_and_sign(table, oracle):
    """NeoX pairs (i, i + 64): e_i rotates to (c, s) at (i, i+64), e_{i+64} to (-s, c)."""
    cs, sn = table
    p = 777
    for i in (0, 5, 63):
        q = np.zeros((1, 28, 128), np.float32)
        q[0, 3, i] = 1.0
        q[0, 4, i + 64] = 1.0
        k = np.zeros((1, 4, 128), np.float32)
        k[0, 1, i] = 1.0
        q2, k2 = oracle.rope_apply("qwen25_7b", q, k, p, cs, sn)
        assert q2[0, 3, i] == cs[p, i] and q2[0, 3, i + 64] == sn[p, i]
        assert q2[0, 4, i] == -sn[p, i] and q2[0, 4, i + 64] == cs[p, i]
        assert k2[0, 1, i] == cs[p, i] and k2[0, 1, i + 64] == sn[p, i]
        assert np.count_nonzero(q2) == 4 and np.count_nonzero(k2) == 2


def test_relative_position_and_norm(table, oracle):
    """q.k after RoPE depends only on the position difference; pairs keep their norm."""
    cs, sn = table
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 28, 128)).astype(np.float32)
    k = rng.standard_normal((1, 4, 128)).astype(np.float32)

    def dots(pq, pk):
        q2, _ = oracle.rope_apply("qwen25_7b", q, k, pq, cs, sn)
        _, k2 = oracle.rope_apply("qwen25_7b", q, k, pk, cs, sn)
        return np.einsum("hd,d->h", q2[0, :7].astype(np.float64), k2[0, 0].astype(np.float64)), q2

    a, q2 = dots(10, 3)
    b, _ = dots(1010, 1003)
    assert np.allclose(a, b, rtol=1e-4, atol=1e-3)
    n0 = q[0, :, :64].astype(np.float64) ** 2 + q[0, :, 64:].astype(np.float64) ** 2
    n1 = q2[0, :, :64].astype(np.float64) ** 2 + q2[0, :, 64:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-6)


def test_rope_kv_store_is_rope_then_append(table, oracle):
    """The fused oracle equals or_rope_apply followed by the fp16 page append."""
    cs, sn = table
    model, n, pos0, nb = "qwen25_7b", 21, 45, 12
    rng = np.random.default_rng(2)
    q = rng.standard_normal((n, 28, 128)).astype(np.float32)
    k = rng.standard_normal((n, 4, 128)).astype(np.float32)
    v = rng.standard_normal((n, 4, 128)).astype(np.float32)
    table_ = rng.permutation(nb).astype(np.int32)
    shape = (2 * nb, 16, 4, 128)
    pk = np.full(shape, 0x7E00, np.uint16)
    pv = np.full(shape, 0x7E00, np.uint16)
    q2 = oracle.rope_kv_store_paged(model, q, k, v, cs, sn, pk, pv, table_, 1, nb, pos0)
    qr, kr = oracle.rope_apply(model, q, k, pos0, cs, sn)
    assert np.array_equal(q2, qr)
    got_k = oracle.kv_gather_paged(model, pk, table_, 1, nb, pos0 + n)
    got_v = oracle.kv_gather_paged(model, pv, table_, 1, nb, pos0 + n)
    assert np.array_equal(got_k[pos0:], kr.astype(np.float16).view(np.uint16))
    assert np.array_equal(got_v[pos0:], v.astype(np.float16).view(np.uint16))
    assert np.all(got_k[:pos0] == 0x7E00) and np.all(pk[:nb] == 0x7E00)   # other positions, other layer
