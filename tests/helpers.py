"""Shared helpers for the parity tests: seeded inputs, pool setup, tolerances."""
from __future__ import annotations

import numpy as np

# attention tolerance of the task statement: max-abs 2e-3 / rel 1e-2 against the
# fp32-accumulated reference
ATOL = 2e-3
RTOL = 1e-2


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance; "
                           f"max abs err {err.max():.3e}")
    return float(err.max())


def f16(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16).view(np.uint16)


class PagedFixture:
    """A small paged pool on the device plus its host mirror for one layer.

    Pages of `layer` are random fp16; other layers stay untouched device memory
    (never read).  Sessions get tables drawn from a seeded permutation of the
    pool, so pages are scattered as in a fragmented pool."""

    def __init__(self, nova, nb, layer, seed):
        self.nova, self.nb, self.layer = nova, nb, layer
        self.rng = np.random.default_rng(seed)
        page = nova.kb * nova.kvw
        self.page_halves = page
        per_pool = nova.n_layers * nb * page * 2
        self.k = nova.alloc(per_pool)
        self.v = nova.alloc(per_pool)
        self.hk = f16(self.rng, (nb, nova.kb, nova.nkv, nova.hd))
        self.hv = f16(self.rng, (nb, nova.kb, nova.nkv, nova.hd))
        self.push()

    def layer_off(self):
        return self.layer * self.nb * self.page_halves * 2

    def push(self):
        n = self.nova
        n.dev_upload(self.k.ptr + self.layer_off(), self.hk.ctypes.data, self.hk.nbytes)
        n.dev_upload(self.v.ptr + self.layer_off(), self.hv.ctypes.data, self.hv.nbytes)

    def pull(self):
        n = self.nova
        k = np.empty_like(self.hk)
        v = np.empty_like(self.hv)
        n.dev_download(k.ctypes.data, self.k.ptr + self.layer_off(), k.nbytes)
        n.dev_download(v.ctypes.data, self.v.ptr + self.layer_off(), v.nbytes)
        return k, v

    def tables(self, n_sess, max_pages):
        perm = self.rng.permutation(self.nb).astype(np.int32)
        assert n_sess * max_pages <= self.nb
        return np.ascontiguousarray(perm[: n_sess * max_pages].reshape(n_sess, max_pages))


class LayerPool:
    """A device pool sized for layers 0..layer only (the kernels address layer
    `layer` at page offset layer*nb, lower layers are never touched), with the
    pages of `layer` filled on the device by the seeded testkit generator and
    mirrored on the host.  For the full-size configurations, where a host
    generator would take minutes."""

    def __init__(self, nova, nb, layer, seed):
        self.nova, self.nb, self.layer = nova, nb, layer
        self.page_halves = nova.kb * nova.kvw
        per_layer = nb * self.page_halves
        self.k = nova.alloc((layer + 1) * per_layer * 2)
        self.v = nova.alloc((layer + 1) * per_layer * 2)
        off = layer * per_layer * 2
        nova.testkit_fill_normal_f16(self.k.ptr + off, per_layer, seed * 2 + 1, 1.0, None)
        nova.testkit_fill_normal_f16(self.v.ptr + off, per_layer, seed * 2 + 2, 1.0, None)
        nova.dev_sync()
        self.hk, self.hv = self.pull()

    def layer_off(self):
        return self.layer * self.nb * self.page_halves * 2

    def pull(self):
        n = self.nova
        shape = (self.nb, n.kb, n.nkv, n.hd)
        return (n.download(self.k, shape, np.uint16, self.layer_off()),
                n.download(self.v, shape, np.uint16, self.layer_off()))


def scattered_tables(rng, nb, pages):
    """one table row per session (width max(pages)), rows drawn without
    replacement from a seeded permutation of the pool: pages scattered as in a
    fragmented pool"""
    pages = np.asarray(pages, np.int64)
    perm = rng.permutation(nb).astype(np.int32)
    assert pages.sum() <= nb
    tables = np.zeros((len(pages), int(pages.max())), np.int32)
    off = 0
    for i, p in enumerate(pages):
        tables[i, :p] = perm[off:off + p]
        off += p
    return tables


def gather_f64(pool, table, n_keys):
    pos = np.arange(n_keys)
    return pool[table[pos >> 4], pos & 15].view(np.float16).astype(np.float64)   # [n_keys][NKV][HD]


def decode_f64(q, hk, hv, table, n_keys, group):
    """Textbook softmax(q.K^T / sqrt(HD)).V in float64 over keys [0, n_keys) of a
    paged pool, one kv head at a time (no repeated K/V)."""
    nh, hd = q.shape
    k = gather_f64(hk, table, n_keys)
    v = gather_f64(hv, table, n_keys)
    out = np.empty((nh, hd))
    for kvh in range(nh // group):
        qs = q[kvh * group:(kvh + 1) * group].astype(np.float64)
        s = qs @ k[:, kvh].T / np.sqrt(hd)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[kvh * group:(kvh + 1) * group] = (p @ v[:, kvh]) / p.sum(axis=1, keepdims=True)
    return out


def causal_f64(q, hk, hv, table, n_q, n_past, group):
    """Textbook causal softmax attention in float64 of n_q queries at positions
    n_past.. over the paged pool, one kv head at a time."""
    nh, hd = q.shape[1], q.shape[2]
    n_keys = n_past + n_q
    k = gather_f64(hk, table, n_keys)
    v = gather_f64(hv, table, n_keys)
    mask = np.arange(n_keys)[None, :] > (n_past + np.arange(n_q))[:, None]
    out = np.empty((n_q, nh, hd))
    for kvh in range(nh // group):
        qs = q[:, kvh * group:(kvh + 1) * group].astype(np.float64)          # [n_q][G][HD]
        s = np.einsum("qgd,kd->qgk", qs, k[:, kvh]) / np.sqrt(hd)
        s = np.where(mask[:, None, :], -np.inf, s)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        out[:, kvh * group:(kvh + 1) * group] = np.einsum("qgk,kd->qgd", p, v[:, kvh]) / p.sum(-1, keepdims=True)
    return out


def host_threads():
    import os
    return max(1, min(16, os.cpu_count() or 1))
