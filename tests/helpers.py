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
