"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE).

Loads oracle/liboracle.so (the C restatement of the reference) and, where
present, the reference harnesses in oracle/_ref/.  Only tests/, smoke() and
bench.py's cpu_baseline leg may use this module, as the checker / the CPU
baseline -- never as the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF_DIR = HERE / "_ref"

vp, i32, i64, u64, sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_size_t
P_int = C.POINTER(C.c_int)
P_i32 = C.POINTER(C.c_int32)
P_i64 = C.POINTER(C.c_int64)


class Geom(C.Structure):
    _fields_ = [("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("kb", C.c_int)]


GEOMS = {
    "qwen25_1p5b": (12, 2, 128, 28),
    "qwen25_7b": (28, 4, 128, 28),
    "qwen25_14b": (40, 8, 128, 48),
}


def geom(model: str) -> Geom:
    nh, nkv, hd, _ = GEOMS[model]
    return Geom(nh, nkv, hd, 16)


_POOL_SIGS = {
    "new": (vp, [i32, i64]), "delete": (None, [vp]), "acquire": (i32, [vp]),
    "alloc_block": (i32, [vp]), "free_block": (None, [vp, i32]), "ref_block": (None, [vp, i32]),
    "refcnt": (i32, [vp, i32]), "attach": (None, [vp, i32, i32, i32]),
    "attach_prefix": (None, [vp, i32, i32, i64]), "cow_slice": (i32, [vp, i32, i64]),
    "release": (None, [vp, i32]), "nblocks": (i32, [vp]), "nb_total": (i32, [vp]),
    "cow_count": (i32, [vp]), "free_blocks": (i32, [vp]), "used": (i32, [vp]),
    "free_slices": (i32, [vp]), "free_list": (i32, [vp, P_int, i32]),
    "table": (i32, [vp, i32, P_i32, i32]), "n_past": (i64, [vp, i32]),
    "need_copy": (i32, [vp, i32, P_int, P_int]),
}
_REG_SIGS = {
    "new": (vp, []), "delete": (None, [vp]), "set_capacity": (None, [vp, sz]),
    "put": (None, [vp, u64, u64, i32, i32, i64, i64]),
    "find": (i32, [vp, u64, u64, P_int, P_int, P_i64, P_i64]),
    "live": (i32, [vp]), "total": (i32, [vp]),
}


class PoolAPI:
    """Uniform view of a KvPool implementation (oracle 'or_pool_', reference
    harness 'ref_pool_', product 'nova_kvpool_') so tests can drive all three
    with the same op sequence."""

    def __init__(self, lib, prefix: str, has_refcnts: bool):
        self.lib, self.prefix = lib, prefix
        for name, (res, args) in _POOL_SIGS.items():
            fn = getattr(lib, prefix + name)
            fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)
        self.has_refcnts = has_refcnts

    def free_list_arr(self, h) -> list[int]:
        n = self.free_list(h, None, 0)
        buf = (C.c_int * max(n, 1))()
        self.free_list(h, buf, n)
        return list(buf[:n])

    def table_arr(self, h, s) -> list[int]:
        n = self.table(h, s, None, 0)
        buf = (C.c_int32 * max(n, 1))()
        self.table(h, s, buf, n)
        return list(buf[:n])

    def refcnt_arr(self, h) -> list[int]:
        return [self.refcnt(h, b) for b in range(self.nb_total(h))]

    def need_copy_pair(self, h, s):
        a, b = C.c_int(), C.c_int()
        self.need_copy(h, s, C.byref(a), C.byref(b))
        return a.value, b.value


class RegistryAPI:
    def __init__(self, lib, prefix: str):
        for name, (res, args) in _REG_SIGS.items():
            fn = getattr(lib, prefix + name)
            fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)

    def find_tuple(self, h, p, s):
        a, b, c, d = C.c_int(), C.c_int(), C.c_int64(), C.c_int64()
        ok = self.find(h, p, s, C.byref(a), C.byref(b), C.byref(c), C.byref(d))
        return (a.value, b.value, c.value, d.value) if ok else None


class Oracle:
    def __init__(self):
        self.lib = C.CDLL(str(HERE / "liboracle.so"))
        L = self.lib
        L.or_pool_new.restype = vp
        self.pool = PoolAPI(L, "or_pool_", True)
        self.registry = RegistryAPI(L, "or_registry_")
        L.or_kv_hash_ids.restype, L.or_kv_hash_ids.argtypes = u64, [P_int, sz]
        L.or_kv_hash_text.restype, L.or_kv_hash_text.argtypes = u64, [C.c_char_p, sz]
        L.or_kv_block_id.restype, L.or_kv_block_id.argtypes = None, [u64, u64, C.c_char_p]
        L.or_kv_store_paged.argtypes = [Geom, vp, vp, vp, i32, i32, i32, i64, vp, vp]
        L.or_kv_gather_paged.argtypes = [Geom, vp, vp, i32, i32, i64, vp]
        L.or_cow_copy.argtypes = [Geom, vp, vp, i32, i32, i32, i32]
        L.or_attn_decode_paged.argtypes = [Geom, vp, vp, vp, vp, i32, i32, i32, vp]
        L.or_attn_decode_paged_f64.argtypes = [Geom, vp, vp, vp, vp, i32, i32, i32, vp]
        L.or_attn_prefill_paged.argtypes = [Geom, vp, vp, vp, vp, i32, i32, i32, i32, vp]
        L.or_attn_prefill_paged_f64.argtypes = [Geom, vp, vp, vp, vp, i32, i32, i32, i32, vp]
        L.or_attn_decode_batch.argtypes = [Geom, vp, vp, vp, vp, i32, vp, i32, i32, i32, vp, i32]
        L.or_rope_table.argtypes = [vp, vp, i32, i32, C.c_double]
        L.or_q4k_half.restype, L.or_q4k_half.argtypes = C.c_float, [C.c_uint16]
        L.or_q4k_dequant_block.argtypes = [vp, vp]
        L.or_quant_q8.argtypes = [vp, i32, i32, vp, vp, vp]
        L.or_gemv_q4k.argtypes = [vp, i64, i64, vp, vp, vp, vp]
        L.or_rope_apply.argtypes = [Geom, vp, vp, i32, i64, vp, vp]
        L.or_rope_kv_store_paged.argtypes = [Geom, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i64]

    # ---- hashing ----
    def kv_hash_ids(self, ids) -> int:
        a = (C.c_int * max(len(ids), 1))(*ids)
        return self.lib.or_kv_hash_ids(a, len(ids))

    def kv_hash_text(self, text: bytes) -> int:
        return self.lib.or_kv_hash_text(text, len(text))

    def kv_block_id(self, p: int, s: int) -> str:
        out = C.create_string_buffer(40)
        self.lib.or_kv_block_id(p, s, out)
        return out.value.decode()

    # ---- paged data path (numpy in / out) ----
    @staticmethod
    def _p(a: np.ndarray):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data

    def kv_store_paged(self, model, pool_k, pool_v, table, layer, nb, n, pos0, k, v):
        self.lib.or_kv_store_paged(geom(model), self._p(pool_k), self._p(pool_v), self._p(table),
                                   layer, nb, n, pos0, self._p(k), self._p(v))

    def kv_gather_paged(self, model, pool, table, layer, nb, n) -> np.ndarray:
        g = geom(model)
        out = np.empty((n, g.nkv, g.hd), np.uint16)
        self.lib.or_kv_gather_paged(g, self._p(pool), self._p(table), layer, nb, n, self._p(out))
        return out

    def cow_copy(self, model, pool_k, pool_v, n_layers, nb, src, dst):
        self.lib.or_cow_copy(geom(model), self._p(pool_k), self._p(pool_v), n_layers, nb, src, dst)

    def attn_decode_paged(self, model, q, pool_k, pool_v, table, layer, nb, n_keys, f64=False):
        g = geom(model)
        out = np.empty((g.nh, g.hd), np.float64 if f64 else np.float32)
        fn = self.lib.or_attn_decode_paged_f64 if f64 else self.lib.or_attn_decode_paged
        fn(g, self._p(q), self._p(pool_k), self._p(pool_v), self._p(table), layer, nb, n_keys, self._p(out))
        return out

    def attn_prefill_paged(self, model, q, pool_k, pool_v, table, layer, nb, n_q, n_past, f64=False):
        g = geom(model)
        out = np.empty((n_q, g.nh, g.hd), np.float64 if f64 else np.float32)
        fn = self.lib.or_attn_prefill_paged_f64 if f64 else self.lib.or_attn_prefill_paged
        fn(g, self._p(q), self._p(pool_k), self._p(pool_v), self._p(table), layer, nb, n_q, n_past,
           self._p(out))
        return out

    # ---- Q4_K ----
    def q4k_half(self, h: int) -> float:
        return self.lib.or_q4k_half(h)

    def q4k_dequant_block(self, block: np.ndarray) -> np.ndarray:
        block = np.ascontiguousarray(block, np.uint8)
        y = np.empty(256, np.float32)
        self.lib.or_q4k_dequant_block(self._p(block), self._p(y))
        return y

    def quant_q8(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        qs = np.empty((rows, cols), np.int8)
        d = np.empty((rows, cols // 32), np.float32)
        s = np.empty((rows, cols // 16), np.int32)
        self.lib.or_quant_q8(self._p(x), rows, cols, self._p(qs), self._p(d), self._p(s))
        return qs, d, s

    def gemv_q4k(self, w: np.ndarray, rows: int, cols: int, qs, d, s) -> np.ndarray:
        out = np.empty(rows, np.float64)
        self.lib.or_gemv_q4k(self._p(np.ascontiguousarray(w, np.uint8)), rows, cols, self._p(qs), self._p(d),
                             self._p(s), self._p(out))
        return out

    # ---- RoPE ----
    def rope_table(self, rows, half=64, theta=1e6):
        cs = np.empty((rows, half), np.float32)
        sn = np.empty((rows, half), np.float32)
        self.lib.or_rope_table(self._p(cs), self._p(sn), rows, half, theta)
        return cs, sn

    def rope_apply(self, model, q, k, pos0, cs, sn):
        """Rotate q [n][nh][hd] and k [n][nkv][hd] (fp32, in place copies returned)."""
        q = np.array(q, np.float32, order="C")
        k = np.array(k, np.float32, order="C")
        self.lib.or_rope_apply(geom(model), self._p(q), self._p(k), q.shape[0], pos0, self._p(cs), self._p(sn))
        return q, k

    def rope_kv_store_paged(self, model, q, k, v, cs, sn, pool_k, pool_v, table, layer, nb, pos0):
        """Returns the rotated q; pool_k / pool_v are updated in place."""
        q = np.array(q, np.float32, order="C")
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.lib.or_rope_kv_store_paged(geom(model), self._p(q), self._p(k), self._p(v), self._p(cs), self._p(sn),
                                        self._p(pool_k), self._p(pool_v), self._p(table), layer, nb,
                                        q.shape[0], pos0)
        return q

    def attn_decode_batch(self, model, q, pool_k, pool_v, tables, n_keys, layer, nb, n_threads):
        g = geom(model)
        n = len(n_keys)
        out = np.empty((n, g.nh, g.hd), np.float32)
        nk = np.ascontiguousarray(n_keys, dtype=np.int32)
        self.lib.or_attn_decode_batch(g, self._p(q), self._p(pool_k), self._p(pool_v), self._p(tables),
                                      tables.shape[1], self._p(nk), n, layer, nb, self._p(out), n_threads)
        return out


class CpuBaseline:
    """oracle/libcpubase.so: the throughput CPU restatement bench.py times as
    its cpu_baseline (AVX2/F16C, a thread pool over work units).  Agrees with
    the oracle to the attention tolerance, not bit for bit."""

    def __init__(self):
        self.lib = C.CDLL(str(HERE / "libcpubase.so"))
        self.lib.cb_attn_decode_batch.restype = None
        self.lib.cb_attn_prefill_batch.restype = None

    def attn_decode_batch(self, model, q, pool_k, pool_v, tables, n_keys, layer, nb, n_threads):
        g = geom(model)
        n = len(n_keys)
        out = np.empty((n, g.nh, g.hd), np.float32)
        nk = np.ascontiguousarray(n_keys, dtype=np.int32)
        p = lambda a: a.ctypes.data_as(vp)
        self.lib.cb_attn_decode_batch(g, p(q), p(pool_k), p(pool_v), p(tables), i32(tables.shape[1]), p(nk),
                                      i32(n), i32(layer), i32(nb), p(out), i32(n_threads))
        return out

    def attn_prefill_batch(self, model, q, pool_k, pool_v, tables, n_past, n_q, layer, nb, n_threads):
        """q [n_sess][n_q][nh][hd] f32; returns o of the same shape."""
        g = geom(model)
        n = len(n_past)
        out = np.empty((n, n_q, g.nh, g.hd), np.float32)
        npst = np.ascontiguousarray(n_past, dtype=np.int32)
        p = lambda a: a.ctypes.data_as(vp)
        self.lib.cb_attn_prefill_batch(g, p(q), p(pool_k), p(pool_v), p(tables), i32(tables.shape[1]), p(npst),
                                       i32(n), i32(n_q), i32(layer), i32(nb), p(out), i32(n_threads))
        return out


class Reference:
    """The reference's own headers / SYCL kernels compiled into oracle/_ref."""

    def __init__(self):
        self.lib = C.CDLL(str(REF_DIR / "libnova_ref_pool.so"))
        L = self.lib
        L.ref_pool_new.restype = vp
        self.pool = PoolAPI(L, "ref_pool_", True)
        self.registry = RegistryAPI(L, "ref_registry_")
        L.ref_kv_hash_ids.restype, L.ref_kv_hash_ids.argtypes = u64, [P_int, sz]
        L.ref_kv_hash_text.restype, L.ref_kv_hash_text.argtypes = u64, [C.c_char_p, sz]
        L.ref_kv_block_id.restype, L.ref_kv_block_id.argtypes = None, [u64, u64, C.c_char_p]
        self.q4k = None
        p = REF_DIR / "libnova_ref_q4k.so"
        if p.exists():
            self.q4k = C.CDLL(str(p))
            self.q4k.ref_q4k_half.restype, self.q4k.ref_q4k_half.argtypes = C.c_float, [C.c_uint16]
            self.q4k.ref_q4k_dequant_block.argtypes = [vp, vp]
            self.q4k.ref_q4k_selftest_block.argtypes = [vp]
        self.attn = {}
        for model, tag in (("qwen25_7b", "7b"), ("qwen25_1p5b", "1p5b")):
            p = REF_DIR / f"libnova_ref_attn_{tag}.so"
            if p.exists():
                a = C.CDLL(str(p))
                a.ref_attn_decode.argtypes = [vp, vp, vp, vp, i32, vp]
                a.ref_attn_prefill.argtypes = [vp, vp, vp, vp, i32, i32]
                a.ref_attn_decode_scratch_floats.restype = i32
                self.attn[model] = a

    @staticmethod
    def available() -> bool:
        return (REF_DIR / "libnova_ref_pool.so").exists()

    def kv_hash_ids(self, ids) -> int:
        a = (C.c_int * max(len(ids), 1))(*ids)
        return self.lib.ref_kv_hash_ids(a, len(ids))

    def kv_hash_text(self, text: bytes) -> int:
        return self.lib.ref_kv_hash_text(text, len(text))

    def kv_block_id(self, p: int, s: int) -> str:
        out = C.create_string_buffer(40)
        self.lib.ref_kv_block_id(p, s, out)
        return out.value.decode()

    def attn_decode(self, model, q, kc, vc, n_past):
        """contiguous kc/vc [pos][NKV][HD] fp32; keys [0, n_past]"""
        a = self.attn[model]
        nh, _, hd, _ = GEOMS[model]
        out = np.empty((nh, hd), np.float32)
        scr = np.empty(a.ref_attn_decode_scratch_floats(), np.float32)
        a.ref_attn_decode(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, out.ctypes.data, n_past, scr.ctypes.data)
        return out

    def attn_prefill(self, model, q, kc, vc, n_q, n_past):
        a = self.attn[model]
        nh, _, hd, _ = GEOMS[model]
        out = np.empty((n_q, nh, hd), np.float32)
        a.ref_attn_prefill(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, out.ctypes.data, n_q, n_past)
        return out
