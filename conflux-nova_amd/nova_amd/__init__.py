"""ctypes binding of the gfx950 paged KV-cache libraries.

One shared library per model geometry (``libnova_hip_<model>.so``), as the
reference builds one binary per model.  ``load("qwen25_7b")`` returns a
:class:`Nova` whose attributes are the C entry points of include/hal.h,
include/nova_kernel.h and include/nova_graph.h with their argument types set,
plus a few numpy conveniences (``upload``, ``download``, ``DeviceBuffer``).

The binding never falls back to anything: a missing library raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
# NOVA_LIB_DIR: an explicit alternative build directory (A/B measurements)
LIB_DIR = Path(os.environ.get("NOVA_LIB_DIR", str(PKG / "lib")))
MODELS = ("qwen25_1p5b", "qwen25_7b", "qwen25_14b")

vp, i32, i64, u64, f32, sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_size_t
P_i32 = C.POINTER(C.c_int32)
P_i64 = C.POINTER(C.c_int64)
P_int = C.POINTER(C.c_int)
P_u64 = C.POINTER(C.c_uint64)


class Geometry(C.Structure):
    _fields_ = [("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("n_layers", C.c_int),
                ("kv_block", C.c_int), ("max_split", C.c_int), ("name", C.c_char_p)]


class CowOp(C.Structure):
    _fields_ = [("src", C.c_int32), ("dst", C.c_int32), ("table_index", C.c_int64)]


# name -> (restype, argtypes)
_SIGS = {
    # hal.h
    "dev_alloc": (vp, [u64]),
    "dev_free": (None, [vp]),
    "dev_upload": (None, [vp, vp, u64]),
    "dev_download": (None, [vp, vp, u64]),
    "dev_sync": (None, []),
    "dev_max_alloc": (u64, []),
    "dev_copy_d2d": (None, [vp, vp, u64, vp]),
    "dev_upload_async": (None, [vp, vp, u64, vp]),
    "dev_download_async": (None, [vp, vp, u64, vp]),
    "dev_zero": (None, [vp, u64, vp]),
    "dev_stream_create": (vp, []),
    "dev_stream_destroy": (None, [vp]),
    "dev_stream_sync": (None, [vp]),
    "dev_event_create": (vp, []),
    "dev_event_destroy": (None, [vp]),
    "dev_event_record": (None, [vp, vp]),
    "dev_event_elapsed_ms": (f32, [vp, vp]),
    "dev_graph_begin": (None, [vp]),
    "dev_graph_end": (vp, [vp]),
    "dev_graph_launch": (None, [vp, vp]),
    "dev_graph_destroy": (None, [vp]),
    "dev_cu_count": (i32, []),
    "dev_count": (i32, []),
    "dev_arch_name": (C.c_char_p, []),
    # nova_kernel.h
    "nova_model_geometry": (Geometry, []),
    "launch_kv_store_paged": (None, [vp, vp, vp, i32, i32, i32, i64, vp, vp, vp]),
    "launch_attn_decode_paged": (None, [vp, vp, vp, vp, i32, i32, i32, vp, vp, vp]),
    "launch_attn_prefill_paged": (None, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "attn_decode_batch_workspace_bytes": (sz, [i32]),
    "launch_attn_decode_paged_rope_planned": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp]),
    "launch_attn_decode_paged_rope_batch": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, vp, vp, vp]),
    "launch_attn_decode_paged_batch": (None, [vp, vp, vp, vp, i32, vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "launch_attn_decode_paged_batch_noalloc": (None, [vp, vp, vp, vp, i32, vp, i32, i32, i32, vp, vp, vp, vp]),
    "launch_attn_decode_paged_solo": (None, [vp, vp, vp, vp, i32, vp, i32, i32, i32, vp, vp, vp, vp]),
    "launch_attn_decode_paged_rope_solo": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, vp, vp]),
    "attn_decode_batch_status": (i32, [vp, i32]),
    "launch_attn_decode_plan": (None, [vp, i32, vp, i32, vp, vp]),
    "launch_attn_decode_paged_planned": (None, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp]),
    "launch_attn_prefill_paged_batch": (None, [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, vp, vp]),
    "launch_kv_store_paged_batch": (None, [vp, vp, vp, i32, vp, i32, i32, i32, i32, vp, vp, vp]),
    "launch_quant_q8": (None, [vp, vp, vp, vp, i32, i32, vp]),
    "launch_gemv_q4k": (None, [vp, i64, i32, vp, vp, vp, vp, vp]),
    "launch_gemv4_q4k": (None, [vp, i64, i32, vp, vp, vp, vp, vp]),
    "launch_gemv_q4k_f32": (None, [C.POINTER(vp), P_i64, C.POINTER(vp), i32, i32, vp, vp]),
    "launch_rope_table": (None, [vp, vp, vp]),
    "launch_rope_table_rows": (None, [vp, vp, i32, vp]),
    "launch_rope_batch": (None, [vp, vp, i32, i64, vp, vp, vp]),
    "launch_rope": (None, [vp, vp, i64, vp, vp, vp]),
    "launch_rope_kv_store_paged": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i64, vp]),
    "launch_rope_kv_store_paged_batch": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, vp]),
    "launch_kv_cow_copy": (None, [vp, vp, i32, vp, vp, i32, vp]),
    "launch_kv_cow_apply": (None, [vp, vp, i32, vp, C.POINTER(CowOp), i32, vp]),
    "launch_kv_zero_pages": (None, [vp, vp, i32, vp, i32, vp]),
    "launch_table_patch": (None, [vp, vp, vp, i32, vp]),
    # nova_graph.h
    "nova_kvpool_new": (vp, [i32, i64]),
    "nova_kvpool_delete": (None, [vp]),
    "nova_kvpool_acquire": (i32, [vp]),
    "nova_kvpool_alloc_block": (i32, [vp]),
    "nova_kvpool_free_block": (None, [vp, i32]),
    "nova_kvpool_ref_block": (None, [vp, i32]),
    "nova_kvpool_refcnt": (i32, [vp, i32]),
    "nova_kvpool_attach": (None, [vp, i32, i32, i32]),
    "nova_kvpool_attach_prefix": (None, [vp, i32, i32, i64]),
    "nova_kvpool_cow_slice": (i32, [vp, i32, i64]),
    "nova_kvpool_release": (None, [vp, i32]),
    "nova_kvpool_nblocks": (i32, [vp]),
    "nova_kvpool_nb_total": (i32, [vp]),
    "nova_kvpool_cow_count": (i32, [vp]),
    "nova_kvpool_free_blocks": (i32, [vp]),
    "nova_kvpool_used": (i32, [vp]),
    "nova_kvpool_free_slices": (i32, [vp]),
    "nova_kvpool_free_list": (i32, [vp, P_int, i32]),
    "nova_kvpool_refcnts": (i32, [vp, P_int, i32]),
    "nova_kvpool_table": (i32, [vp, i32, P_i32, i32]),
    "nova_kvpool_n_past": (i64, [vp, i32]),
    "nova_kvpool_set_n_past": (None, [vp, i32, i64]),
    "nova_kvpool_need_copy": (i32, [vp, i32, P_int, P_int]),
    "nova_kv_hash_ids": (u64, [P_int, sz]),
    "nova_kv_hash_text": (u64, [C.c_char_p, sz]),
    "nova_kv_hash_hex": (None, [u64, C.c_char_p]),
    "nova_kv_block_id": (None, [u64, u64, C.c_char_p]),
    "nova_registry_new": (vp, []),
    "nova_registry_delete": (None, [vp]),
    "nova_registry_set_capacity": (None, [vp, sz]),
    "nova_registry_put": (None, [vp, u64, u64, i32, i32, i64, i64]),
    "nova_registry_find": (i32, [vp, u64, u64, P_int, P_int, P_i64, P_i64]),
    "nova_registry_live": (i32, [vp]),
    "nova_registry_total": (i32, [vp]),
    "nova_paged_new": (vp, [i32, i64]),
    "nova_paged_delete": (None, [vp]),
    "nova_paged_pool": (vp, [vp]),
    "nova_paged_pool_k": (vp, [vp]),
    "nova_paged_pool_v": (vp, [vp]),
    "nova_paged_tables": (vp, [vp]),
    "nova_paged_nb": (i32, [vp]),
    "nova_paged_stream": (vp, [vp]),
    "nova_paged_create_session": (i32, [vp, i32]),
    "nova_paged_destroy_session": (None, [vp, i32]),
    "nova_paged_attach": (None, [vp, i32, i32, i32]),
    "nova_paged_attach_prefix": (None, [vp, i32, i32, i64]),
    "nova_paged_cow_guard": (i32, [vp, i32, i64, vp]),
    "nova_paged_session_cow": (None, [vp, i32, i64, i32, vp]),
    "nova_paged_cow_batch": (i32, [vp, P_int, P_i64, P_int, i32, vp]),
    "nova_paged_create_sessions": (i32, [vp, i32, i32, P_int]),
    "nova_paged_push_tables": (None, [vp, P_int, i32]),
    "nova_paged_table_dev": (vp, [vp, i32]),
}

# test kit library (conflux-nova_amd/testkit/nova_testkit.h): not part of the
# product; bound onto the same handle when it is built
_TESTKIT_SIGS = {
    "testkit_fill_normal_f16": (None, [vp, u64, u64, f32, vp]),
    "testkit_copy": (None, [vp, vp, u64, vp]),
    "testkit_stream_read": (None, [vp, u64, i32, vp, vp]),
    "testkit_attn_decode_split_only": (None, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp]),
    "testkit_decode_stream_floor": (None, [vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "testkit_attn_decode_planned_spin": (None, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
}


def lib_path(model: str) -> Path:
    return LIB_DIR / f"libnova_hip_{model}.so"


def testkit_path(model: str) -> Path:
    return LIB_DIR / f"libnova_testkit_{model}.so"


class Nova:
    """Typed handle on one model library."""

    def __init__(self, model: str):
        path = lib_path(model)
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        self.model = model
        self.path = path
        self.lib = C.CDLL(str(path), mode=C.RTLD_LOCAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)
        tk = testkit_path(model)
        self.testkit = C.CDLL(str(tk), mode=C.RTLD_LOCAL) if tk.exists() else None
        if self.testkit is not None:
            for name, (res, args) in _TESTKIT_SIGS.items():
                fn = getattr(self.testkit, name)
                fn.restype = res
                fn.argtypes = args
                setattr(self, name, fn)
        g = self.nova_model_geometry()
        self.nh, self.nkv, self.hd, self.n_layers, self.kb = g.nh, g.nkv, g.hd, g.n_layers, g.kv_block
        self.group = self.nh // self.nkv
        self.kvw = self.nkv * self.hd

    # ---------------- numpy conveniences ----------------
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, max(a.nbytes, 1))
        if a.nbytes:
            self.dev_upload(b.ptr, a.ctypes.data, a.nbytes)
        b.shape, b.dtype = a.shape, a.dtype
        return b

    def download(self, buf, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        ptr = buf.ptr if isinstance(buf, DeviceBuffer) else buf
        if out.nbytes:
            self.dev_download(out.ctypes.data, ptr + offset, out.nbytes)
        return out


class DeviceBuffer:
    """dev_alloc'd memory freed with the object (or explicitly with free())."""

    def __init__(self, nova: Nova, nbytes: int):
        self.nova = nova
        self.nbytes = int(nbytes)
        self.ptr = nova.dev_alloc(self.nbytes) if self.nbytes else None
        self.shape = None
        self.dtype = None

    def free(self):
        if self.ptr:
            self.nova.dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def numpy(self, shape=None, dtype=None) -> np.ndarray:
        return self.nova.download(self, shape or self.shape, dtype or self.dtype)


_CACHE: dict[str, Nova] = {}


def load(model: str = "qwen25_7b") -> Nova:
    if model not in _CACHE:
        _CACHE[model] = Nova(model)
    return _CACHE[model]


def f16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 (round-to-nearest-even) as uint16 bit patterns."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def gpu_present() -> bool:
    """True when a GPU is visible.  Reads the KFD topology, so it does not
    initialise HIP (CPU nodes report gfx_target_version 0)."""
    if os.environ.get("HIP_VISIBLE_DEVICES", None) == "":
        return False
    nodes = Path("/sys/class/kfd/kfd/topology/nodes")
    if not nodes.exists():
        return False
    for n in nodes.iterdir():
        try:
            for line in (n / "properties").read_text().splitlines():
                if line.startswith("gfx_target_version") and int(line.split()[1]) != 0:
                    return True
        except (OSError, ValueError, IndexError):
            continue
    return False
