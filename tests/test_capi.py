"""The C-ABI libraries load on a machine without a GPU and export every entry
point that include/*.h declares; the Python binding declares the same set."""
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))
TESTKIT_HEADER = ROOT / "conflux-nova_amd" / "testkit" / "nova_testkit.h"


def declared_functions(headers=None):
    names = set()
    for h in headers or HEADERS:
        text = re.sub(r"/\*.*?\*/", " ", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text):
            name = m.group(1)
            before = text[:m.start()].rstrip()
            if name in {"if", "for", "while", "sizeof", "return", "defined"} or before.endswith("typedef"):
                continue
            # a declaration: preceded by a type token at statement start
            line = before.split(";")[-1].split("{")[-1].split("}")[-1]
            if re.search(r"(void|int|float|size_t|uint16_t|uint64_t|int64_t|int32_t|char|nova_\w+_t|nova_geometry)\s*\**\s*$",
                         line.strip() + " "):
                names.add(name)
    return names


def test_headers_declare_the_boundary():
    names = declared_functions()
    for must in ("dev_alloc", "dev_free", "dev_upload", "dev_download", "dev_sync", "dev_max_alloc",
                 "launch_kv_store_paged", "launch_attn_decode_paged", "launch_attn_prefill_paged",
                 "nova_kvpool_cow_slice", "nova_kv_hash_ids", "nova_paged_cow_batch"):
        assert must in names, must


@pytest.mark.parametrize("model", ["qwen25_1p5b", "qwen25_7b", "qwen25_14b"])
def test_library_exports_every_declared_symbol(model):
    import nova_amd
    lib = nova_amd.lib_path(model)
    assert lib.exists(), f"{lib} not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = sorted(declared_functions() - exported)
    assert not missing, missing
    # and nothing else: the product library exports the contract and its
    # marked extensions only (the test kit lives in its own library)
    extra = sorted(exported - declared_functions())
    assert not extra, extra
    assert not any(n.startswith("testkit_") for n in exported)


@pytest.mark.parametrize("model", ["qwen25_1p5b", "qwen25_7b", "qwen25_14b"])
def test_testkit_library_exports_its_header(model):
    import nova_amd
    lib = nova_amd.testkit_path(model)
    assert lib.exists(), f"{lib} not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == declared_functions([TESTKIT_HEADER])


def test_binding_covers_every_declared_symbol():
    import nova_amd
    missing = sorted(declared_functions() - set(nova_amd._SIGS))
    assert not missing, missing
    assert set(nova_amd._TESTKIT_SIGS) == declared_functions([TESTKIT_HEADER])
    assert not set(nova_amd._TESTKIT_SIGS) & set(nova_amd._SIGS)


def test_library_loads_without_gpu(nova7):
    # host-only calls work; the device count is simply 0 here
    assert nova7.nova_model_geometry().nh == 28
    h = nova7.nova_kvpool_new(2, 64)
    assert nova7.nova_kvpool_acquire(h) == 0
    nova7.nova_kvpool_delete(h)


def _abort_run(code):
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                          env={"PYTHONPATH": str(ROOT / "conflux-nova_amd"), "HIP_VISIBLE_DEVICES": ""})


@pytest.mark.parametrize("call,needle", [
    ("n.launch_attn_decode_paged(1, 1, 1, 1, 0, 4, 0, 1, 1, None)", "n_keys >= 1"),
    ("n.launch_attn_decode_paged(1, 1, 1, 1, 99, 4, 5, 1, 1, None)", "layer < Model::L"),
    ("n.launch_kv_store_paged(1, 1, 1, 0, 0, 1, 0, 1, 1, None)", "nb > 0"),
    ("n.launch_attn_prefill_paged(0, 1, 1, 1, 0, 4, 1, 0, 1, None)", "q && pool_k"),
    ("n.launch_gemv_q4k(1, 4, 300, 1, 1, 1, 1, None)", "cols % kQK == 0"),
    ("n.launch_gemv_q4k(1, 4, 65536, 1, 1, 1, 1, None)", "cols <= kMaxCols"),
    ("n.launch_quant_q8(1, 1, 1, 1, 1, 33, None)", "cols % 32 == 0"),
    ("n.launch_gemv4_q4k(1, 4, 28928, 1, 1, 1, 1, None)", "cols <= kMaxCols4"),
    ("n.launch_gemv_q4k(1, 4, 256, 256, 260, 512, 1, None)", "aligned16(xd)"),
    ("n.launch_gemv4_q4k(1, 4, 256, 264, 256, 512, 1, None)", "aligned16(xq)"),
    ("n.launch_attn_decode_paged_rope_planned(1, 1, 1, None, 1, 1, 1, 1, 1, 1, 0, 4, 1, 1, None)",
     "q && k_new && v_new && cs && sn"),
    ("n.launch_attn_decode_paged_rope_planned(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 28, 4, 1, 1, None)",
     "layer < Model::L"),
    ("import ctypes as C; n.launch_gemv_q4k_f32((C.c_void_p * 5)(*[1] * 5), (C.c_int64 * 5)(*[1] * 5), "
     "(C.c_void_p * 5)(*[1] * 5), 5, 256, 1, None)", "n_mat <= kMaxMats"),
    ("import ctypes as C; n.launch_gemv_q4k_f32((C.c_void_p * 1)(1), (C.c_int64 * 1)(1), (C.c_void_p * 1)(1), "
     "1, 300, 1, None)", "cols % kQK == 0"),
    ("n.launch_rope_kv_store_paged(1, 1, 1, 1, 1, 1, 1, 1, 28, 4, 1, 0, None)", "layer < Model::L"),
    ("n.launch_rope_batch(1, 1, 2, -1, 1, 1, None)", "pos0 >= 0"),
])
def test_bad_arguments_abort_before_launch(call, needle):
    """the reference's abort-only convention (include/nova/config.h:42-63):
    argument checks fire on the host before anything reaches a device"""
    r = _abort_run(f"import nova_amd; n = nova_amd.load('qwen25_7b'); {call}")
    assert r.returncode != 0
    assert "requirement failed" in r.stderr and needle in r.stderr, r.stderr[-500:]


@pytest.mark.parametrize("n_sess", [0, 65])
def test_noalloc_decode_rejects_sizes_beyond_its_workspace(n_sess):
    """the allocation-free batched decode refuses session counts its static
    workspace does not cover, on the host, before any HIP call"""
    r = _abort_run("import nova_amd; n = nova_amd.load('qwen25_7b'); "
                   f"n.launch_attn_decode_paged_batch_noalloc(1, 1, 1, 1, 4, 1, {n_sess}, 0, 4, None, None, 1, None)")
    assert r.returncode != 0
    assert "static workspace" in r.stderr and f"n_sess {n_sess}" in r.stderr, r.stderr[-500:]


def _consumer():
    exe = Path(__file__).resolve().parent / "cpp" / "abi_consumer"
    if not exe.exists():
        pytest.skip("tests/cpp/abi_consumer is not built (build() makes it)")
    return exe


def test_cpp_consumer_builds_and_loads():
    """tests/cpp/abi_consumer.cpp compiles against the public headers alone
    (built by build()) and links and loads the 1.5B library; without a GPU it
    reports the skip code 77 before touching the device."""
    r = subprocess.run([str(_consumer())], capture_output=True, text=True, timeout=120)
    assert r.returncode in (0, 77), r.stdout + r.stderr


@pytest.mark.gpu
def test_cpp_consumer_on_gpu():
    """The C++ caller drives a fork, a COW, appends and decodes through the C
    ABI exactly as the reference's engine would, and checks its own results."""
    print("[case] tests/cpp/abi_consumer", flush=True)
    r = subprocess.run([str(_consumer())], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_consumer: PASS" in r.stdout
