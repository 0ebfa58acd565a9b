"""Build recipe for the gfx950 libraries (one per model geometry).

    python conflux-nova_amd/build.py            # all models, in-tree
    python conflux-nova_amd/build.py 7b         # one model

Each model library libnova_hip_<model>.so holds the device contract
(include/hal.h), the kernel entry points (include/nova_kernel.h) and the host
paging layer's C ABI (include/nova_graph.h), compiled for exactly one geometry
(-DNOVA_MODEL_*), as the reference welds one model per binary
(include/nova/model/select.h).  Output goes to conflux-nova_amd/lib/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "lib"
OBJ = PKG / "_build"

MODELS = {
    "qwen25_1p5b": "NOVA_MODEL_QWEN25_1P5B",
    "qwen25_7b": "NOVA_MODEL_QWEN25_7B",
    "qwen25_14b": "NOVA_MODEL_QWEN25_14B",
}
ALIASES = {"1p5b": "qwen25_1p5b", "7b": "qwen25_7b", "14b": "qwen25_14b"}

HIP_SOURCES = [
    "code/device/hip/hal_hip.hip",
    "code/kernel/hip/attn_decode.hip",
    "code/kernel/hip/attn_prefill.hip",
    "code/kernel/hip/kv_pages.hip",
    "code/kernel/hip/rope.hip",
    "code/kernel/hip/q4k.hip",
]
# the test kit library libnova_testkit_<model>.so (testkit/nova_testkit.h):
# synthetic fills, calibration kernels, and the decode kernels' test entry
# points compiled from the product source with -DNOVA_TESTKIT
TESTKIT_SOURCES = [
    ("testkit/testkit.hip", []),
    ("code/kernel/hip/attn_decode.hip", ["-DNOVA_TESTKIT"]),
]
CXX_SOURCES = [
    "code/capi/graph_capi.cpp",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-std=c++17", "-O3", "-fPIC", "-Wall", "-Wno-unused-function",
    f"-I{ROOT / 'include'}", f"-I{PKG / 'code'}", f"-I{PKG / 'code/kernel/hip'}", f"-I{PKG / 'testkit'}",
]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    # packed-FP32 VALU ops stay disabled on this fleet (see the build notes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")


def _compile(src: str, model: str, define: str, extra: tuple = (), sub: str = "") -> Path:
    out = OBJ / model / sub / (Path(src).stem + ".o")
    out.parent.mkdir(parents=True, exist_ok=True)
    path = PKG / src
    if src.endswith(".hip"):
        cmd = [HIPCC, *COMMON, *HIP_FLAGS, f"-D{define}", *extra, "-c", str(path), "-o", str(out)]
    else:
        cmd = [HIPCC, *COMMON, f"-D{define}", "-x", "c++", "-c", str(path), "-o", str(out)]
    _run(cmd)
    return out


def build(models: list[str] | None = None, jobs: int | None = None) -> list[Path]:
    names = [ALIASES.get(m, m) for m in (models or list(MODELS))]
    LIB.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    built = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = {}
        for name in names:
            define = MODELS[name]
            for src in HIP_SOURCES + CXX_SOURCES:
                futs[ex.submit(_compile, src, name, define)] = (name, "hip")
            for src, extra in TESTKIT_SOURCES:
                futs[ex.submit(_compile, src, name, define, tuple(extra), "testkit")] = (name, "testkit")
        objs: dict[tuple, list[Path]] = {}
        for f in cf.as_completed(futs):
            objs.setdefault(futs[f], []).append(f.result())
    for name in names:
        for kind in ("hip", "testkit"):
            out = LIB / f"libnova_{kind}_{name}.so"
            tmp = out.with_suffix(".so.tmp")
            _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
                  *sorted(map(str, objs[(name, kind)])), "-lpthread"])
            os.replace(tmp, out)
            built.append(out)
    return built


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)


if __name__ == "__main__":
    for p in build(sys.argv[1:] or None):
        print(p)
