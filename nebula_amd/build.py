"""In-tree build of the native libraries (hipcc for gfx950, gcc for host C).

libqwen_gpu.so   HIP kernels + runtime behind the reference's GPU C ABI
                 (include/qwen_gpu.h).
libnebula_moe.so C host driver of the layer and the 48-layer stack
                 (include/nebula_moe.h), calling libqwen_gpu.so's C ABI only.

Built .so files stay next to their sources (nebula_amd/lib/) so they travel to
the GPU box with the tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
HIP_SOURCES = ["qg_runtime.hip", "qg_ops.hip", "qg_moe.hip", "qg_decode.hip", "qg_prefill.hip", "nb_synth.hip"]
HOST_SOURCES = ["moe_host.c", "qwen_moe.c"]
ARCH = os.environ.get("NEBULA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{ROOT / 'include'}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if proc.returncode:
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False) -> dict[str, Path]:
    """Compile every native source; returns the built library paths."""
    LIBDIR.mkdir(exist_ok=True)
    objs = []
    for src in HIP_SOURCES:
        obj = LIBDIR / (Path(src).stem + ".o")
        _run(["hipcc", *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    gpu = LIBDIR / "libqwen_gpu.so"
    tmp = gpu.with_suffix(".so.tmp")
    _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    tmp.replace(gpu)
    host = LIBDIR / "libnebula_moe.so"
    tmp = host.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{ROOT / 'include'}",
          *[str(CSRC / s) for s in HOST_SOURCES], f"-L{LIBDIR}", "-lqwen_gpu", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    tmp.replace(host)
    for o in objs:
        Path(o).unlink(missing_ok=True)
    return {"gpu": gpu, "host": host}


def build_oracle() -> None:
    """The test oracle (own C restatement, and the reference's cpu.c when the
    reference tree is present)."""
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "all" if Path("/root/reference/qwen/cpu.c").exists() else "own"])


if __name__ == "__main__":
    print(build())
    build_oracle()
