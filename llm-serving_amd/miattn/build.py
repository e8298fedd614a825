"""Build ``libmiattn.so`` from ``csrc/*.hip`` with hipcc for gfx950, in-tree.

The library is the C-ABI declared in ``include/miattn.h``. It is compiled here (CPU-only
hosts cross-compile gfx950 fine) and shipped next to this file, so GPU boxes load the
prebuilt object and never compile.

Every HIP translation unit is compiled with packed-FP32 instruction selection disabled
(``-target-feature -packed-fp32-ops``): the kernels accumulate in plain fp32 and must not
be rewritten into ``v_pk_*_f32`` forms.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR.parent / "csrc"
REPO_ROOT = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
LIB_NAME = "libmiattn.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR.parent / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

SOURCES = ["capi.hip", "slot_write.hip", "paged_decode.hip", "varlen_prefill.hip", "decode_epilogue.hip",
           "decode_step.hip", "rows_gemm.hip"]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link ``libmiattn.so``; always rebuilds.

    Sources compile in parallel (one hipcc per file). Raises ``RuntimeError`` with the
    compiler output when a step fails.
    """
    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    procs = []
    objects = []
    pending = list(SOURCES)
    running: list[tuple[str, subprocess.Popen]] = []

    def _start(name: str) -> None:
        obj = OBJ_DIR / (Path(name).stem + ".o")
        objects.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-c", str(CSRC_DIR / name), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        running.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))

    while pending or running:
        while pending and len(running) < jobs:
            _start(pending.pop(0))
        name, proc = running.pop(0)
        output, _ = proc.communicate()
        procs.append(name)
        text = output.decode(errors="replace")
        if proc.returncode != 0:
            for _, other in running:
                other.kill()
            raise RuntimeError(f"hipcc failed on {name}:\n{text}")
        if verbose and text.strip():
            print(text, flush=True)

    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    if verbose:
        print(" ".join(link), flush=True)
    result = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout.decode(errors='replace')}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
