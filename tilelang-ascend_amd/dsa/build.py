"""Ahead-of-time build of libdsa_mi355x.so for gfx950 with hipcc.

Each source under ``csrc/`` is compiled to an object in ``_build/`` (in parallel)
and the objects are linked into ``dsa/libdsa_mi355x.so`` next to this file, so the
library travels with the source tree.  Run ``python -m dsa.build`` (with
``tilelang-ascend_amd`` on ``sys.path``) or call :func:`build`.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libdsa_mi355x.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

SOURCES = ["capi.cpp", "topk.hip", "indexer.hip", "indexer_h16.hip", "sparse_mla.hip", "sparse_flash_mla.hip",
           "quant.hip", "block_sparse_indexer.hip"]

# Packed-fp32 VALU forms are disabled for all device code (they are generated
# from ordinary float code at -O3 otherwise).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, "-I", str(CSRC), "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def _agpr_uses_outside_asm(body: str) -> int:
    """Instructions of a kernel body, outside its inline-asm blocks, that name an
    accumulation register (``a5``, ``a[0:3]``): a copy, a spill, or a load or LDS
    read into the AGPRs, all of which the compiler may generate on gfx950."""
    n, in_asm = 0, False
    for line in body.splitlines():
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if in_asm or not t or t[0] in ";.":
            continue
        if re.search(r"(?<![\w.])a\[?\d", t.split(";")[0]):
            n += 1
    return n


def _check_accumulators() -> None:
    """The 4-wave sparse MLA keeps O in the accumulation registers (AGPRs), which
    only its inline asm names; the compiler must not place any value of its own
    there.  Fails the build if the device assembly of those kernels holds any
    compiler-generated instruction with an AGPR operand."""
    src = CSRC / "sparse_mla.hip"
    asm = BUILD_DIR / "sparse_mla.s"
    cmd = [hipcc(), *COMMON_FLAGS, "-I", str(CSRC), "-x", "hip", "--cuda-device-only", "-S", str(src),
           "-o", str(asm)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src.name}:\n{res.stderr}")
    text = asm.read_text()
    bad = []
    for m in re.finditer(r"^(_ZN\w*mla_w4_kernel\w*):", text, re.M):
        end = text.index(".Lfunc_end", m.start())
        n = _agpr_uses_outside_asm(text[m.start():end])
        if n:
            bad.append(f"{m.group(1)}: {n}")
    if bad:
        raise RuntimeError("compiler-allocated accumulation registers in the 4-wave sparse MLA "
                           "(they hold O there):\n" + "\n".join(bad))


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    work = []
    for name in SOURCES:
        src = CSRC / name
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        work.append((src, obj))
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(work)))) as ex:
        futs = [ex.submit(_compile, *sw) for sw in work]
        futs.append(ex.submit(_check_accumulators))
        for fut in futs:
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
