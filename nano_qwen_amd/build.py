"""Build libnq_attn.so (HIP, gfx950) in-tree with hipcc.

Usage: ``python -m nano_qwen_amd.build`` (or ``build()`` from Python).
Every ``csrc/*.hip`` file is compiled to an object in ``csrc/_build`` and the
objects are linked into ``nano_qwen_amd/libnq_attn.so``.  Flags:

* ``--offload-arch=gfx950``: MI355X only, no other targets;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: the kernels never
  emit packed-FP32 VALU instructions;
* ``-O3 -fPIC -shared``, C++17.
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
CSRC = PKG / "csrc"
BUILD = CSRC / "_build"
LIB = PKG / "libnq_attn.so"
INCLUDE = ROOT / "include"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
        f"-I{INCLUDE}", f"-I{CSRC}",
    ]


# Per-source extra flags.  The prefill kernels keep their MFMA accumulators
# in VGPR form: with the default heuristics the 64-row kernel spends about
# 175 AGPR<->VGPR moves per key tile.  Their work-queue atomics stay plain
# atomics: the atomic optimizer rewrites one into a wave-wide add whose
# result is needed at once, so the wave would wait for every K/V copy in
# flight right after it instead of where the fetched index is used.
EXTRA_FLAGS = {
    "varlen_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *_flags(), *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    if verbose and r.stderr.strip():
        # hipcc's host pass warns that it does not know packed-fp32-ops: harmless.
        lines = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if any(ln.strip() for ln in lines):
            print("\n".join(lines), file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source and link ``libnq_attn.so``; returns its path."""
    BUILD.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(srcs), 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
