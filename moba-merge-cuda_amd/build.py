"""Build libmoba_hip.so (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` (device code) and ``csrc/*.cpp`` (host-only runtime:
page pool, prepared-decode driver) file is compiled to an object under ``_build/`` and
linked into ``moba_hip/libmoba_hip.so``.  Objects are rebuilt when their
source or any header changed.  ``python build.py`` builds; ``--force``
rebuilds everything.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT_DIR = ROOT / "_build"
LIB = ROOT / "moba_hip" / "libmoba_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    # packed fp32 ops are disabled on this pool (device-side flag; the host
    # pass warns that it does not know the feature).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: no accumulator round trips through AGPRs for
    # the short-lived S / dP tiles
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-result",
]


def _headers():
    hs = list(CSRC.glob("*.h")) + list((ROOT.parent / "include").glob("*.h"))
    return max((h.stat().st_mtime for h in hs), default=0.0)


# Per-source flag changes.  attn_dkdv.hip runs one wave per SIMD: its dK / dV
# accumulators belong in AGPRs, so it is built without the VGPR-form flag.
NO_VGPR_FORM = {"attn_dkdv.hip"}


def _flags(src: Path):
    if src.suffix == ".cpp":  # host-only sources: the host compiler, HIP runtime API only
        return ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", "-D__HIP_PLATFORM_AMD__",
                "-I/opt/rocm/include"]
    if src.name in NO_VGPR_FORM:
        i = FLAGS.index("-amdgpu-mfma-vgpr-form")
        return FLAGS[:i - 1] + FLAGS[i + 1:]
    return FLAGS


def _compile(src: Path, force: bool) -> Path:
    obj = OUT_DIR / (src.name + ".o")  # suffix kept: foo.hip and foo.cpp get distinct objects
    if force or not obj.exists() or obj.stat().st_mtime < max(src.stat().st_mtime, _headers()):
        cc = os.environ.get("CXX", "g++") if src.suffix == ".cpp" else HIPCC
        cmd = [cc, *_flags(src), "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"hipcc failed on {src.name}")
    return obj


def build(force: bool = False, jobs: int = 8) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), sources))
    newest = max(o.stat().st_mtime for o in objs)
    if force or not LIB.exists() or LIB.stat().st_mtime < newest:
        tmp = LIB.with_suffix(f".so.{os.getpid()}")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
        subprocess.check_call(cmd)
        os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
