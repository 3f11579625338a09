"""Build the gfx950 C-ABI library ``libmoonmath_gfx950.so`` in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object for gfx950 only, then all
objects are linked into one shared library next to this file. No torch
extension machinery is involved: the library exports plain ``extern "C"``
symbols that ``_lib.py`` binds with ctypes.
"""
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
PKG_DIR = ROOT / "moonmath_attention"
SRC_DIR = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libmoonmath_gfx950.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"
# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32 (ordinary
# float code is compiled to scalar v_*_f32 instead).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Compiler-generated MFMAs keep their accumulators in VGPRs; AGPRs are used
    # only by the hand-placed inline-asm accumulators.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources():
    return sorted(SRC_DIR.glob("*.hip"))


def build(verbose=False):
    """Compile all sources (in parallel) and link the shared library."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in sources():
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        cmd = [hipcc, *DEVICE_FLAGS, "-I", str(SRC_DIR), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.decode(errors="replace").splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed.append((src, text))
        elif text.strip() and verbose:
            print(text)
    if failed:
        msg = "\n".join(f"--- {s.name}\n{t}" for s, t in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
