"""Builds libspectral_hip.so (gfx950) in-tree, next to the Python package.

    python unsloth-spectral_amd/build.py [--verbose]

Every .hip/.cpp file under csrc/ is compiled with hipcc for gfx950 and linked
into unsloth_spectral/libspectral_hip.so.  Packed FP32 instructions are
disabled for the device code (-Xclang -target-feature -Xclang
-packed-fp32-ops); the host pass prints a harmless warning about the feature.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "unsloth_spectral")
LIB_NAME = "libspectral_hip.so"
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = os.environ.get("SPECTRAL_HIP_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-fPIC", "-std=c++17", f"-I{INCLUDE}", f"-I{CSRC}"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]


def _sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src, verbose):
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *COMMON, "-x", "hip", *DEVICE, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    if verbose:
        noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if noise:
            print("\n".join(noise), file=sys.stderr)
    return obj


def build(verbose=False):
    """Compiles every source and links the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    out = os.path.join(OUT_DIR, LIB_NAME)
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="--verbose" in sys.argv)
    print(path)
