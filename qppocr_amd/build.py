"""Builds the gfx950 HIP library qppocr_amd/libqppocr_hip.so from csrc/*.hip.

hipcc cross-compiles for gfx950 without a GPU.  Device code is built with
-ffp-contract=off (no a*b+c fusion beyond explicit fmaf, so every rounding
step matches the CPU path) and f32 denormal flushing (the CPU executor runs
with FTZ|DAZ).  Packed-fp32 instruction selection is disabled.
"""
import ctypes
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqppocr_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["qph_runtime.hip", "qph_gemm.hip", "qph_conv.hip", "qph_block.hip", "qph_rows.hip",
           "qph_net.hip", "qph_aux.hip", "qph_plan.hip"]

CFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-fgpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# host-code sanitizers only (the device code is built as usual): each
# -fsanitize= goes to the host compilation alone
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host",
            "-fno-omit-frame-pointer"]


def _compile(src, build_dir=None, extra=()):
    obj = os.path.join(build_dir or BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + CFLAGS + list(extra) + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose=False, sanitize=False):
    """sanitize: a host-code ASan + UBSan build into _build/sanitize/ (for CPU
    runs of the host-side checks under LD_PRELOAD of the ASan runtime, with
    QPPOCR_HIP_LIB pointing at it); the product library is not touched."""
    bdir = os.path.join(BUILD, "sanitize") if sanitize else BUILD
    lib = os.path.join(bdir, "libqppocr_hip.so") if sanitize else LIB
    extra = SANITIZE if sanitize else []
    os.makedirs(bdir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, bdir, extra), SOURCES))
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    if sanitize:   # host code only: no GPU sanitizer on the link either
        cmd[1:1] = ["-fno-gpu-sanitize", "-fsanitize=address", "-fsanitize=undefined", "-shared-libsan"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    # every symbol must resolve (a kernel whose host stub was dropped shows
    # up here, not at the first launch); a sanitizer build needs its runtime
    # preloaded to load, so it is not loaded here
    if not sanitize:
        try:
            ctypes.CDLL(os.path.abspath(tmp), mode=os.RTLD_NOW)
        except OSError as e:
            os.remove(tmp)
            raise RuntimeError(f"built library does not load: {e}")
    os.replace(tmp, lib)
    if verbose:
        print("built", lib)
    return lib


if __name__ == "__main__":
    build(verbose=True, sanitize="--sanitize" in sys.argv[1:])
