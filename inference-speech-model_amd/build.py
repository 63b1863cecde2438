"""Build libspeechkv.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage:  python inference-speech-model_amd/build.py [--debug]

The library lands next to the Python package that loads it
(speech_serving/libspeechkv.so) so it travels with the source tree.
"""
from __future__ import annotations

import argparse
import glob
import hashlib
import os
import shutil
import subprocess
import sys

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
SOURCES = [os.path.join(CSRC, "skv_kernels.hip"), os.path.join(CSRC, "skv_linear.hip")]
OUTPUT = os.path.join(PKG_ROOT, "speech_serving", "libspeechkv.so")
ARCH = "gfx950"


def code_flags(debug: bool = False) -> list:
    """The code-generation flags of a build (paths and output names excluded)."""
    return [
        f"--offload-arch={ARCH}",
        "-std=c++17",
        "-O1" if debug else "-O3",
        "-fPIC",
        "-shared",
        # Packed fp32 VALU ops are kept out of every kernel on purpose.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # The first 16 kernel-argument dwords arrive in scalar registers when a
        # wave starts (the attention kernel puts its address-chain parameters there).
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-fvisibility=hidden",
        "-Wno-unused-parameter",
    ]


def hashed_files() -> list:
    """Every file whose bytes reach the library: the HIP sources, their headers and the C-ABI header."""
    files = glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.h")) + \
        glob.glob(os.path.join(INCLUDE, "*.h"))
    return sorted(files, key=lambda f: os.path.relpath(f, REPO_ROOT))


def source_digest(debug: bool = False) -> str:
    """SHA-256 (first 16 hex digits) of the sources and code flags a build compiles.

    The build embeds it in skv_version() ("src:<digest>"); the Python binding
    recomputes it from the checked-out tree and refuses a library built from
    anything else."""
    h = hashlib.sha256()
    for f in hashed_files():
        h.update(os.path.relpath(f, REPO_ROOT).replace(os.sep, "/").encode() + b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
        h.update(b"\0")
    h.update(" ".join(code_flags(debug)).encode())
    return h.hexdigest()[:16]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(debug: bool = False, verbose: bool = False) -> str:
    """Compile every HIP source into one shared library; returns its path."""
    tmp = OUTPUT + ".tmp"
    cmd = [
        hipcc(),
        *code_flags(debug),
        f"-DSKV_SOURCE_DIGEST=\"{source_digest(debug)}\"",
        "-I", INCLUDE,
        "-I", CSRC,
        "-o", tmp,
        *SOURCES,
        # skv_linear's GEMMs (loaded after torch, the library binds to torch's copy of hipBLASLt)
        "-L", os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(hipcc()))), "lib"),
        "-lhipblaslt",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--debug", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(debug=args.debug, verbose=args.verbose))


if __name__ == "__main__":
    main()
