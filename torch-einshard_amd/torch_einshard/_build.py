"""Build libeinshard_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

    python -m torch_einshard._build [--verbose]

Each ``csrc/*.hip`` file is compiled to an object in ``<pkg root>/_build``
(in parallel), then linked into ``torch_einshard/_lib/libeinshard_hip.so``.
Every HIP translation unit is compiled with packed fp32 instructions disabled.
"""

import argparse
import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

_PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PACKAGE_DIR)  # torch-einshard_amd/
_REPO = os.path.dirname(_ROOT)
CSRC = os.path.join(_ROOT, "csrc")
INCLUDE = os.path.join(_REPO, "include")
BUILD_DIR = os.path.join(_ROOT, "_build")
LIB_DIR = os.path.join(_PACKAGE_DIR, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libeinshard_hip.so")

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc():
    found = shutil.which("hipcc")
    if found:
        return found
    candidate = "/opt/rocm/bin/hipcc"
    if os.path.exists(candidate):
        return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build libeinshard_hip)")


def _compile(hipcc, src, verbose):
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    noise = "is not a recognized feature for this target"
    messages = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{messages}")
    if verbose and messages.strip():
        print(messages, flush=True)
    return obj


def build(verbose=False, jobs=None):
    """Compile every HIP source and link the library; returns the library path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda src: _compile(hipcc, src, verbose), sources))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--verbose", action="store_true")
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args(argv)
    path = build(verbose=args.verbose, jobs=args.jobs)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
