"""Builds libhardshell_hip.so (the C-ABI backend) and libtaco_hip.so (the host harness that
plays taco's role above it) in-tree, for gfx950 only."""

import hashlib
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(ROOT, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
# Host-only sources go through the host compiler; the HIP runtime calls and kernels through hipcc.
HOST_SOURCES = {"common.cpp", "hsm.cpp", "taco/harness.cpp", "taco/tokenizer.cpp"}

BACKEND_SOURCES = ["common.cpp", "hsm.cpp", "hs_api.cpp", "kernels.hip"]
HARNESS_SOURCES = ["taco/harness.cpp", "taco/tokenizer.cpp"]  # hs::fail, sha256: the backend's (one error state)

LIB_BACKEND = os.path.join(HERE, "libhardshell_hip.so")
LIB_HARNESS = os.path.join(HERE, "libtaco_hip.so")


def source_sha256() -> str:
    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC)):
        p = os.path.join(CSRC, name)
        if os.path.isfile(p):
            h.update(name.encode())
            h.update(open(p, "rb").read())
    return h.hexdigest()


def _compile(src: str, obj: str, sha: str, verbose: bool):
    rel = os.path.relpath(src, CSRC).replace(os.sep, "/")
    if rel in HOST_SOURCES:
        cmd = [CXX, "-O3", "-std=c++17", "-fPIC", "-pthread", "-I", os.path.join(ROOT, "include"),
               "-I", CSRC, f'-DHS_SOURCE_SHA256="{sha[:16]}"', "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{CXX} failed for {src}:\n{r.stdout}\n{r.stderr}")
        return
    cmd = [
        HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
        # packed FP32 ops stay off (no float arithmetic here; the flag keeps hipcc from emitting
        # v_pk_* f32 forms in any future code)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
        f'-DHS_SOURCE_SHA256="{sha[:16]}"',
        "-c", src, "-o", obj,
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")


def _link(objs, out, extra, verbose):
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out + ".tmp", *objs, *extra]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(out + ".tmp", out)


def build(verbose: bool = False, jobs: int = 8):
    os.makedirs(BUILD, exist_ok=True)
    sha = source_sha256()
    srcs = sorted(set(BACKEND_SOURCES + HARNESS_SOURCES))
    srcs = [s for s in srcs if os.path.exists(os.path.join(CSRC, s))]
    objs = {s: os.path.join(BUILD, s.replace("/", "_") + ".o") for s in srcs}
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, os.path.join(CSRC, s), objs[s], sha, verbose) for s in srcs]
        for f in futs:
            f.result()
    _link([objs[s] for s in BACKEND_SOURCES], LIB_BACKEND, [], verbose)
    harness = [s for s in HARNESS_SOURCES if s in objs]
    if "taco/harness.cpp" in objs:
        _link([objs[s] for s in harness], LIB_HARNESS,
              ["-L", HERE, "-lhardshell_hip", "-Wl,-rpath,$ORIGIN", "-pthread"], verbose)
    return LIB_BACKEND


if __name__ == "__main__":
    print(build(verbose=True))
