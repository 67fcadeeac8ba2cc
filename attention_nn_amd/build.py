"""Build libattnnn.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m attention_nn_amd.build              # or attention_nn_amd.build.build()
    python -m attention_nn_amd.build --changed    # only sources newer than their objects

Every ``csrc/*.hip`` file is compiled for gfx950 only, then linked into
``attention_nn_amd/libattnnn.so``.  Objects go to ``attention_nn_amd/_build``.
"""

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libattnnn.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code.
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include"), "-I", CSRC]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def _stale(src, headers):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(f) > t for f in [src, *headers])


def build(verbose=False, changed_only=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    headers.append(os.path.join(ROOT, "include", "attnnn.h"))
    todo = [s for s in srcs if _stale(s, headers)] if changed_only else srcs
    jobs = min(max(len(todo), 1), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_compile, todo))
    if verbose and changed_only:
        print("compiled: " + (", ".join(os.path.basename(s) for s in todo) or "nothing"))
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]
    tmp = LIB + ".tmp"
    # -z defs: an unresolved symbol fails the link instead of the first load
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-z,defs", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True, changed_only="--changed" in sys.argv[1:])
    sys.exit(0)
