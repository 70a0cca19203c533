"""Build the fermix_amd HIP library in-tree: every ``csrc/*.hip`` is compiled for gfx950
with hipcc and linked into ``fermix_amd/libfermix_amd.so`` (a plain C-ABI shared
library, no torch types). Run ``python -m fermix_amd.build``."""

import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libfermix_amd.so")
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from forming v_pk_{add,mul,fma}_f32 (the host pass warns
# that it does not know the feature; harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # a variable read before it is set is a build error, not a warning
    "-Werror=uninitialized",
]


# Per-source additions. pf_small.hip (the n <= 128 Parlett-Reid, whose one-wave pair steps
# are bound by instruction issue): the max-ILP machine scheduler gave C2 0.1710 -> 0.1641
# ms/step with the same registers, no spills and the same bits; the default scheduler is
# kept elsewhere (the n <= 128 LU lost 1 % under it).
EXTRA_FLAGS = {
    "pf_small.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build fermix_amd)")


def _compile(hipcc, src, obj):
    cmd = [hipcc, *HIP_FLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-I", CSRC, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stderr}")
    return obj


def _stale(src, obj, deps_mtime):
    """True when obj is missing or older than its source, any shared header or an
    implementation file (.inc) the source includes."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    incs = re.findall(r'#include "([\w.]+\.inc)"', open(src).read())
    inc_mtime = max((os.path.getmtime(os.path.join(CSRC, i)) for i in incs), default=0.0)
    return t < os.path.getmtime(src) or t < deps_mtime or t < inc_mtime


def build(verbose=False, jobs=None, incremental=False):
    """Compile and link the library; returns its path. incremental=True recompiles only
    the sources whose object is older than the source or a header (the default compiles
    everything)."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    headers.append(os.path.join(os.path.dirname(HERE), "include", "fermix.h"))
    headers.append(os.path.abspath(__file__))  # the flags live here
    deps = max(os.path.getmtime(h) for h in headers if os.path.exists(h))
    todo = [(s, o) for s, o in zip(srcs, objs) if not incremental or _stale(s, o, deps)]
    jobs = jobs or min(max(1, len(todo)), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_compile, hipcc, s, o) for s, o in todo]
        for f in futs:
            o = f.result()
            if verbose:
                print("compiled", os.path.relpath(o, HERE), flush=True)
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("linked", LIB, flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv[1:])
    sys.exit(0)
