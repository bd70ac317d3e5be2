"""Build libemeans_hip.so (gfx950) in-tree with hipcc.

Flags that carry the exactness contract:
  -ffp-contract=off                           no multiply/add fusion the reference does not do
  -fno-gpu-flush-denormals-to-zero            f32 denormals kept (the split nudge makes them)
  -fhip-fp32-correctly-rounded-divide-sqrt    IEEE f32 division and sqrt
and one that avoids a hardware hazard of this platform:
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-FP32 VALU instructions
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libemeans_hip.so")
OBJ = os.path.join(HERE, "_obj")
SOURCES = ["emh_api.cpp", "emh_host.cpp", "emh_ops.hip", "emh_scatter.hip", "emh_screen.hip",
           "emh_screen3.hip", "emh_screen4.hip", "emh_screen_t1_bf3.hip", "emh_screen_t1_f32.hip",
           "emh_screen_kn_bf3_self.hip", "emh_screen_kn_bf3_any.hip",
           "emh_screen_kn_f32_self.hip", "emh_screen_kn_f32_any.hip", "emh_rescore.hip",
           "emh_verify.hip", "emh_autok.hip", "emh_topk_long.hip", "emh_screen4kn.hip",
           "emh_update.hip", "emh_perm.cpp"]
# Plain host C++ (no HIP), built by the system compiler.
HOST_ONLY = {"emh_perm.cpp"}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _compile(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    if src in HOST_ONLY:
        cmd = [CXX, "-O3", "-std=c++17", "-fPIC", "-Wall", "-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed on {src}:\n{r.stderr}")
    err = "\n".join(l for l in r.stderr.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l
                    and l.strip())
    return obj, err


def _stale(src):
    """Whether src's object is missing or older than src or any header."""
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    if not os.path.exists(obj):
        return True
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in os.listdir(CSRC)
                                        if h.endswith(".h")]
    deps.append(os.path.join(os.path.dirname(HERE), "include", "emeans_hip.h"))
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in deps)


def build(verbose=False, incremental=False):
    """Compile every source (or, with incremental, those whose object is
    older than the source or a header) and link the library."""
    os.makedirs(OBJ, exist_ok=True)
    todo = [s for s in SOURCES if _stale(s)] if incremental else SOURCES
    with ThreadPoolExecutor(max_workers=max(1, min(len(todo), os.cpu_count() or 8))) as ex:
        results = list(ex.map(_compile, todo))
    results += [(os.path.join(OBJ, os.path.splitext(s)[0] + ".o"), "") for s in SOURCES
                if s not in todo]
    for _, err in results:
        if err and verbose:
            print(err, file=sys.stderr)
    objs = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
