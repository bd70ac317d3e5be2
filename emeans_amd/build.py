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
           "emh_rescore.hip", "emh_verify.hip", "emh_perm.cpp"]
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


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, err in results:
        if err and verbose:
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
