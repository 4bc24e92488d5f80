"""Build libzs.so (gfx950) in-tree with hipcc.

The library is the product: hand-written HIP kernels + the C ABI of
include/zs.h. `python -m zllm_amd.build` or `build()` compiles every source
each time it is called.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libzs.so")

SOURCES = ["zs_api.cpp", "zs_grammar.cpp", "zs_regex.cpp", "zs_schema.cpp", "zs_tokens.cpp", "zs_wire.cpp", "zs_sample.hip", "zs_row.hip", "zs_sums.hip", "zs_dfa.hip", "zs_lane.hip", "zs_spec.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # IEEE f32 behaviour the exact paths rely on: keep denormals, no contraction
    "-fno-gpu-flush-denormals-to-zero",
    "-ffp-contract=off",
    "-fno-fast-math",
    # packed fp32 VALU ops are disabled for correctness on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
    "-Wno-unused-result",
]


def build(verbose=False):
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    cmd = [HIPCC] + FLAGS + srcs + ["-o", LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libzs.so")
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
