"""Builds, in-tree:
  libaps_moe.so     all HIP sources under csrc/ (gfx950): the C ABI;
  libaps_layers.so  the C++ host API (cpp/*.cpp: Tensor, tensor_ops,
                    PhiMLP, PhiMoE) over libaps_moe.so;
  tests/cpp/layer_check  the GPU check program of the C++ API;
  tests/cpp/libmodel_drive.so  a C ABI over PhiTinyMoEModel for the tests
                    and bench.py --host cpp;
  probe/libaps_probe.so  bench.py's measurement of the fp32 FMA chain cost
                    (probe/fma_chain.hip), not part of the library.

    python -m aps2026_amd.build

Flags:
  --offload-arch=gfx950                  MI355X only
  -ffp-contract=off                      no implicit FMA contraction; every
                                         fused multiply-add is explicit
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE division in the router's
                                         quantisation step (reference semantics)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                         no packed fp32 instructions

Environment: APS_USE_TC=1 builds the C++ layer with the reference's USE_TC
(the LM head and the last layer's attention projections on the split-bf16
Linear), APS_USE_TC_ALL=1 with USE_TC and USE_TC_ALL (every attention
projection, four products); both are off by default, as in the reference.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libaps_moe.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-fvisibility=hidden", "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


LAYERS_LIB = os.path.join(HERE, "libaps_layers.so")
REPO = os.path.dirname(HERE)
CHECK_SRC = os.path.join(REPO, "tests", "cpp", "layer_check.cpp")
CHECK_BIN = os.path.join(REPO, "tests", "cpp", "layer_check")
# C ABI driver of the C++ model for the tests and bench.py --host cpp
DRIVE_SRC = os.path.join(REPO, "tests", "cpp", "model_drive.cpp")
DRIVE_LIB = os.path.join(REPO, "tests", "cpp", "libmodel_drive.so")

# bench.py's FMA-chain probe (a separate library: not part of the C ABI)
PROBE_SRC = os.path.join(HERE, "probe", "fma_chain.hip")
PROBE_LIB = os.path.join(HERE, "probe", "libaps_probe.so")

# host-only C++ (HIP runtime API, no device code): the system C++ compiler
CXX = os.environ.get("CXX", "g++")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include")]
if os.environ.get("APS_USE_TC_ALL") == "1":
    HOST_FLAGS += ["-DUSE_TC", "-DUSE_TC_ALL"]
elif os.environ.get("APS_USE_TC") == "1":
    HOST_FLAGS += ["-DUSE_TC"]
HIP_LINK = ["-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib")]


def _run(cmd, verbose):
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l and "(ignoring feature)" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"{os.path.basename(cmd[0])} failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


OBJ_DIR = os.path.join(HERE, "_build")


def build_hip(out: str = LIB, defines=(), verbose: bool = False, jobs: int = 0) -> str:
    """Compile every csrc/*.hip to an object (in parallel) and link them into
    the shared library `out`.  `defines` are extra -D flags (A/B builds)."""
    from concurrent.futures import ThreadPoolExecutor
    tag = "_".join(d.replace("=", "-") for d in defines) or "default"
    odir = os.path.join(OBJ_DIR, tag)
    os.makedirs(odir, exist_ok=True)
    cflags = [f for f in FLAGS if f not in ("-shared",)] + ["-D" + d for d in defines]
    srcs = sources()
    objs = [os.path.join(odir, os.path.basename(src)[:-4] + ".o") for src in srcs]
    jobs = jobs or max(1, min(len(srcs), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run([HIPCC, *cflags, "-c", "-o", so[1], so[0]], verbose), zip(srcs, objs)))
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> str:
    build_hip(LIB, verbose=verbose)
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, *FLAGS, "-o", tmp, PROBE_SRC], verbose)
    os.replace(tmp, PROBE_LIB)
    # C++ host API over the C ABI
    tmp = LAYERS_LIB + ".tmp"
    cpp = sorted(glob.glob(os.path.join(HERE, "cpp", "*.cpp")))
    _run([CXX, *HOST_FLAGS, "-shared", "-o", tmp, *cpp, "-L" + HERE, "-laps_moe",
          "-Wl,-rpath,$ORIGIN", *HIP_LINK], verbose)
    os.replace(tmp, LAYERS_LIB)
    if os.path.exists(CHECK_SRC):
        tmp = CHECK_BIN + ".tmp"
        _run([CXX, *HOST_FLAGS, "-o", tmp, CHECK_SRC, "-L" + HERE, "-laps_layers", "-laps_moe",
              "-Wl,-rpath,$ORIGIN/../../aps2026_amd", *HIP_LINK], verbose)
        os.replace(tmp, CHECK_BIN)
    if os.path.exists(DRIVE_SRC):
        tmp = DRIVE_LIB + ".tmp"
        _run([CXX, *HOST_FLAGS, "-shared", "-o", tmp, DRIVE_SRC, "-L" + HERE, "-laps_layers", "-laps_moe",
              "-Wl,-rpath,$ORIGIN/../../aps2026_amd", *HIP_LINK], verbose)
        os.replace(tmp, DRIVE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
