"""Build libqi_hip.so (HIP for gfx950 only) in-tree with hipcc.

Every translation unit is compiled with -ffp-contract=off (a multiply-add is
fused only where the source calls fmaf) and packed FP32 instructions disabled;
f32 denormals are kept (no flush-to-zero), as on the CPU reference.

The compiler's per-kernel resource report (registers, scratch, occupancy) is
written to _build/kernel_resources.json, and a kernel that spills registers
to scratch memory fails the build: the hot kernels run at one to four
wavefronts per SIMD with no room for scratch traffic.
"""
from __future__ import annotations

import concurrent.futures
import json
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqi_hip.so")
# profiling build: the same sources with the GEMV's timeline stamps compiled in
TIMELINE_LIB = os.path.join(HERE, "libqi_hip_timeline.so")
# measurement aid (bench.py --workload calib): plain streaming reads
CALIB_SRC = os.path.join(HERE, "calib", "stream_read.hip")
CALIB_LIB = os.path.join(HERE, "calib", "libqi_calib.so")

def read_sources() -> list:
    """The translation units, from csrc/sources.txt (shared with the Rust
    crate's build.rs, backends/hip/build.rs)."""
    with open(os.path.join(CSRC, "sources.txt")) as f:
        return [ln.strip() for ln in f if ln.strip() and not ln.lstrip().startswith("#")]


SOURCES = read_sources()

ARCH = "gfx950"
LINK = ["-Wl,-rpath,/opt/rocm/lib"]
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-ffp-contract=off", "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-file code generation: the GEMV keeps its matrix-instruction results in
# ordinary VGPRs (the accumulator-register form cost four moves per digit
# sum read in its combine; its accumulators are small). The GEMMs keep the
# default: their 128-register accumulator tiles need the accumulator file.
FILE_FLAGS = {"qi_gemv_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "qi_gemv_rows.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "qi_gemv_rm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libqi_hip.so")
    return path


_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]|SGPRs Spill|VGPRs Spill|LDS Size \[bytes/block\]):\s*(\S+)")
_KEYS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch",
         "Occupancy [waves/SIMD]": "waves_per_simd", "SGPRs Spill": "sgpr_spill",
         "VGPRs Spill": "vgpr_spill", "LDS Size [bytes/block]": "lds"}


def _resources(stderr: str) -> dict:
    """Per-kernel figures from -Rpass-analysis=kernel-resource-usage remarks."""
    out, cur = {}, None
    for key, val in _REMARK.findall(stderr):
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[_KEYS[key]] = int(val) if val.isdigit() else val
    return out


def _compile(src: str, timeline: bool = False):
    obj = os.path.join(BUILD, ("timeline_" if timeline else "") + os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    defs = ["-DQI_TIMELINE"] if timeline else []
    cmd = [hipcc(), *lang, *FLAGS, *FILE_FLAGS.get(src, []), *defs, "-Rpass-analysis=kernel-resource-usage",
           "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj, _resources(res.stderr)


def build_calib(verbose: bool = False) -> str:
    """libqi_calib.so, the streaming-read calibration of bench.py --workload calib."""
    tmp = CALIB_LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, "-shared", CALIB_SRC, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {CALIB_SRC}:\n{res.stderr}")
    os.replace(tmp, CALIB_LIB)
    if verbose:
        print(CALIB_LIB)
    return CALIB_LIB


def build(verbose: bool = False, timeline: bool = False) -> str:
    """libqi_hip.so (and the calibration library), or with timeline=True the
    profiling build libqi_hip_timeline.so."""
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        done = list(ex.map(lambda src: _compile(src, timeline), SOURCES))
    objs = [o for o, _ in done]
    kernels = {name: r for _, res in done for name, r in res.items()}
    if not timeline:
        with open(os.path.join(BUILD, "kernel_resources.json"), "w") as f:
            json.dump(kernels, f, indent=1, sort_keys=True)
    spills = sorted(n for n, r in kernels.items()
                    if r.get("scratch", 0) or r.get("vgpr_spill", 0) or r.get("sgpr_spill", 0))
    if spills:
        raise RuntimeError("kernels spill registers to scratch memory (see _build/kernel_resources.json): "
                           + ", ".join(spills))
    out = TIMELINE_LIB if timeline else LIB
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *LINK]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(out)
    if not timeline:
        build_calib(verbose)
    return out


if __name__ == "__main__":
    build(verbose=True, timeline="--timeline" in sys.argv[1:])
