"""Build the gfx950 S6 selective-scan library in-tree.

    python ml-experiments_amd/build.py            # -> ml-experiments_amd/s6scan/libs6scan.so

Every HIP source is compiled with hipcc for gfx950 only.  Packed FP32 instructions are
disabled (``-packed-fp32-ops``); the kernels are written for scalar fp32 VALU.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "s6scan", "libs6scan.so")
# (source, object name, extra defines): the scan kernels are compiled once per input
# dtype so the translation units build in parallel.
_TIO = {"f32": "float", "bf16": "s6::bf16", "f16": "s6::f16"}
UNITS = [("s6_abi.cpp", "s6_abi", []), ("s6_misc.hip", "s6_misc", []),
         ("s6_conv.hip", "s6_conv", []), ("s6_ssu.hip", "s6_ssu", []),
         ("s6_ssd.hip", "s6_ssd", []), ("s6_ssd_bwd.hip", "s6_ssd_bwd", [])]
UNITS += [(f"s6_{d}.hip", f"s6_{d}_{t}", [f"-DS6_TIO={ty}"])
          for d in ("fwd", "bwd") for t, ty in _TIO.items()]
# The single-pass forward is split further, per state count and B/C dtype.
UNITS += [("s6_fwd_lanes.hip", f"s6_fwd_lanes_{t}_n{ns}_bc{bcf}",
           [f"-DS6_TIO={ty}", f"-DS6_LANES_NS={ns}", f"-DS6_LANES_BCF32={bcf}"])
          for t, ty in _TIO.items() for ns in (16, 32, 64) for bcf in (0, 1)]
# The chunked forward's and the backward's row-block kernels (S6_FWD_VEC=1, S6_BWD_VEC=1)
# are a second unit per dtype each.
UNITS += [("s6_fwd.hip", f"s6_fwd_vec_{t}", [f"-DS6_TIO={ty}", "-DS6_FWD_VEC=1"])
          for t, ty in _TIO.items()]
UNITS += [("s6_bwd.hip", f"s6_bwd_vec_{t}", [f"-DS6_TIO={ty}", "-DS6_BWD_VEC=1"])
          for t, ty in _TIO.items()]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-command-line-argument",
]


def _compile(unit):
    src, name, defs = unit
    obj = os.path.join(BUILD, name + ".o")
    cmd = [HIPCC, *CFLAGS, *defs, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(UNITS), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, UNITS))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
