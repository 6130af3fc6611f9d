"""In-tree build of the gfx950 library and its Python binding.

Outputs (next to this file, loaded by the package):
  libfusedtok_amd.so   the C-ABI library (include/fusedtok_amd.h): HIP kernels
                       for gfx950 plus the host launchers, built with hipcc;
  _fusedtok<EXT>.so    the pybind11 module (csrc/bindings.cpp), plain g++,
                       linked against libfusedtok_amd.so with an $ORIGIN rpath.

Every HIP translation unit is compiled with
  --offload-arch=gfx950 -O3 -std=c++17
  -fhip-fp32-correctly-rounded-divide-sqrt   (IEEE f32 divide / sqrt: the
                                              quantize scale and reciprocal
                                              are bit-exact contracts)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             (no packed-FP32 instructions)
and no fast-math. Outputs are written to a temporary name and renamed, so a
process that has the old library mapped never sees a half-written file.
"""

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = [
    "runtime.hip",
    "attention.hip",
    "qgemm.hip",
    "quantize.hip",
    "norm_rope_act.hip",
    "fused.hip",
    "layer.hip",
    "prefill.hip",
    "sampling.hip",
]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
]

LIB = os.path.join(PKG, "libfusedtok_amd.so")
EXT = os.path.join(PKG, "_fusedtok" + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        # hipcc's host pass warns about the gfx-only feature flag; only a
        # failing command is reported
        sys.stderr.write(p.stdout + p.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")
    return p


def _compile_hip(src, verbose):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj], verbose)
    return obj


def build_library(verbose=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(HIP_SOURCES), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile_hip(s, verbose), HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
         verbose)
    os.replace(tmp, LIB)
    return LIB


def build_binding(verbose=False):
    import pybind11

    inc = [
        "-I", pybind11.get_include(),
        "-I", sysconfig.get_paths()["include"],
        "-I", INCLUDE,
    ]
    tmp = EXT + ".tmp"
    _run(["g++", "-O2", "-shared", "-fPIC", "-std=c++17", "-fvisibility=hidden",
          *inc, os.path.join(CSRC, "bindings.cpp"), "-o", tmp,
          "-L", PKG, "-lfusedtok_amd", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, EXT)
    return EXT


def build(verbose=False):
    """Compile the HIP library and the binding; returns the output paths."""
    lib = build_library(verbose)
    ext = build_binding(verbose)
    return lib, ext


def built():
    return os.path.exists(LIB) and os.path.exists(EXT)


if __name__ == "__main__":
    print("\n".join(build(verbose="-v" in sys.argv)))
