"""In-tree build of the native parts (no cmake, no JIT cache).

  adaptq_amd/libadaptq.so          C ABI + gfx950 kernels (hipcc)
  adaptq_amd/adaptq_py*.so         pybind11 module (MHAContext), links the above

  adaptq_amd/libadaptq_clk.so      timing library: the same library with decode.hip
                                   compiled with AQ_CLOCK_STAMPS (per-block
                                   shader-clock stamps of the LUT decode kernel,
                                   read by ``bench.py --clock-stamps``)
  adaptq_amd/libadaptq_probe.so    timing library: the bulk append's memory
                                   traffic without its codec (probe_rows.hip,
                                   read by ``bench.py --append-floor``)

Run ``python -m adaptq_amd.build`` or call :func:`build` (all four).  Every
call recompiles.  ``--clock-stamps`` or ``--probes`` builds only that timing
library.  The product never loads the timing libraries.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libadaptq.so")
CLK_LIB = os.path.join(PKG, "libadaptq_clk.so")
PROBE_LIB = os.path.join(PKG, "libadaptq_probe.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# -ffp-contract=off keeps every a*b+c that is not written fmaf() as two
# roundings (the bit-exact codec depends on it); correctly rounded fp32
# divide/sqrt and preserved denormals match the reference's x86 arithmetic;
# packed-FP32 instructions are disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]

SOURCES = ["append.hip", "decode.hip", "mquery.hip", "sparse.hip", "layout.hip", "kbackend.hip", "c_api.cpp", "vtable.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {os.path.basename(cmd[-1])}")
    return r


def build_lib(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(BUILD, src + ".o")
        lang = ["-x", "hip"]
        _run([HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-Wl,-rpath,{ROCM}/lib", "-Wl,-soname,libadaptq.so"])
    os.replace(tmp, LIB)
    return LIB


def build_clock_lib() -> str:
    """libadaptq_clk.so: decode.hip with AQ_CLOCK_STAMPS, the other objects
    from the last build_lib()."""
    os.makedirs(BUILD, exist_ok=True)
    obj = os.path.join(BUILD, "decode_clk.hip.o")
    _run([HIPCC, *HIP_FLAGS, "-DAQ_CLOCK_STAMPS", "-x", "hip", "-c",
          os.path.join(CSRC, "decode.hip"), "-o", obj])
    objs = [obj] + [os.path.join(BUILD, s + ".o") for s in SOURCES if s != "decode.hip"]
    missing = [o for o in objs if not os.path.exists(o)]
    if missing:
        raise RuntimeError(f"build the library first (missing {missing})")
    tmp = CLK_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-Wl,-rpath,{ROCM}/lib", "-Wl,-soname,libadaptq.so"])
    os.replace(tmp, CLK_LIB)
    return CLK_LIB


def build_probe_lib() -> str:
    """libadaptq_probe.so: the bulk append's memory traffic without its codec
    (probe_rows.hip; bench.py --append-floor)."""
    os.makedirs(BUILD, exist_ok=True)
    obj = os.path.join(BUILD, "probe_rows.hip.o")
    _run([HIPCC, *HIP_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, "probe_rows.hip"), "-o", obj])
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", obj, "-o", tmp,
          f"-Wl,-rpath,{ROCM}/lib", "-Wl,-soname,libadaptq_probe.so"])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_pybind() -> str:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "adaptq_py" + suffix)
    inc = sysconfig.get_paths()["include"]
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{pybind11.get_include()}",
          f"-I{inc}", f"-I{os.path.join(ROOT, 'include')}",
          os.path.join(CSRC, "adapter_python.cpp"), "-o", tmp,
          f"-L{PKG}", "-ladaptq", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build(jobs: int = 8) -> None:
    """The library, its Python module and the two timing libraries."""
    build_lib(jobs)
    build_pybind()
    build_clock_lib()
    build_probe_lib()


if __name__ == "__main__":
    if "--clock-stamps" in sys.argv[1:]:
        print("built", build_clock_lib())
    elif "--probes" in sys.argv[1:]:
        print("built", build_probe_lib())
    else:
        build()
        print("built", LIB)
