"""Build the two native artefacts of wush_int4_kernel_amd, in place:

* ``libwush_int4.so`` -- every HIP kernel plus the C ABI of
  ``include/wush_int4.h``, compiled by hipcc for gfx950 only;
* ``_C<ext-suffix>.so`` -- the torch/pybind11 module that mirrors the
  reference's ``my_int4._C`` ops and calls the C ABI (g++, no device code).

Numerics flags: no FMA contraction, fp32 denormals kept, correctly rounded
division and square root (the quantizers are bit-exact with the reference);
packed-fp32 instructions are disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libwush_int4.so")
EXT = os.path.join(PKG, "_C" + sysconfig.get_config_var("EXT_SUFFIX"))

HIP_SOURCES = ["quant.hip", "fused_tq.hip", "gemv.hip", "gemm_s4.hip", "gemm_h16.hip", "gemm_h16q.hip", "gemm_h16s.hip", "setup.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]

# MFMA results in VGPRs: the int8 kernels' fold reads every accumulator
# element, and an AGPR destination would add one v_accvgpr_read per element.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]


def source_flags(src: str) -> list:
    # gemm_h16q.hip and gemm_h16s.hip hold up to 256 fp32 accumulators per
    # lane: they live in AGPRs
    return HIPCC_FLAGS + ([] if src in ("gemm_h16q.hip", "gemm_h16s.hip") else VGPR_FORM)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"command failed ({out.returncode}): {' '.join(cmd)}\n{out.stdout}\n{out.stderr}")
    return out


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def tuning_defines(spec: str | None = None) -> list:
    """-D flags for the build-time tuning macros of csrc/*.hip, from ``spec``
    or else the WUSH_DEFINES environment variable
    ("WUSH_TQ_SMALLM_PAIRS=8192 WUSH_GEMV_WAVES=8").
    Only WUSH_* names with plain values are accepted; anything else is an error."""
    flags = []
    for item in (os.environ.get("WUSH_DEFINES", "") if spec is None else spec).split():
        name, eq, value = item.partition("=")
        if not re.fullmatch(r"WUSH_[A-Z0-9_]+", name) or not re.fullmatch(r"[0-9A-Za-z_]*", value):
            raise ValueError(f"WUSH_DEFINES: {item!r} is not WUSH_NAME or WUSH_NAME=value")
        flags.append(f"-D{name}{eq}{value}")
    return flags


def build_capi(verbose: bool = False, lib_path: str = LIB, build_dir: str = BUILD,
               defines: str | None = None) -> str:
    """Compile libwush_int4.so (to ``lib_path``, objects in ``build_dir``) with
    the tuning macros of ``defines`` (default: the WUSH_DEFINES variable)."""
    os.makedirs(build_dir, exist_ok=True)
    cc = hipcc()
    dflags = tuning_defines(defines)

    def compile_one(src):
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        _run([cc, *source_flags(src), *dflags, f"-I{INCLUDE}", "-c", os.path.join(CSRC, src), "-o", obj],
             verbose)
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(6, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = lib_path + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, lib_path)
    return lib_path


def build_torch_ext(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], "/opt/rocm/include", INCLUDE]
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in inc],
        os.path.join(CSRC, "bindings.cpp"),
        *[f"-L{p}" for p in libdirs],
        f"-L{PKG}", "-lwush_int4",
        "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN",
        "-o", EXT + ".tmp",
    ]
    _run(cmd, verbose)
    os.replace(EXT + ".tmp", EXT)
    return EXT


def build(verbose: bool = False):
    """Compile libwush_int4.so, then the torch module that links it."""
    lib = build_capi(verbose)
    ext = build_torch_ext(verbose)
    return lib, ext


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print("built", p)
