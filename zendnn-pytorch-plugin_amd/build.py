"""In-tree build of the two native libraries of the zentorch package.

* zentorch/libzentorch_hip.so -- the gfx950 HIP kernels and the C-ABI of
  include/zentorch_hip.h (no torch dependency), built with hipcc.
* zentorch/_C.so -- TORCH_LIBRARY(zentorch) registration and the AOTInductor
  shims of include/shim_cuda_zentorch.h, linked against the library above and
  PyTorch-ROCm.
* tests/native/read_floor -- a plain streaming read of given sizes, the read
  floor bench.py --only floors reports beside the decode kernels.
* tests/native/bf16_rne_check -- a GPU program that checks the kernels' bf16
  rounding on every fp32 bit pattern (run by tests/test_bf16_rne_gpu.py).

Run ``python zendnn-pytorch-plugin_amd/build.py`` (or __graft_entry__.build()).
Every call compiles; objects go to zendnn-pytorch-plugin_amd/_build/.
"""
import concurrent.futures
import os
import shlex
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
PKG = os.path.join(HERE, "zentorch")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_SOURCES = ["woq_kernels.hip", "dynq_kernels.hip", "moe_kernels.hip", "capi.hip"]
TORCH_SOURCES = ["ops.cpp", "shim_cuda_zentorch.cpp"]

# -packed-fp32-ops: no v_pk_*_f32 from the compiler (hipcc's host pass warns
# it does not know the feature; that warning is harmless).
# -ffp-contract=off: a*b+c stays two roundings unless a kernel calls fmaf.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE, "-I" + CSRC,
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _torch_flags():
    import torch
    import torch.utils.cpp_extension as ce

    incs = ce.include_paths(device_type="cuda")
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-I" + INCLUDE, "-I" + CSRC,
              "-I" + os.path.join(ROCM, "include")]
    cflags += ["-I" + i for i in incs]
    ldflags = ["-L" + libdir, "-Wl,-rpath," + libdir, "-lc10", "-lc10_hip",
               "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-L" + PKG, "-lzentorch_hip",
               "-Wl,-rpath,$ORIGIN", "-L" + os.path.join(ROCM, "lib"), "-lamdhip64",
               "-lrocprofiler-sdk-roctx"]
    return cflags, ldflags


def _check_no_undefined_kernels(lib):
    """A kernel whose host launch stub the compiler did not emit links fine
    into a shared library and only fails when the library is loaded: refuse
    such a library here."""
    p = subprocess.run(["nm", "-u", lib], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    missing = [ln.split()[-1] for ln in p.stdout.splitlines() if "__device_stub__" in ln]
    if missing:
        raise RuntimeError(f"{lib}: kernel launch stubs not emitted: {missing}")


def build(verbose=False, jobs=8):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(PKG, exist_ok=True)
    cmds = []
    hip_objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        hip_objs.append(obj)
        cmds.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
    cflags, ldflags = _torch_flags()
    torch_objs = []
    for src in TORCH_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        torch_objs.append(obj)
        cmds.append(["g++"] + cflags + ["-c", os.path.join(CSRC, src), "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    hiplib = os.path.join(PKG, "libzentorch_hip.so")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", hiplib + ".tmp"]
         + hip_objs, verbose)
    _check_no_undefined_kernels(hiplib + ".tmp")
    os.replace(hiplib + ".tmp", hiplib)
    clib = os.path.join(PKG, "_C.so")
    _run(["g++", "-shared", "-o", clib + ".tmp"] + torch_objs + ldflags, verbose)
    os.replace(clib + ".tmp", clib)
    # the GPU test of the library's bf16 rounding (tests/test_bf16_rne_gpu.py)
    check = os.path.join(ROOT, "tests", "native", "bf16_rne_check")
    _run([HIPCC] + HIP_FLAGS + ["-o", check + ".tmp", check + ".hip"], verbose)
    os.replace(check + ".tmp", check)
    # the plain streaming read bench.py --only floors times beside the library
    floor = os.path.join(ROOT, "tests", "native", "read_floor")
    _run([HIPCC] + HIP_FLAGS + ["-o", floor + ".tmp", floor + ".hip"], verbose)
    os.replace(floor + ".tmp", floor)
    return hiplib, clib


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print(p)
