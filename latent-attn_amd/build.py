"""Build the in-tree native artefacts of the latent_attn package.

* ``latent_attn/liblatent_attn_hip.so`` -- the HIP kernels and the C ABI of
  include/latent_attn.h, compiled for gfx950 with hipcc (one object per
  source, compiled in parallel, then linked).
* ``latent_attn/_C<ext>`` -- the PyTorch-ROCm extension (pybind11) that wraps
  the C ABI; host-only C++ compiled with g++ against torch's headers and
  linked to the library with an $ORIGIN rpath.
* ``tests/cpp/reference_caller`` -- the C++ drop-in test program (a caller
  of include/fused_mla.cuh written like the reference's C++ test), run by
  tests/test_gpu_cpp_caller.py.
* with ``--phase-stamps`` only: ``_build/phase/liblatent_attn_hip.so``, the
  same sources compiled with -DLA_PHASE_STAMPS (kernels that record clock
  stamps at their phase boundaries), read by latent-attn_amd/phase_profile.py.
  It is a measurement build, never loaded by the package.

Usage: ``python latent-attn_amd/build.py [--lib-only] [--phase-stamps]``. Always recompiles.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "latent_attn")
INC = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

LIB_NAME = "liblatent_attn_hip.so"
HIP_SOURCES = ["la_append.hip", "la_capi.hip", "la_generic.hip", "la_mfma.hip", "la_naive.hip", "la_proj.hip"]

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INC}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}")


PHASE_LIB = os.path.join(BUILD, "phase", LIB_NAME)


def build_lib(jobs: int = 8, phase_stamps: bool = False) -> str:
    bdir = os.path.join(BUILD, "phase") if phase_stamps else BUILD
    os.makedirs(bdir, exist_ok=True)
    objs = []
    cmds = []
    extra = ["-DLA_PHASE_STAMPS"] if phase_stamps else []
    for src in HIP_SOURCES:
        obj = os.path.join(bdir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(cmds)))) as ex:
        list(ex.map(_run, cmds))
    out = PHASE_LIB if phase_stamps else os.path.join(PKG, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def build_ext() -> str:
    import torch
    from torch.utils import cpp_extension

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(PKG, "_C" + suffix)
    obj = os.path.join(BUILD, "bindings.o")
    os.makedirs(BUILD, exist_ok=True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], os.path.join(ROCM, "include"), INC]
    cflags = [
        "-O2", "-std=c++17", "-fPIC", "-w",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{i}" for i in incs],
    ]
    _run(["g++", *cflags, "-c", os.path.join(CSRC, "bindings.cpp"), "-o", obj])
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    tmp = out + ".tmp"
    _run([
        "g++", "-shared", "-o", tmp, obj,
        f"-L{PKG}", "-llatent_attn_hip",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
    ])
    os.replace(tmp, out)
    return out


def build_cpp_caller() -> str:
    src = os.path.join(ROOT, "tests", "cpp", "reference_caller.cpp")
    out = os.path.join(ROOT, "tests", "cpp", "reference_caller")
    tmp = out + ".tmp"
    _run([HIPCC, "-x", "hip", "--offload-arch=gfx950", "-std=c++17", "-O2", "-Wno-implicit-const-int-float-conversion",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{INC}", src, "-o", tmp, f"-L{PKG}",
          "-llatent_attn_hip", "-Wl,-rpath,$ORIGIN/../../latent-attn_amd/latent_attn"])
    os.replace(tmp, out)
    return out


def build(lib_only: bool = False) -> None:
    build_lib()
    if not lib_only:
        build_ext()
        build_cpp_caller()


if __name__ == "__main__":
    if "--phase-stamps" in sys.argv:
        print("built", build_lib(phase_stamps=True))
    else:
        build(lib_only="--lib-only" in sys.argv)
        print("built", os.path.join(PKG, LIB_NAME))
