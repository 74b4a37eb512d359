"""Builds morphocore_amd's native code for AMD Instinct MI355X (gfx950), in place:

    python setup.py build_ext --inplace [--force]

Two shared libraries, both written for gfx950 only:
  * morphocore_amd/libmorphocore_amd.so — the hand-written HIP kernels and their C ABI
    (include/morphocore_amd.h), compiled by hipcc with --offload-arch=gfx950; it depends only on the
    HIP runtime;
  * morphocore_amd/_C*.so — the PyTorch-ROCm extension that registers torch.ops.morphocore.* and its
    C++ autograd Functions (csrc/torch_ops.cpp, host code compiled against torch's headers), linked
    to the kernel library.
The sources are HIP and C++ only: no CUDA sources, no hipify step, no Triton. Objects are rebuilt when
a source or a shared header is newer than them (--force rebuilds everything); sources compile in
parallel. (Reference counterpart: setup.py:101-125, a CppExtension / CUDAExtension "morphocore._C".)
"""
import os
import shlex
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

from setuptools import Extension, setup
from setuptools.command.build_ext import build_ext

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "morphocore_amd")
CSRC = os.path.join(PKG, "csrc")
OBJDIR = os.path.join(CSRC, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM_INCLUDE = "/opt/rocm/include"

KERNEL_SOURCES = ["morpho_fwd.hip", "morpho_fwd_half.hip", "morpho_bwd.hip", "morpho_ident.hip", "morpho_fused.hip", "smorph.hip", "smorph_static.hip", "util.hip", "capi.cpp", "stack.cpp"]
KERNEL_HEADERS = ["common.hpp", "launch.hpp", "morpho_fwd.hpp", "smorph_common.hpp", os.path.join("..", "..", "include", "morphocore_amd.h")]
# Packed FP32 instructions stay disabled: only scalar fp32 VALU forms are emitted.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
KERNEL_LIB = os.path.join(PKG, "libmorphocore_amd.so")


def _run(cmd):
    print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    subprocess.run(cmd, check=True)


def _stale(target, deps, force):
    if force or not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


class HipBuildExt(build_ext):
    """build_ext that compiles the gfx950 kernel library with hipcc, then the torch extension."""

    def build_extensions(self):
        self._build_kernel_library()
        for ext in self.extensions:
            self._build_torch_extension(ext)

    def _jobs(self):
        return max(1, min(int(os.environ.get("MAX_JOBS", "8")), os.cpu_count() or 1))

    def _build_kernel_library(self):
        os.makedirs(OBJDIR, exist_ok=True)
        headers = [os.path.normpath(os.path.join(CSRC, h)) for h in KERNEL_HEADERS]
        jobs, objs = [], []
        for src in KERNEL_SOURCES:
            path = os.path.join(CSRC, src)
            obj = os.path.join(OBJDIR, src + ".o")
            objs.append(obj)
            if _stale(obj, [path] + headers, self.force):
                jobs.append([HIPCC] + HIP_FLAGS + ["-c", path, "-o", obj])
        with ThreadPoolExecutor(self._jobs()) as pool:
            for f in [pool.submit(_run, j) for j in jobs]:
                f.result()
        if jobs or _stale(KERNEL_LIB, objs, self.force):
            _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", KERNEL_LIB + ".tmp"])
            os.replace(KERNEL_LIB + ".tmp", KERNEL_LIB)

    def _build_torch_extension(self, ext):
        import torch
        from torch.utils import cpp_extension

        target = self.get_ext_fullpath(ext.name)
        os.makedirs(os.path.dirname(target), exist_ok=True)
        torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
        deps = list(ext.sources) + [os.path.join(ROOT, "include", "morphocore_amd.h"), KERNEL_LIB]
        if not _stale(target, deps, self.force):
            return
        abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
        cxx = os.environ.get("CXX", "g++")
        includes = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], ROCM_INCLUDE]
        cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
                  "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C"]
        obj = os.path.join(OBJDIR, "torch_ops.cpp.o")
        _run([cxx] + cflags + [f"-I{p}" for p in includes] + ["-c", ext.sources[0], "-o", obj])
        libdir = os.path.dirname(KERNEL_LIB)
        # The extension finds libmorphocore_amd.so next to itself; torch's libraries (and the HIP
        # runtime torch loads) are already in the process when it is imported.
        _run([cxx, "-shared", obj, "-o", target + ".tmp", f"-L{libdir}", "-lmorphocore_amd", "-Wl,-rpath,$ORIGIN", f"-L{torch_lib}",
              "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lamdhip64", f"-Wl,-rpath,{torch_lib}"])
        os.replace(target + ".tmp", target)


setup(
    name="morphocore_amd",
    version="0.13.1",
    description="morphocore's dilation / erosion / smorph hot path as HIP kernels for AMD Instinct MI355X (gfx950)",
    packages=["morphocore_amd", "morphocore_amd.functional", "morphocore_amd.nn"],
    ext_modules=[Extension("morphocore_amd._C", sources=[os.path.join("morphocore_amd", "csrc", "torch_ops.cpp")])],
    cmdclass={"build_ext": HipBuildExt},
    python_requires=">=3.9",
)
