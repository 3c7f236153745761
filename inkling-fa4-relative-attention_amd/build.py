"""Build the gfx950 library and its torch binding in-tree.

Outputs (next to the Python package, git-ignored, shipped with the tree):
  inkling_fa4/libifa4.so        HIP kernels + C ABI (include/ifa4.h); no torch
  inkling_fa4/_ifa4_torch.so    torch.ops.inkling_fa4.{fwd,decode} binding

Usage:  python inkling-fa4-relative-attention_amd/build.py [--jobs N]
Cross-compiles for gfx950 without a GPU.
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "inkling_fa4")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

LIB_SOURCES = ["prefill_fwd.hip", "decode_fwd.hip", "decode_noalloc.hip", "ifa4_api.cpp"]
LIB_NAME = "libifa4.so"
EXT_NAME = "_ifa4_torch.so"

# Device code: gfx950 only; no packed-fp32 VALU forms (v_pk_{add,mul,fma}_f32).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_library(jobs, out_dir=PKG, defines=(), build_dir=BUILD, csrc=CSRC, include=INCLUDE):
    """Compile the kernels and the C ABI into out_dir/libifa4.so.  `defines`:
    extra -D flags (tile-sweep knobs of the kernel sources); `csrc` / `include`:
    source directories (a sweep builds every variant from one snapshot)."""
    os.makedirs(build_dir, exist_ok=True)
    flags = [f for f in HIP_FLAGS if not f.startswith("-I")] + [f"-I{include}", f"-I{csrc}"]
    flags += [f"-D{d}" for d in defines]
    objs = []
    cmds = []
    for src in LIB_SOURCES:
        obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmds.append([HIPCC] + flags + lang + ["-c", os.path.join(csrc, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, out)
    return out


def build_torch_binding():
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths()
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = os.path.join(PKG, EXT_NAME)
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           os.path.join(CSRC, "torch_ext.cpp"), "-o", tmp,
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-I{INCLUDE}", f"-I{ROCM}/include"]
    cmd += [f"-I{p}" for p in inc]
    cmd += [f"-L{p}" for p in libdirs] + [f"-L{PKG}", f"-L{ROCM}/lib"]
    cmd += ["-lifa4", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch", "-lamdhip64",
            "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(jobs=4):
    lib = build_library(jobs)
    ext = build_torch_binding()
    return lib, ext


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--lib-only", action="store_true")
    args = ap.parse_args()
    lib = build_library(args.jobs)
    print("built", os.path.relpath(lib, REPO))
    if not args.lib_only:
        ext = build_torch_binding()
        print("built", os.path.relpath(ext, REPO))
    return 0


if __name__ == "__main__":
    sys.exit(main())
