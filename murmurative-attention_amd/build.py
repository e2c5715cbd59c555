"""Build the MI355X (gfx950) libraries in-tree.

    python murmurative-attention_amd/build.py [--jobs N]

Outputs, next to the Python package (murmurative-attention_amd/murmurative/):
  libmurmurative_hip.so           HIP kernels + the C ABI of include/murmurative_hip.h
  murmurative_attention_ops.so    PyTorch extension registering torch.ops.murmurative_attention
                                  (links libmurmurative_hip.so through $ORIGIN)

HIP sources are compiled with hipcc directly (no hipify pass); the torch
binding is host-only C++ compiled with g++ against the installed PyTorch.
"""

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
TEXT = os.path.join(HERE, "torch-ext")
PKG = os.path.join(HERE, "murmurative")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

EXT_SOURCES = ["torch_binding.cpp", "wrappers.cpp"]


def hip_units():
    """(source, object name, extra flags) of every HIP translation unit: each
    csrc/*.hip once, except murm_tokens.hip, built once per token dtype."""
    units = []
    for src in sorted(f for f in os.listdir(CSRC) if f.endswith(".hip")):
        stem = src[:-4]
        if src == "murm_tokens.hip":
            for dt, sfx in ((0, "f32"), (1, "f16"), (2, "bf16")):
                units.append((src, f"{stem}_{sfx}.o", [f"-DMURM_TOKENS_DT={dt}"]))
        else:
            units.append((src, stem + ".o", []))
    return units

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-mcode-object-version=5",
    "-fno-gpu-flush-denormals-to-zero",
    # packed fp32 VALU forms stay off (hipcc -O3 would otherwise emit them)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"build step failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _torch_flags():
    import torch
    from torch.utils import cpp_extension as ce
    inc = ce.include_paths()
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=murmurative_attention_ops",
              f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}", f"-I{ROCM}/include"]
    cflags += [f"-I{p}" for p in inc]
    ldflags = [f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10_hip",
               "-ltorch_python", f"-L{PKG}", "-lmurmurative_hip",
               "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    return cflags, ldflags


def _stale(obj, deps):
    """True when obj is missing or older than any of its dependencies."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in deps)


def build(jobs: int = 8, verbose: bool = False, incremental: bool = False):
    """Compile everything (incremental=True skips objects newer than their
    source and every header they may include)."""
    os.makedirs(BUILD, exist_ok=True)
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    headers += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    units = hip_units()
    hip_objs = [os.path.join(BUILD, o) for _, o, _ in units]
    cflags, ldflags = _torch_flags()
    ext_objs = [os.path.join(BUILD, s.replace(".cpp", ".o")) for s in EXT_SOURCES]
    ext_hdrs = headers + [os.path.join(TEXT, f) for f in os.listdir(TEXT) if f.endswith(".h")]

    def hip_job(i):
        src, _, extra = units[i]
        if incremental and not _stale(hip_objs[i], [os.path.join(CSRC, src)] + headers):
            return ""
        return _run(["hipcc", *HIPCC_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", hip_objs[i]])

    def ext_job(i):
        src = os.path.join(TEXT, EXT_SOURCES[i])
        if incremental and not _stale(ext_objs[i], [src] + ext_hdrs):
            return ""
        return _run(["g++", *cflags, "-c", src, "-o", ext_objs[i]])

    # the slowest units first, so they start while the rest are queued
    order = sorted(range(len(units)), key=lambda i: units[i][0] != "murm_tokens.hip")
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(hip_job, i) for i in order]
        futs += [ex.submit(ext_job, i) for i in range(len(EXT_SOURCES))]
        logs = [f.result() for f in futs]
    lib = os.path.join(PKG, "libmurmurative_hip.so")
    if not incremental or _stale(lib, hip_objs):
        _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libmurmurative_hip.so",
              *hip_objs, "-o", lib + ".tmp"])
        os.replace(lib + ".tmp", lib)
    ext = os.path.join(PKG, "murmurative_attention_ops.so")
    if not incremental or _stale(ext, ext_objs + [lib]):
        _run(["g++", "-shared", *ext_objs, "-o", ext + ".tmp", *ldflags])
        os.replace(ext + ".tmp", ext)
    if verbose:
        for l in logs:
            if l.strip():
                print(l)
    return lib, ext


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("-i", "--incremental", action="store_true",
                    help="skip objects newer than their sources and headers")
    a = ap.parse_args()
    lib, ext = build(a.jobs, a.verbose, a.incremental)
    print("built", os.path.relpath(lib, ROOT), os.path.relpath(ext, ROOT))


if __name__ == "__main__":
    sys.exit(main())
