"""Build recipe for the MI355X (gfx950) libraries.

  _build/libvrt_hip.so   HIP kernels + the C ABI declared in include/vrt_hip.h
  _build/libvortexrt.so  the vortexrt:: C++ surface (include/vortexrt/*.hpp) over the C ABI
  _build/vortexrt-gemma  the Gemma 3 command line (csrc/cli/gemma_main.cpp) over libvortexrt.so

Every HIP source is compiled for gfx950 with packed-fp32 instruction selection disabled.
Only the vrt_* symbols are exported from libvrt_hip.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shlex
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "_build")
INCLUDE = os.path.join(REPO, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-I" + INCLUDE, "-I" + CSRC,
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument"]
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-I" + INCLUDE, "-Wall", "-Wextra", "-Wno-unused-parameter"]

LIB_HIP = os.path.join(OUT, "libvrt_hip.so")
LIB_CPP = os.path.join(OUT, "libvortexrt.so")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(shlex.quote(c) for c in cmd) + "\n" + r.stdout + r.stderr)
    # hipcc's host pass warns about the device-only target feature; keep other warnings
    noise = ("packed-fp32-ops", "warning: feature flag", "1 warning generated", "warnings generated")
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if l.strip() and not any(n in l for n in noise))
    if msg.strip():
        print(msg, file=sys.stderr)


def build_hip(jobs: int = 8) -> str:
    os.makedirs(OUT, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(OUT, os.path.basename(s)[:-4] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _run([HIPCC] + HIP_FLAGS + ["-c", so[0], "-o", so[1]]), zip(srcs, objs)))
    vers = os.path.join(OUT, "vrt_hip.map")
    with open(vers, "w") as fp:
        fp.write("{ global: vrt_*; local: *; };\n")
    tmp = LIB_HIP + ".tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs +
         ["-Wl,--version-script=" + vers])
    os.replace(tmp, LIB_HIP)
    return LIB_HIP


def build_cpp() -> str:
    """The C++ surface: compiled with the host compiler, linked against libvrt_hip.so."""
    srcs = sorted(glob.glob(os.path.join(CSRC, "host", "*.cpp")))
    if not srcs:
        return ""
    tmp = LIB_CPP + ".tmp"
    _run(["g++"] + CXX_FLAGS + ["-shared", "-o", tmp] + srcs +
         ["-L" + OUT, "-lvrt_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, LIB_CPP)
    return LIB_CPP


CLI = {"gemma_main.cpp": "vortexrt-gemma"}   # command-line programs: source -> executable


def build_cli() -> list:
    """The command-line programs of csrc/cli, linked against libvortexrt.so (rpath $ORIGIN)."""
    out = []
    for src, exe in CLI.items():
        path = os.path.join(OUT, exe)
        _run(["g++"] + CXX_FLAGS + ["-o", path + ".tmp", os.path.join(CSRC, "cli", src), "-L" + OUT, "-lvortexrt",
                                    "-lvrt_hip", "-Wl,-rpath,$ORIGIN"])
        os.replace(path + ".tmp", path)
        out.append(path)
    return out


CPP_TESTS = os.path.join(REPO, "tests", "cpp")


def build_cpp_tests(jobs: int = 8) -> list:
    """The C++ test programs of tests/cpp against libvortexrt.so, into tests/cpp/_build."""
    srcs = sorted(glob.glob(os.path.join(CPP_TESTS, "*.cpp")))
    out_dir = os.path.join(CPP_TESTS, "_build")
    os.makedirs(out_dir, exist_ok=True)
    rpath = "-Wl,-rpath,$ORIGIN/../../../vortex-rt_amd/_build"

    def one(src):
        exe = os.path.join(out_dir, os.path.basename(src)[:-4])
        _run(["g++"] + CXX_FLAGS + ["-I" + CPP_TESTS, "-I" + CSRC, "-o", exe + ".tmp", src, "-L" + OUT, "-lvortexrt",
                                    "-lvrt_hip", rpath])
        os.replace(exe + ".tmp", exe)
        return exe

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        return list(ex.map(one, srcs))


def build_all(jobs: int = 8):
    build_hip(jobs)
    build_cpp()
    build_cli()
    build_cpp_tests(jobs)


if __name__ == "__main__":
    build_all()
    print(LIB_HIP)
