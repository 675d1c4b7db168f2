"""Build libgfd_amd.so in-tree: HIP sources with hipcc for gfx950, host C++
with g++, linked by hipcc.  Run ``python -m gfd_amd.builder`` or call build().

Kernels under csrc/aql/ are not part of the HIP fat binary: each is built
device-only into a raw gfx950 code object, embedded in the library as a byte
array (symbol gfd_<name>_code_object) and loaded through the HSA runtime by
the code that dispatches it on a queue of its own.

Objects go to gfd_amd/_build/, the library to gfd_amd/libgfd_amd.so.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgfd_amd.so")
ARCH = os.environ.get("GFD_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CXX = os.environ.get("CXX", "g++")

INCLUDES = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "-I/opt/rocm/include"]
HIP_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17", "-Wall",
    # packed fp32 instructions are not to be generated for this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
CXX_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-pthread", "-Wall", "-Wextra", "-Wno-unused-parameter",
             "-D__HIP_PLATFORM_AMD__"]


AQL = os.path.join(CSRC, "aql")


def sources():
    out = []
    for d, _, files in os.walk(CSRC):
        if os.path.abspath(d).startswith(AQL):
            continue
        for f in sorted(files):
            if f.endswith((".hip", ".cpp")):
                out.append(os.path.join(d, f))
    return sorted(out)


def aql_sources():
    return sorted(os.path.join(AQL, f) for f in os.listdir(AQL) if f.endswith(".hip")) if os.path.isdir(AQL) else []


def _embed_code_object(src):
    """Device-only raw code object of `src`, then a C++ file holding its bytes,
    compiled; returns the object file."""
    name = os.path.splitext(os.path.basename(src))[0]
    co = os.path.join(BUILD, "aql_%s.co" % name)
    cmd = [HIPCC, "-x", "hip", "--cuda-device-only", "--no-gpu-bundle-output"] + HIP_FLAGS + INCLUDES + [
        "-c", src, "-o", co]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    data = open(co, "rb").read()
    cpp = os.path.join(BUILD, "aql_%s_code_object.cpp" % name)
    rows = [", ".join("0x%02x" % b for b in data[i:i + 24]) for i in range(0, len(data), 24)]
    with open(cpp, "w") as f:
        f.write("// Generated from %s by gfd_amd/builder.py.\n#include <cstddef>\n" % os.path.relpath(src, ROOT))
        f.write('extern "C" const unsigned char gfd_%s_code_object[] = {\n%s\n};\n' % (name, ",\n".join(rows)))
        f.write('extern "C" const size_t gfd_%s_code_object_size = sizeof(gfd_%s_code_object);\n' % (name, name))
    obj = cpp + ".o"
    cmd = [CXX] + CXX_FLAGS + ["-c", cpp, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    return obj


def _compile(src):
    rel = os.path.relpath(src, CSRC).replace(os.sep, "_")
    obj = os.path.join(BUILD, rel + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC] + HIP_FLAGS + INCLUDES + ["-c", src, "-o", obj]
    else:
        cmd = [CXX] + CXX_FLAGS + INCLUDES + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name: drop that warning
    err = "\n".join(l for l in r.stderr.splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, err))
    return obj, err.strip()


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = min(8, len(srcs)) or 1
    objs = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        embedded = list(ex.map(_embed_code_object, aql_sources()))
        for obj, warn in ex.map(_compile, srcs):
            objs.append(obj)
            if warn and verbose:
                print(warn, file=sys.stderr)
    objs += embedded
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-o", tmp] + objs + [
        "-L/opt/rocm/lib", "-lhsa-runtime64", "-Wl,-rpath,/opt/rocm/lib", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
