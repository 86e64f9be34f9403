"""Build the engine library and tools in-tree (no JIT cache, nothing installed).

    python nano-inference_amd/build.py            # libminfer.so + minfer CLI
Outputs go to nano-inference_amd/_build/ (git-ignored; travels to the GPU box).
Device code is compiled for gfx950 only, with -ffp-contract=off (the kernels'
float order is explicit) and packed fp32 ops disabled.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function", "-I", os.path.join(ROOT, "include"), "-I", SRC]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include"), "-I", SRC]

HIP_SOURCES = ["kernels.hip", "engine.hip"]
CXX_SOURCES = ["gguf.cpp", "synth.cpp", "spec.cpp", "detok.cpp", "teacher.cpp"]


def run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), err))
    return err


def build(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    jobs = []
    objs = []
    for s in HIP_SOURCES:
        o = os.path.join(OUT, s.replace(".hip", ".o"))
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(SRC, s), "-o", o])
        objs.append(o)
    for s in CXX_SOURCES:
        o = os.path.join(OUT, s.replace(".cpp", ".o"))
        jobs.append(["g++"] + CXX_FLAGS + ["-c", os.path.join(SRC, s), "-o", o])
        objs.append(o)
    with ThreadPoolExecutor(max_workers=4) as ex:
        for err in ex.map(run, jobs):
            if verbose and err.strip():
                print(err)
    lib = os.path.join(OUT, "libminfer.so")
    run([HIPCC, "-shared", "-fPIC", "-o", lib + ".tmp"] + objs + ["-lpthread"])
    os.replace(lib + ".tmp", lib)
    cli = os.path.join(SRC, "cli.cpp")
    if os.path.exists(cli):
        run(["g++"] + CXX_FLAGS + [cli, "-o", os.path.join(OUT, "minfer"), "-L", OUT, "-lminfer",
                                   "-Wl,-rpath,$ORIGIN"])
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
