"""Build libforgeserve_hip.so (the gfx950 kernels behind the C ABI of include/forgeserve_amd.h).

hipcc cross-compiles for gfx950 without a GPU. Each .hip file becomes one object (compiled in
parallel), then the objects are linked in-tree into forgeserve_amd/libforgeserve_hip.so, which is
the file the Python package loads.

    python -m forgeserve_amd.build            # build
    python -m forgeserve_amd.build --check    # build, then list the exported fs_* symbols
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libforgeserve_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: a*b - c*d stays two roundings, as in the PyTorch reference.
# -packed-fp32-ops: keep the compiler from emitting packed f32 VALU instructions.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]

SOURCES = ["abi.hip", "kv.hip", "attention.hip", "norm.hip", "gemm.hip", "sample.hip", "rng.hip"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in p.stdout.splitlines() if "is not a recognized feature for this target" not in line)
    return p.returncode, out


def build(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        rc, out = _run(cmd)
        return src, obj, rc, out, cmd

    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(SOURCES)))) as ex:
        results = list(ex.map(compile_one, SOURCES))
    failed = [r for r in results if r[2] != 0]
    for src, _, rc, out, cmd in results:
        if verbose or rc != 0:
            if out.strip():
                print(f"--- {src}\n{out}", file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(r[0] for r in failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[r[1] for r in results]]
    rc, out = _run(cmd)
    if rc != 0:
        raise RuntimeError("link failed:\n" + out)
    os.replace(tmp, LIB)
    return LIB


def exported_symbols(path: str = LIB):
    rc, out = _run(["nm", "-D", "--defined-only", path])
    if rc != 0:
        raise RuntimeError(out)
    return sorted(line.split()[-1] for line in out.splitlines() if line.split() and line.split()[-1].startswith("fs_"))


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
    if "--check" in sys.argv:
        print("\n".join(exported_symbols(path)))
