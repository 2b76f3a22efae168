"""Build libfvsr.so (all HIP kernels + the C ABI) for gfx950, in-tree.

    python flashvsr-sm89-ops_amd/build.py [-j N]

Each csrc/*.hip is compiled to an object under _build/ in parallel, then
linked into flashvsr_sm89_ops/libfvsr.so next to the Python package that
loads it.  First, csrc/gelu_table_gen.c is compiled with gcc and run to
write _build/gelu_table.inc (the bf16 GELU lookup table the quantisation
kernels embed).  Flags: -O3 for gfx950 only, packed-fp32 instructions disabled
(hipcc's host pass prints that it does not know the feature; harmless).
"""
import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "flashvsr_sm89_ops", "libfvsr.so")
ARCH = os.environ.get("FVSR_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

CC = os.environ.get("CC", shutil.which("gcc") or "gcc")

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-I", OUT_DIR,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _gelu_table() -> None:
    """Generate _build/gelu_table.inc with the host generator."""
    exe = os.path.join(OUT_DIR, "gelu_table_gen")
    subprocess.run([CC, "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(CSRC, "gelu_table_gen.c"), "-o", exe, "-lm"], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    if out.count("0x") != 65536:
        raise RuntimeError("gelu_table_gen produced a short table")
    tmp = os.path.join(OUT_DIR, "gelu_table.inc.tmp")
    with open(tmp, "w") as fh:
        fh.write(out)
    os.replace(tmp, os.path.join(OUT_DIR, "gelu_table.inc"))


def build(jobs: int = 8) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    _gelu_table()
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True, capture_output=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    print(build(ap.parse_args().j))
