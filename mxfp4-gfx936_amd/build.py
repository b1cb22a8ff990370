"""Build libmxfp4_gfx950.so for MI355X (gfx950) in-tree.

``python mxfp4-gfx936_amd/build.py`` compiles every ``csrc/*.hip`` with
hipcc (in parallel, objects under ``_build/``) and links
``mxfp4_amd/libmxfp4_gfx950.so`` next to the Python package that loads it,
and ``mxfp4_amd/libmxfp4_probe.so`` (``csrc/probe/``: a plain HBM read that
bench.py times as the floor of the decode kernels; not part of the library).

Flags: ``-O3`` for gfx950 only; packed-FP32 instruction selection is turned
off (``-Xclang -target-feature -Xclang -packed-fp32-ops``); denormals are
kept (no fast-math / flush-to-zero), which the bit-exact dequant and the
subnormal E8M0 scale (s = 0 -> 2^-127) rely on.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
OBJ_DIR = os.path.join(HERE, "_build")
GEN_DIR = os.path.join(OBJ_DIR, "gen")  # generated sources (silu_table.inc)
LIB = os.path.join(HERE, "mxfp4_amd", "libmxfp4_gfx950.so")
# measurement aid for bench.py (a plain HBM read), kept out of the library
PROBE_SRC = os.path.join(CSRC, "probe", "read_floor.hip")
PROBE_LIB = os.path.join(HERE, "mxfp4_amd", "libmxfp4_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{GEN_DIR}",
]


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so;
    # that line is expected, anything else is shown.
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
    if msgs and verbose:
        print("\n".join(msgs), flush=True)
    return obj


def build(verbose: bool = False) -> str:
    """Compile all HIP sources and link the shared library; returns its path."""
    os.makedirs(GEN_DIR, exist_ok=True)
    sys.path.insert(0, HERE)
    import silu_table  # the SiLU lookup tables of csrc/silu.h
    silu_table.write_inc(os.path.join(GEN_DIR, "silu_table.inc"))
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    tmp = PROBE_LIB + ".tmp"
    cmd = [HIPCC, *CFLAGS, "-shared", PROBE_SRC, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC}:\n{res.stdout}{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
