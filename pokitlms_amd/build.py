"""Build recipe of libpokit_hip.so (hand-written HIP for gfx950).

``python -m pokitlms_amd.build`` compiles every ``csrc/*.hip`` translation unit
with hipcc for gfx950 and links them into ``pokitlms_amd/libpokit_hip.so``,
in-tree, so the library travels with the source tree to the GPU host.  It
also compiles and runs ``host/expf_table.c``, which writes ``libm_expf.bin``:
the float inputs on which this host's libm ``expf`` differs from the correctly
rounded exponential, with libm's results (the reference-order decode uses them
to return the CPU's bits).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpokit_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
EXPF_TABLE = os.path.join(HERE, "libm_expf.bin")

# -ffp-contract=off: every fused multiply-add is written out (fmaf), so the
# bit-exact router recurrence and the reference's unfused orders stay intact.
# The target-feature switch keeps hipcc from emitting packed-FP32 VALU ops.
# Kernel-argument preloading: the leading scalar and pointer arguments of a
# kernel arrive in SGPRs with the wave instead of through a load of the
# argument block (the code object keeps the loading path for firmware that
# does not preload).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _compile(src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build_expf_table(obj_dir: str) -> str:
    """Compile the libm expf scan with gcc and write EXPF_TABLE (about 8 s on
    8 cores: every finite float is evaluated once)."""
    exe = os.path.join(obj_dir, "expf_table")
    src = os.path.join(HERE, "host", "expf_table.c")
    r = subprocess.run(["gcc", "-O2", "-pthread", src, "-o", exe, "-lm"], capture_output=True,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed for {src}:\n{r.stderr[-4000:]}")
    tmp = EXPF_TABLE + ".tmp"
    r = subprocess.run([exe, tmp], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"expf_table failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, EXPF_TABLE)
    return EXPF_TABLE


def build(verbose: bool = False) -> str:
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    build_expf_table(obj_dir)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
