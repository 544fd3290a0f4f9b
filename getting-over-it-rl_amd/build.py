"""Build libgoi_b2.so for gfx950 in-tree (getting-over-it-rl_amd/lib/libgoi_b2.so).

Flags: no FMA contraction, IEEE division and square root, denormals kept (one rounding per C operation, as the
reference's float32 discipline requires), packed-FP32 instructions disabled.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = [HERE / "csrc" / "goi_b2.hip", HERE / "csrc" / "goi_b2_rig.hip", HERE / "csrc" / "goi_b2_island.hip"]
OUT = HERE / "lib" / "libgoi_b2.so"

FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc():
    h = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(h).exists():
        raise FileNotFoundError("hipcc not found")
    return h


def build(out=OUT, extra=()):
    out = Path(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, *extra, "-parallel-jobs=3", "-o", str(tmp), *map(str, SRC)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode})")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
