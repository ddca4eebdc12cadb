"""Build recipe of liblocals_amd.so: every HIP source under csrc/ compiled for gfx950 into one shared library
(plus libread_probe.so, the bench's streaming-read probe, from probe/read_probe.hip).

Run ``python -m locals_amd.build`` (``__graft_entry__.build()`` calls ``build()``).  The library links the HIP
runtime that torch ships (``torch/lib/libamdhip64.so``), so a process that already imported torch keeps a single
HIP runtime; ``ldd`` on the result shows which one was recorded.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "liblocals_amd.so")
# the bench's streaming-read probe: a library of its own, outside the attention ABI
PROBE_SRC = os.path.join(HERE, "probe", "read_probe.hip")
PROBE_OUT = os.path.join(HERE, "libread_probe.so")
BUILD = os.path.join(ROOT, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed FP32 (v_pk_*_f32) stays off: only scalar fp32 VALU code is emitted
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
    f"-I{CSRC}",
]


def _torch_lib() -> str | None:
    try:
        import importlib.util

        spec = importlib.util.find_spec("torch")
        if spec and spec.origin:
            d = os.path.join(os.path.dirname(spec.origin), "lib")
            if os.path.exists(os.path.join(d, "libamdhip64.so")):
                return d
    except Exception:
        pass
    return None


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(BUILD, os.path.basename(s) + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _run([HIPCC, *FLAGS, "-c", so[0], "-o", so[1]]), zip(srcs, objs)))
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", OUT + ".tmp"]
    tl = _torch_lib()
    if tl:
        link[1:1] = [f"-L{tl}", f"-Wl,-rpath,{tl}"]
    _run(link)
    os.replace(OUT + ".tmp", OUT)
    probe = [HIPCC, *FLAGS, "-shared", PROBE_SRC, "-o", PROBE_OUT + ".tmp"]
    if tl:
        probe[1:1] = [f"-L{tl}", f"-Wl,-rpath,{tl}"]
    _run(probe)
    os.replace(PROBE_OUT + ".tmp", PROBE_OUT)
    if verbose:
        print("built", OUT, "and", PROBE_OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
