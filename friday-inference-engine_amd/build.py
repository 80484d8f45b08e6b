"""Build recipe of libfriday_attn.so (gfx950 only).

    python friday-inference-engine_amd/build.py     # compile + link, in-tree

Every HIP translation unit under csrc/ is compiled with hipcc for gfx950 and
linked into lib/libfriday_attn.so next to this file. Packed-FP32 instruction
selection is disabled (-packed-fp32-ops) for every device pass.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libfriday_attn.so")
# bench-only: the same library with the decode kernels' phase timestamps compiled in
# (FA_STAMPS=1; bench.py --config stamps), never loaded by the product or the tests
STAMPS_LIB = os.path.join(LIB_DIR, "libfriday_attn_stamps.so")
SOURCES = ["fa_api.cpp", "fa_append.hip", "fa_decode.hip", "fa_prefill.hip", "kq_gemm.hip"]
# benchmark-only helpers (synthetic fill, counter-calibration copy): a separate library
# next to bench.py, not part of the product
BENCHKIT_SRC = os.path.join(HERE, "..", "bench_kit", "fa_benchkit.hip")
BENCHKIT = os.path.join(HERE, "..", "bench_kit", "libfa_benchkit.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


# Per-source device-compiler options: MFMA accumulators in ordinary VGPRs. The default
# AGPR form makes the compiler copy accumulators between AGPRs and VGPRs in the loops
# (every K/V stage in prefill) and inflates the register count by up to ~40 %.
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCE_FLAGS = {"fa_prefill.hip": _VGPR_MFMA, "fa_decode.hip": _VGPR_MFMA, "kq_gemm.hip": _VGPR_MFMA}


def _compile(sources, ex, defines=(), suffix=""):
    objs, jobs = [], []
    for src in sources:
        path = src if os.path.isabs(src) else os.path.join(CSRC, src)
        obj = os.path.join(OBJ, os.path.splitext(os.path.basename(src))[0] + suffix + ".o")
        objs.append(obj)
        jobs.append(ex.submit(_run, [HIPCC, *CFLAGS, *SOURCE_FLAGS.get(src, []), *defines, "-c", path, "-o", obj]))
    return objs, jobs


def _link(objs, target):
    tmp = target + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, target)


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        objs, jobs = _compile(SOURCES, ex)
        bobjs, bjobs = _compile([os.path.abspath(BENCHKIT_SRC)], ex)
        sobjs, sjobs = _compile(["fa_decode.hip"], ex, ["-DFA_STAMPS=1"], "_stamps")
        for j in jobs + bjobs + sjobs:
            out = j.result()
            if verbose and out.strip():
                print(out)
    _link(objs, LIB)
    _link(bobjs, BENCHKIT)
    _link([o if not o.endswith("fa_decode.o") else sobjs[0] for o in objs], STAMPS_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
