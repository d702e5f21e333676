"""Build the native libraries of the kq package in-tree.

* ``kq/libkq.so``     -- HIP kernels + C ABI (include/kq.h), gfx950 only, built with hipcc.
* ``kq/libkqhost.so`` -- host-side synthetic weight quantizer (include/kq_host.h), g++ + OpenMP.

Every HIP translation unit is compiled with -ffp-contract=off (the numerical contract of the
kernels spells out each fused multiply-add explicitly) and with packed fp32 instructions disabled.
Run ``python oxcoder-9b_amd/build.py`` or call ``build()``.
"""
import concurrent.futures as cf
import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "kq")
OBJ = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["api.hip", "q8k_quantize.hip", "producers.hip", "argmax.hip", "gemv_q8k.hip", "gemv_mfma.hip",
               "gemv_f32.hip", "gemm_q8k.hip"]
HIP_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I" + CSRC, "-I" + os.path.join(ROOT, "include"),
]
# No -fgpu-flush-denormals-to-zero or fast-math: the fp32-activation GEMV multiplies each weight code as an
# f16 subnormal (v_fma_mix_f32 with the code in a half's mantissa bits), so f16 denormals must stay on (the
# default denormal mode 3; tests/test_gpu_exact.py fails at once otherwise).
# Per-source extra flags.  The MFMA kernels keep their accumulators in ordinary VGPRs (the epilogue
# reads them with VALU instructions every super-block; accumulators in AGPRs would need a copy each).
# The decode and verify kernels (GEMV, small-batch MFMA GEMV, quantizer, producers, argmax) take their
# leading scalar arguments preloaded into scalar registers at dispatch, so a wave's first loads wait
# for no argument fetch (decode layer step 39.1 -> 37.7 us).
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
HIP_EXTRA = {"gemm_q8k.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
             "gemv_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"] + PRELOAD,
             "gemv_q8k.hip": PRELOAD, "q8k_quantize.hip": PRELOAD, "producers.hip": PRELOAD, "argmax.hip": PRELOAD}
HOST_SOURCES = ["host/quantize_weights.cpp"]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
              "-fno-math-errno", "-Wall", "-I" + os.path.join(ROOT, "include")]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError("build step failed: " + os.path.basename(cmd[-1]))
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected.
    noise = "is not a recognized feature for this target"
    rest = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if rest.strip():
        sys.stderr.write(rest + "\n")


def source_hash():
    """sha256 (first 16 hex digits) of every source that decides libkq's arithmetic: the kernels,
    their headers and include/kq.h, in name order.  Compiled into the library (kq_source_hash) so
    an engine can key saved states on the code that made them."""
    h = hashlib.sha256()
    files = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".h")))
    for f in files + ["../../include/kq.h"]:
        path = os.path.normpath(os.path.join(CSRC, f))
        h.update(os.path.basename(path).encode() + b"\0" + open(path, "rb").read())
    return h.hexdigest()[:16]


def _compile_hip(src):
    extra = HIP_EXTRA.get(src, [])
    if src == "api.hip":
        extra = extra + ['-DKQ_SOURCE_HASH="%s"' % source_hash()]
    obj = os.path.join(OBJ, os.path.splitext(os.path.basename(src))[0] + ".o")
    _run([HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build(jobs=8):
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile_hip, HIP_SOURCES))
    so = os.path.join(OUT, "libkq.so")
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", so + ".tmp"])
    os.replace(so + ".tmp", so)
    host = os.path.join(OUT, "libkqhost.so")
    _run(["g++", *HOST_FLAGS, *[os.path.join(CSRC, s) for s in HOST_SOURCES], "-o", host + ".tmp"])
    os.replace(host + ".tmp", host)
    return so, host


if __name__ == "__main__":
    for p in build():
        print("built", os.path.relpath(p, ROOT))
