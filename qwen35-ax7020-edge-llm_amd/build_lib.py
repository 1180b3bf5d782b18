"""Build libqwen_kernels.so (gfx950) in-tree with hipcc.

    python qwen35-ax7020-edge-llm_amd/build_lib.py

Translation units:
  csrc/bfp8_ftz.hip          GEMV kernels, f32 flush-to-zero (Advanced SIMD semantics)
  csrc/bfp8_ieee.hip         quantizer / scalar-order kernels, IEEE subnormals
  csrc/select.hip            general top-k selection (tile lists, sort) and the sampler, IEEE
  csrc/noalloc.hip           the fixed device scratch of the no-alloc lm_head entry point
  csrc/bf16_head.hip         bf16 tied-embedding lm_head, f32 flush-to-zero
  csrc/runtime_ftz.hip       decode runtime kernels (norms, conv, GDN, swiglu), f32 flush-to-zero
  csrc/fused_gemv.hip        the forward's GEMVs with their activation prologue, f32 flush-to-zero
  csrc/sweep.hip             a whole plan in one launch (a tile queue, LDS-quantized activations, in-launch top-k)
  csrc/batch_mfma.hip        the batched GEMV (8..16 vectors) on the matrix cores, f32 flush-to-zero
  csrc/qwen_kernels_api.cpp  C ABI host code (include/qwen_kernels.h)
  csrc/qwen_runtime_api.cpp  C ABI of the runtime kernels and the forward loop
  csrc/qwen_weights.cpp      manifest-driven weight-image loader

Every device TU is built with -ffp-contract=off (no fused multiply-add: the
reference rounds every product and sum) and without packed FP32 ops.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libqwen_kernels.so"
OUT_SAMPLING = PKG / "libqwen_sampling.so"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-fvisibility=hidden",
    f"-I{CSRC}", f"-I{ROOT / 'include'}",
]
UNITS = {
    "bfp8_ftz.hip": ["-fgpu-flush-denormals-to-zero"],
    "bf16_head.hip": ["-fgpu-flush-denormals-to-zero"],
    "runtime_ftz.hip": ["-fgpu-flush-denormals-to-zero"],
    "fused_gemv.hip": ["-fgpu-flush-denormals-to-zero"],
    # (the ticket atomic stays one plain atomic: no wave-level combining,
    # whose result arithmetic would wait for every load in flight)
    "sweep.hip": ["-fgpu-flush-denormals-to-zero", "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
    # MFMA results straight into VGPRs (no accumulator-register copies)
    "batch_mfma.hip": ["-fgpu-flush-denormals-to-zero", "-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "bfp8_ieee.hip": [],
    "select.hip": [],
    "noalloc.hip": [],
    "qwen_kernels_api.cpp": [],
    "qwen_runtime_api.cpp": [],
    "qwen_weights.cpp": [],
}


def _compile(src: str, extra: list[str]) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(UNITS)) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), UNITS.items()))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, OUT)
    # libqwen_sampling.so: host-only forwarding library, resolved next to
    # libqwen_kernels.so through its run path
    tmp = OUT_SAMPLING.with_suffix(".so.tmp")
    cmd = [HIPCC, "-O2", "-fPIC", "-shared", "-std=c++17", "-fvisibility=hidden", f"-I{ROOT / 'include'}",
           str(CSRC / "qwen_sampling.cpp"), "-o", str(tmp), f"-L{PKG}", "-lqwen_kernels", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("libqwen_sampling.so link failed")
    os.replace(tmp, OUT_SAMPLING)
    if verbose:
        print(f"built {OUT} and {OUT_SAMPLING}")
    return OUT


# Host code under AddressSanitizer + UndefinedBehaviorSanitizer, for the CPU
# tests only (tests/test_sanitizers.py): the sanitizers apply to the host side
# of every unit (-Xarch_host); the device code is built as usual.  The
# sanitizer runtime is not linked in: the test preloads clang's into the
# Python process.
SAN_BUILD = PKG / "_build_san"
SAN_OUT = PKG / "_san" / "libqwen_kernels.so"
SAN_FLAGS = ["-O1", "-g", "-fPIC", "-std=c++17", "-ffp-contract=off", f"-I{CSRC}", f"-I{ROOT / 'include'}",
             "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]


def build_sanitized(verbose: bool = False) -> Path:
    SAN_BUILD.mkdir(exist_ok=True)
    SAN_OUT.parent.mkdir(exist_ok=True)

    def comp(src: str) -> Path:
        obj = SAN_BUILD / (Path(src).stem + ".o")
        dev = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               *UNITS[src]] if src.endswith(".hip") else []
        res = subprocess.run([HIPCC, *dev, *SAN_FLAGS, "-c", str(CSRC / src), "-o", str(obj)], capture_output=True,
                             text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"sanitized hipcc failed on {src}")
        return obj

    with ThreadPoolExecutor(max_workers=len(UNITS)) as ex:
        objs = list(ex.map(comp, UNITS))
    tmp = SAN_OUT.with_suffix(".so.tmp")
    res = subprocess.run([HIPCC, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("sanitized link failed")
    os.replace(tmp, SAN_OUT)
    if verbose:
        print(f"built {SAN_OUT}")
    return SAN_OUT


if __name__ == "__main__":
    if "--sanitize" in sys.argv[1:]:
        build_sanitized(verbose=True)
    else:
        build(verbose=True)
