"""Python side of the MI355X BFP8 GEMV library.

Mirrors how the reference engine binds its operator library
(04/qwen_real_engine.py:656-725 loads libqwen_kernels.so with ctypes, calls
init_kernels() and declares argtypes; :848-866 rebinds the fast-path symbols;
:1221-1240 ``gemv_bfp8`` calls ``bfp8_gemv(y, x, mant, exps, M, K)`` on numpy
views of the weight mmap).  ``bind`` declares exactly those argtypes, so an
engine that loads this library gets the same ctypes behaviour.

On top of that, device-resident helpers (PyTorch tensors as plain device
memory, torch's current stream as the HIP stream) expose the ``bfp8_dev_*``
and ``bfp8_plan_*`` entry points used by the tests and the benchmark.

There is no CPU fallback: every entry point runs on the GPU, and a missing
library raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_double, c_float, c_int, c_size_t, c_uint64, c_void_p
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libqwen_kernels.so"

BFP8_OK, BFP8_EINVAL, BFP8_EHIP, BFP8_ENOMEM = 0, -1, -2, -3

# Reference symbols whose signatures the engine binds (04/qwen_real_engine.py).
REFERENCE_SYMBOLS = ("add_residual", "bfp8_gemv", "causal_conv1d_update_silu", "forward_linear_layer",
                     "forward_mlp", "forward_token_c", "gdn_gates", "gdn_recurrent_step", "init_kernels",
                     "lm_head_argmax", "qk_l2norm", "qwen_prof_count", "qwen_prof_enable", "qwen_prof_get",
                     "qwen_prof_name", "qwen_prof_reset", "rmsnorm", "rmsnorm_gated", "swiglu")


class bfp8_plan_item(ctypes.Structure):
    """Mirror of ``bfp8_plan_item`` (include/qwen_kernels.h)."""

    _fields_ = [
        ("x", c_void_p), ("y", c_void_p), ("mant_gpu", c_void_p), ("exps_gpu", c_void_p),
        ("M", c_int), ("K", c_int), ("topk", c_int),
        ("out_ids", c_void_p), ("out_scores", c_void_p), ("out_count", c_void_p),
        ("out_argmax", c_void_p),
    ]


# void (*)(int layer, float* h, void* ctx), 04/qwen_real_engine.py:979
FULL_ATTN_CALLBACK = ctypes.CFUNCTYPE(None, c_int, c_void_p, c_void_p)


class LinearLayerPlan(ctypes.Structure):
    """Mirror of ``LinearLayerPlan`` (include/qwen_kernels.h), field for field
    the engine's ``LinearLayerPlanC`` (04/qwen_real_engine.py:20-56)."""

    _fields_ = [
        ("in_ln_w", c_void_p), ("mant_qkv", c_void_p), ("exp_qkv", c_void_p), ("M_qkv", c_int), ("K_qkv", c_int),
        ("conv_w", c_void_p), ("conv_s", c_void_p), ("wa", c_void_p), ("wb", c_void_p), ("nea", c_void_p),
        ("dt", c_void_p), ("state", c_void_p), ("mant_z", c_void_p), ("exp_z", c_void_p), ("M_z", c_int),
        ("K_z", c_int), ("norm_w", c_void_p), ("mant_o", c_void_p), ("exp_o", c_void_p), ("M_o", c_int),
        ("K_o", c_int), ("post_ln_w", c_void_p), ("mant_gate", c_void_p), ("exp_gate", c_void_p),
        ("M_gate", c_int), ("K_gate", c_int), ("mant_up", c_void_p), ("exp_up", c_void_p), ("M_up", c_int),
        ("K_up", c_int), ("mant_down", c_void_p), ("exp_down", c_void_p), ("M_down", c_int), ("K_down", c_int),
    ]


class MlpPlan(ctypes.Structure):
    """Mirror of ``MlpPlan`` (include/qwen_kernels.h; the engine's ``MlpPlanC``)."""

    _fields_ = [
        ("post_ln_w", c_void_p), ("mant_gate", c_void_p), ("exp_gate", c_void_p), ("M_gate", c_int),
        ("K_gate", c_int), ("mant_up", c_void_p), ("exp_up", c_void_p), ("M_up", c_int), ("K_up", c_int),
        ("mant_down", c_void_p), ("exp_down", c_void_p), ("M_down", c_int), ("K_down", c_int),
    ]


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    """Declare argtypes/restypes of every exported symbol."""
    vp, i = c_void_p, c_int
    # reference symbols, as the engine declares them (04/qwen_real_engine.py:680-685, :864-866)
    lib.init_kernels.argtypes = []
    lib.init_kernels.restype = None
    lib.bfp8_gemv.argtypes = [vp, vp, vp, vp, i, i]
    lib.bfp8_gemv.restype = None
    lib.qwen_prof_enable.argtypes = [i]
    lib.qwen_prof_enable.restype = None
    lib.qwen_prof_reset.argtypes = []
    lib.qwen_prof_reset.restype = None
    lib.qwen_prof_count.argtypes = []
    lib.qwen_prof_count.restype = i
    lib.qwen_prof_get.argtypes = [i]
    lib.qwen_prof_get.restype = c_double
    lib.qwen_prof_name.argtypes = [i]
    lib.qwen_prof_name.restype = ctypes.c_char_p
    # new host-pointer symbols
    lib.bfp8_lm_head_topk.argtypes = [vp, vp, vp, i, i, i, vp, vp]
    lib.bfp8_lm_head_topk.restype = i
    lib.bfp8_lm_head_argmax.argtypes = [vp, vp, vp, i, i]
    lib.bfp8_lm_head_argmax.restype = i
    lib.bfp8_gemv_batch.argtypes = [vp, vp, vp, vp, i, i, i]
    lib.bfp8_gemv_batch.restype = None
    lib.bfp8_gemv_fallback.argtypes = [vp, vp, vp, vp, i, i, i]
    lib.bfp8_gemv_fallback.restype = i
    lib.bfp8_dev_gemv_fallback.argtypes = [vp, vp, vp, vp, i, i, i, vp]
    lib.bfp8_dev_gemv_fallback.restype = i
    # the bf16 tied-embedding lm_head (04/qwen_real_engine.py:691-696) and sampler
    lib.lm_head_argmax.argtypes = [vp, vp, i, i]
    lib.lm_head_argmax.restype = i
    lib.qwen_lm_head_topk_bf16.argtypes = [vp, vp, i, i, i, vp, vp]
    lib.qwen_lm_head_topk_bf16.restype = i
    lib.qwen_sample_from_topk.argtypes = [vp, vp, i, c_float, i, c_float, vp]
    lib.qwen_sample_from_topk.restype = i
    # the decode runtime and forward loop, as the engine binds them
    # (04/qwen_real_engine.py:676-725, :852-880, :978-985)
    f = c_float
    lib.rmsnorm.argtypes = [vp, vp, vp, i, f]
    lib.swiglu.argtypes = [vp, vp, vp, i]
    lib.add_residual.argtypes = [vp, vp, i]
    lib.causal_conv1d_update_silu.argtypes = [vp, vp, vp, vp, i]
    lib.qk_l2norm.argtypes = [vp, vp, i, i]
    lib.gdn_gates.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i]
    lib.gdn_recurrent_step.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i]
    lib.rmsnorm_gated.argtypes = [vp, vp, vp, vp, i, i, f]
    lib.forward_linear_layer.argtypes = [vp, vp]
    lib.forward_mlp.argtypes = [vp, vp]
    for name in ("rmsnorm", "swiglu", "add_residual", "causal_conv1d_update_silu", "qk_l2norm", "gdn_gates",
                 "gdn_recurrent_step", "rmsnorm_gated", "forward_linear_layer", "forward_mlp"):
        getattr(lib, name).restype = None
    lib.forward_token_c.argtypes = [i, vp, vp, vp, vp, vp, vp, FULL_ATTN_CALLBACK, vp]
    lib.forward_token_c.restype = i
    lib.qwen_forward_state_resident.argtypes = [i]
    lib.qwen_forward_state_resident.restype = i
    lib.qwen_forward_reset_state.argtypes = []
    lib.qwen_forward_reset_state.restype = None
    lib.qwen_forward_sync_state.argtypes = []
    lib.qwen_forward_sync_state.restype = None
    # the weight-image loader
    lib.qwen_weights_scan.argtypes = [ctypes.c_char_p, c_size_t, vp, vp, vp, vp]
    lib.qwen_weights_scan.restype = i
    lib.qwen_weights_preload.argtypes = [vp, c_size_t, ctypes.c_char_p]
    lib.qwen_weights_preload.restype = i
    lib.qwen_weights_find.argtypes = [ctypes.c_char_p, vp, vp, vp, vp]
    lib.qwen_weights_find.restype = i
    lib.bfp8_dev_pack_rows.argtypes = [vp, vp, vp, i, i, vp]
    lib.bfp8_dev_pack_rows.restype = i
    lib.bfp8_last_error.argtypes = []
    lib.bfp8_last_error.restype = ctypes.c_char_p
    lib.bfp8_gpu_ready.argtypes = []
    lib.bfp8_gpu_ready.restype = ctypes.c_int
    lib.bfp8_cache_clear.argtypes = []
    lib.bfp8_cache_clear.restype = None
    lib.bfp8_device_bytes.argtypes = []
    lib.bfp8_device_bytes.restype = ctypes.c_size_t
    lib.bfp8_debug_device_limit.argtypes = [ctypes.c_size_t]
    lib.bfp8_debug_device_limit.restype = None
    # device level
    for name in ("bfp8_dev_mant_bytes", "bfp8_dev_exps_bytes"):
        getattr(lib, name).argtypes = [i, i]
        getattr(lib, name).restype = c_size_t
    lib.bfp8_dev_xsplit_bytes.argtypes = [i]
    lib.bfp8_dev_xsplit_bytes.restype = c_size_t
    lib.bfp8_dev_pack.argtypes = [vp, vp, vp, vp, i, i, vp]
    lib.bfp8_dev_unpack.argtypes = [vp, vp, vp, vp, i, i, vp]
    lib.bfp8_dev_quantize.argtypes = [vp, vp, vp, vp, i, vp]
    lib.bfp8_dev_gemv.argtypes = [vp, vp, vp, vp, vp, i, i, vp, vp]
    lib.bfp8_dev_gemv_float.argtypes = [vp, vp, vp, vp, i, i, vp]
    lib.bfp8_dev_gemv_batch.argtypes = [vp, vp, vp, vp, vp, i, i, i, vp]
    lib.bfp8_dev_lm_head_topk.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, vp]
    lib.bfp8_dev_lm_head_topk_noalloc.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, vp]
    lib.bfp8_dev_synth_planes.argtypes = [vp, vp, i, i, c_uint64, i, i, vp]
    lib.bfp8_dev_read_probe.argtypes = [vp, c_size_t, vp, vp]
    lib.bfp8_dev_copy_probe.argtypes = [vp, vp, c_size_t, vp]
    lib.bf16_dev_lm_head.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i, i, i, vp]
    lib.bf16_dev_tiles_bytes.argtypes = [i, i]
    lib.bf16_dev_tiles_bytes.restype = c_size_t
    lib.bf16_dev_tile_table.argtypes = [vp, vp, i, i, vp]
    lib.bf16_dev_lm_head_tiles.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i, i, vp]
    lib.bfp8_dev_sample_from_topk.argtypes = [vp, vp, vp, vp, i, c_float, i, c_float, vp, vp, vp]
    for name in ("bf16_dev_lm_head", "bf16_dev_tile_table", "bf16_dev_lm_head_tiles", "bfp8_dev_sample_from_topk", "bfp8_dev_pack", "bfp8_dev_unpack", "bfp8_dev_quantize", "bfp8_dev_gemv",
                 "bfp8_dev_gemv_float", "bfp8_dev_gemv_batch", "bfp8_dev_lm_head_topk", "bfp8_dev_lm_head_topk_noalloc",
                 "bfp8_dev_synth_planes", "bfp8_dev_read_probe", "bfp8_dev_copy_probe"):
        getattr(lib, name).restype = i
    lib.bfp8_plan_create.argtypes = [POINTER(bfp8_plan_item), i]
    lib.bfp8_plan_create.restype = vp
    for name in ("bfp8_plan_run", "bfp8_plan_run_gemv", "bfp8_plan_quantize"):
        getattr(lib, name).argtypes = [vp, vp]
        getattr(lib, name).restype = i
    lib.bfp8_plan_launch.argtypes = [vp, i, vp]
    lib.bfp8_plan_launch.restype = i
    lib.bfp8_plan_kernel_name.argtypes = [vp, i]
    lib.bfp8_plan_kernel_name.restype = ctypes.c_char_p
    lib.bfp8_plan_destroy.argtypes = [vp]
    lib.bfp8_plan_destroy.restype = None
    lib.bfp8_synth_planes_host.argtypes = [vp, vp, i, i, c_uint64, i, i]
    lib.bfp8_synth_planes_host.restype = None
    lib.bfp8_synth_normal.argtypes = [vp, i, c_uint64]
    lib.bfp8_synth_normal.restype = None
    lib.bfp8_synth_swiglu.argtypes = [vp, i, c_uint64, c_double, c_float]
    lib.bfp8_synth_swiglu.restype = None
    lib.bfp8_stream.argtypes = []
    lib.bfp8_stream.restype = vp
    return lib


_LIB: Optional[ctypes.CDLL] = None


def load(path: Optional[str] = None) -> ctypes.CDLL:
    """Load and bind libqwen_kernels.so (raises if it has not been built)."""
    global _LIB
    if path is None and _LIB is not None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} not built: run qwen35-ax7020-edge-llm_amd/build_lib.py")
    lib = bind(ctypes.CDLL(str(p)))
    if path is None:
        _LIB = lib
    return lib


SAMPLING_PATH = LIB_PATH.with_name("libqwen_sampling.so")
_SAMPLING: Optional[ctypes.CDLL] = None


def load_sampling() -> ctypes.CDLL:
    """libqwen_sampling.so, bound as 04/chat_v3.py:150-159 binds the reference's."""
    global _SAMPLING
    if _SAMPLING is None:
        if not SAMPLING_PATH.exists():
            raise FileNotFoundError(f"{SAMPLING_PATH} not built: run qwen35-ax7020-edge-llm_amd/build_lib.py")
        load()
        lib = ctypes.CDLL(str(SAMPLING_PATH))
        lib.lm_head_topk.restype = ctypes.c_int
        lib.lm_head_topk.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_float)]
        lib.sample_from_topk.restype = ctypes.c_int
        lib.sample_from_topk.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_float), ctypes.c_int,
                                         ctypes.c_float, ctypes.c_int, ctypes.c_float, ctypes.POINTER(ctypes.c_uint)]
        _SAMPLING = lib
    return _SAMPLING


def check(rc: int, what: str = "call") -> None:
    if rc != BFP8_OK:
        msg = load().bfp8_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- synthetic inputs (host) ------------------------------------------------------
def synth_planes(M: int, K: int, seed: int, e_lo: int, e_hi: int):
    """Reference-format planes (int8 [M, K], uint8 [M, K/64]) from the counter hash."""
    lib = load()
    mant = np.empty((M, K), dtype=np.int8)
    exps = np.empty((M, K // 64), dtype=np.uint8)
    lib.bfp8_synth_planes_host(_ptr(mant), _ptr(exps), M, K, seed, e_lo, e_hi)
    return mant, exps


def synth_normal(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().bfp8_synth_normal(_ptr(out), n, seed)
    return out


def synth_swiglu(n: int, seed: int, outlier_frac: float = 0.01, mag: float = 20.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().bfp8_synth_swiglu(_ptr(out), n, seed, outlier_frac, mag)
    return out


# ---- host-pointer API (engine-style) ---------------------------------------------------
class Bfp8Kernels:
    """The engine's view of the library: numpy in, numpy out, synchronous.

    ``gemv_bfp8`` mirrors QwenRealEngine.gemv_bfp8 (04/qwen_real_engine.py:1221-1240)
    on explicit planes instead of a tensor name.
    """

    def __init__(self, path: Optional[str] = None):
        self.lib = load(path)
        self.lib.init_kernels()

    def gemv_bfp8(self, x: np.ndarray, mantissas: np.ndarray, exps: np.ndarray, M: int, K: int,
                  y: Optional[np.ndarray] = None) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if y is None:
            y = np.empty(M, dtype=np.float32)
        self.lib.bfp8_gemv(_ptr(y), _ptr(x), _ptr(mantissas), _ptr(exps), M, K)
        return y

    def gemv_fallback(self, x: np.ndarray, mantissas: np.ndarray, exps: np.ndarray, M: int, K: int,
                      pairwise: bool = True) -> np.ndarray:
        """The engine's numpy fallback (04/qwen_real_engine.py:1230-1238) on the GPU."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(M, dtype=np.float32)
        check(self.lib.bfp8_gemv_fallback(_ptr(y), _ptr(x), _ptr(mantissas), _ptr(exps), M, K, int(pairwise)),
              "bfp8_gemv_fallback")
        return y

    def gemv_batch(self, X: np.ndarray, mantissas: np.ndarray, exps: np.ndarray, M: int, K: int) -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.float32)
        B = X.shape[0]
        Y = np.empty((B, M), dtype=np.float32)
        self.lib.bfp8_gemv_batch(_ptr(Y), _ptr(X), _ptr(mantissas), _ptr(exps), M, K, B)
        return Y

    def lm_head_topk(self, h: np.ndarray, mantissas: np.ndarray, exps: np.ndarray, vocab: int,
                     hidden: int, k: int):
        h = np.ascontiguousarray(h, dtype=np.float32)
        ids = np.full(max(k, 1), -1, dtype=np.int32)
        scores = np.zeros(max(k, 1), dtype=np.float32)
        n = self.lib.bfp8_lm_head_topk(_ptr(h), _ptr(mantissas), _ptr(exps), vocab, hidden, k,
                                       _ptr(ids), _ptr(scores))
        return ids[:n], scores[:n]

    def lm_head_argmax(self, h: np.ndarray, mantissas: np.ndarray, exps: np.ndarray, vocab: int,
                       hidden: int) -> int:
        h = np.ascontiguousarray(h, dtype=np.float32)
        return self.lib.bfp8_lm_head_argmax(_ptr(h), _ptr(mantissas), _ptr(exps), vocab, hidden)


# ---- device-resident API (torch tensors as device memory) ------------------------------
def _torch():
    import torch  # noqa: local import keeps the CPU-only paths torch-free

    return torch


def _stream():
    return _torch().cuda.current_stream().cuda_stream


def _dp(t) -> int:
    return t.data_ptr()


class DeviceMatrix:
    """A BFP8 matrix resident in HBM in the GPU layout."""

    def __init__(self, M: int, K: int, mant_gpu, exps_gpu):
        self.M, self.K, self.mant, self.exps = M, K, mant_gpu, exps_gpu

    @staticmethod
    def empty(M: int, K: int, device="cuda"):
        torch = _torch()
        lib = load()
        mg = torch.empty(max(lib.bfp8_dev_mant_bytes(M, K), 1), dtype=torch.int8, device=device)
        eg = torch.empty(max(lib.bfp8_dev_exps_bytes(M, K), 1), dtype=torch.uint8, device=device)
        return DeviceMatrix(M, K, mg, eg)

    @staticmethod
    def from_soa(mant, exps, device="cuda") -> "DeviceMatrix":
        """Convert reference planes (numpy or device tensors) to the GPU layout."""
        torch = _torch()
        M, K = mant.shape
        ms = torch.as_tensor(np.ascontiguousarray(mant)) if isinstance(mant, np.ndarray) else mant
        es = torch.as_tensor(np.ascontiguousarray(exps)) if isinstance(exps, np.ndarray) else exps
        ms, es = ms.to(device).contiguous(), es.to(device).contiguous()
        dm = DeviceMatrix.empty(M, K, device)
        check(load().bfp8_dev_pack(_dp(dm.mant), _dp(dm.exps), _dp(ms), _dp(es), M, K, _stream()), "pack")
        return dm

    @staticmethod
    def synth(M: int, K: int, seed: int, e_lo: int, e_hi: int, device="cuda") -> "DeviceMatrix":
        """Synthetic planes generated on the GPU (same bytes as synth_planes)."""
        torch = _torch()
        ms = torch.empty(M * K, dtype=torch.int8, device=device)
        es = torch.empty(max(M * (K // 64), 1), dtype=torch.uint8, device=device)
        lib = load()
        check(lib.bfp8_dev_synth_planes(_dp(ms), _dp(es), M, K, seed, e_lo, e_hi, _stream()), "synth")
        dm = DeviceMatrix.empty(M, K, device)
        check(lib.bfp8_dev_pack(_dp(dm.mant), _dp(dm.exps), _dp(ms), _dp(es), M, K, _stream()), "pack")
        del ms, es
        return dm

    def unpack(self):
        torch = _torch()
        ms = torch.empty((self.M, self.K), dtype=torch.int8, device=self.mant.device)
        es = torch.empty((self.M, self.K // 64), dtype=torch.uint8, device=self.mant.device)
        check(load().bfp8_dev_unpack(_dp(ms), _dp(es), _dp(self.mant), _dp(self.exps), self.M, self.K,
                                     _stream()), "unpack")
        return ms, es

    @property
    def weight_bytes(self) -> int:
        """Algorithmic bytes: M*K mantissas + M*K/64 exponents."""
        return self.M * self.K + self.M * (self.K // 64)


def quantize(x):
    """x (device float32 [K]) -> (xq int16 [K], xscale f32 [K/64], xsplit int32 words)."""
    torch = _torch()
    K = x.numel()
    nb = K // 64
    xq = torch.empty(max(nb * 64, 1), dtype=torch.int16, device=x.device)
    xs = torch.empty(max(nb, 1), dtype=torch.float32, device=x.device)
    xsp = torch.empty(max(nb * 32, 1), dtype=torch.int32, device=x.device)
    check(load().bfp8_dev_quantize(_dp(xq), _dp(xs), _dp(xsp), _dp(x), K, _stream()), "quantize")
    return xq[: nb * 64], xs[:nb], xsp


def gemv(mat: DeviceMatrix, xsplit, xscale, y=None, lane_sums: bool = False):
    torch = _torch()
    if y is None:
        y = torch.empty(mat.M, dtype=torch.float32, device=mat.mant.device)
    lanes = None
    if lane_sums:
        lanes = torch.empty((mat.M, mat.K // 64, 4), dtype=torch.int32, device=mat.mant.device)
    check(load().bfp8_dev_gemv(_dp(y), _dp(xsplit), _dp(xscale), _dp(mat.mant), _dp(mat.exps), mat.M, mat.K,
                               _dp(lanes) if lanes is not None else None, _stream()), "gemv")
    return (y, lanes) if lane_sums else y


def gemv_float(mat: DeviceMatrix, x, y=None):
    torch = _torch()
    if y is None:
        y = torch.empty(mat.M, dtype=torch.float32, device=mat.mant.device)
    check(load().bfp8_dev_gemv_float(_dp(y), _dp(x), _dp(mat.mant), _dp(mat.exps), mat.M, mat.K, _stream()),
          "gemv_float")
    return y


def gemv_batch(mat: DeviceMatrix, xsplit, xscale, B: int, Y=None):
    torch = _torch()
    if Y is None:
        Y = torch.empty((B, mat.M), dtype=torch.float32, device=mat.mant.device)
    check(load().bfp8_dev_gemv_batch(_dp(Y), _dp(xsplit), _dp(xscale), _dp(mat.mant), _dp(mat.exps), mat.M,
                                     mat.K, B, _stream()), "gemv_batch")
    return Y


def lm_head_topk(mat: DeviceMatrix, xsplit, xscale, k: int):
    """Fused lm_head on the device -> (ids, scores, count, argmax) device tensors."""
    torch = _torch()
    dev = mat.mant.device
    ids = torch.empty(k, dtype=torch.int32, device=dev)
    scores = torch.empty(k, dtype=torch.float32, device=dev)
    cnt = torch.empty(2, dtype=torch.int32, device=dev)
    check(load().bfp8_dev_lm_head_topk(_dp(ids), _dp(scores), _dp(cnt), _dp(cnt) + 4, _dp(xsplit), _dp(xscale),
                                       _dp(mat.mant), _dp(mat.exps), mat.M, mat.K, k, _stream()), "lm_head_topk")
    return ids, scores, cnt[0:1], cnt[1:2]


class SweepPlan:
    """Grouped GEMV plan: per run the persistent streaming launches (the
    lm_head's tiles, a launch that also quantizes every activation, then every
    other GEMV's, whose workgroup 0 also merges the lm_head's top-k); plans
    without an lm_head quantize in a launch of their own first.

    items: sequence of dicts with keys x (device f32 [K]), mat (DeviceMatrix) and either
    y (device f32 [M]) or topk (int) for the fused lm_head (outputs allocated here).
    """

    def __init__(self, items: Sequence[dict]):
        torch = _torch()
        self.items = list(items)
        arr = (bfp8_plan_item * len(self.items))()
        self.topk_out = None
        for i, it in enumerate(self.items):
            m: DeviceMatrix = it["mat"]
            a = arr[i]
            a.x, a.mant_gpu, a.exps_gpu, a.M, a.K = _dp(it["x"]), _dp(m.mant), _dp(m.exps), m.M, m.K
            a.topk = int(it.get("topk", 0))
            if a.topk > 0:
                dev = m.mant.device
                ids = torch.empty(a.topk, dtype=torch.int32, device=dev)
                sc = torch.empty(a.topk, dtype=torch.float32, device=dev)
                cnt = torch.zeros(2, dtype=torch.int32, device=dev)
                self.topk_out = (ids, sc, cnt)
                a.out_ids, a.out_scores, a.out_count, a.out_argmax = _dp(ids), _dp(sc), _dp(cnt), _dp(cnt) + 4
                a.y = None
            else:
                a.y = _dp(it["y"])
        self._arr = arr
        self.handle = load().bfp8_plan_create(arr, len(self.items))
        if not self.handle:
            raise RuntimeError("bfp8_plan_create: " + load().bfp8_last_error().decode())

    def run(self):
        check(load().bfp8_plan_run(self.handle, _stream()), "plan_run")

    def topk_result(self):
        """(ids, scores, argmax) of the lm_head item after run(), waiting for
        the stream; raises when the run reports its top-k invalid (count -1:
        the single launch's merge gave up waiting for a tile's list)."""
        ids, sc, cnt = self.topk_out
        _torch().cuda.current_stream().synchronize()
        n, am = (int(v) for v in cnt.cpu().tolist())
        if n < 0:
            raise RuntimeError("bfp8 plan: the lm_head top-k of this run is invalid (count -1)")
        return ids[:n], sc[:n], am

    def quantize(self):
        check(load().bfp8_plan_quantize(self.handle, _stream()), "plan_quantize")

    def run_gemv(self):
        check(load().bfp8_plan_run_gemv(self.handle, _stream()), "plan_run_gemv")

    def kernel_name(self, stage):
        """Name of the kernel a stage launches ("" if the stage is empty)."""
        return load().bfp8_plan_kernel_name(self.handle, stage).decode()

    def launch(self, stage):
        """One GEMV stage: 0 lm_head tiles, 1 other tiles + merge, 2 tails."""
        check(load().bfp8_plan_launch(self.handle, stage, _stream()), "plan_launch")

    def close(self):
        if self.handle:
            load().bfp8_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
