"""ctypes access to the checkers: oracle/liboracle.so (the C restatement) and
oracle/_ref/*.so (the reference's own C sources built for the host).

Test infrastructure only.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE = ROOT / "oracle" / "liboracle.so"
REF_KERNELS = ROOT / "oracle" / "_ref" / "libref_qwen_kernels.so"
REF_SAMPLING = ROOT / "oracle" / "_ref" / "libref_qwen_sampling.so"

_orc = None


def oracle() -> ctypes.CDLL:
    global _orc
    if _orc is None:
        lib = ctypes.CDLL(str(ORACLE))
        vp, i = c_void_p, c_int
        lib.orc_exp_scale.argtypes = [i]
        lib.orc_exp_scale.restype = c_float
        lib.orc_neon_mul.argtypes = [c_float, c_float]
        lib.orc_neon_mul.restype = c_float
        lib.orc_neon_add.argtypes = [c_float, c_float]
        lib.orc_neon_add.restype = c_float
        lib.orc_quant_x.argtypes = [vp, i, vp, vp]
        lib.orc_lane_sums.argtypes = [vp, vp, i, i, vp]
        lib.orc_gemv_float.argtypes = [vp, vp, vp, vp, i, i]
        lib.orc_gemv_neon.argtypes = [vp, vp, vp, vp, i, i, vp, vp, vp]
        lib.orc_argmax.argtypes = [vp, i]
        lib.orc_argmax.restype = i
        lib.orc_topk.argtypes = [vp, i, i, vp, vp]
        lib.orc_topk.restype = i
        lib.orc_gemv_f64.argtypes = [vp, vp, vp, vp, vp, i, i]
        lib.orc_bf16_dot.argtypes = [vp, vp, i, i]
        lib.orc_bf16_dot.restype = c_float
        lib.orc_bf16_logits.argtypes = [vp, vp, i, i, i, vp]
        lib.orc_sample_from_topk.argtypes = [vp, vp, i, c_float, i, c_float, vp]
        lib.orc_sample_from_topk.restype = i
        _orc = lib
    return _orc


def _p(a):
    return None if a is None else a.ctypes.data


def quant_x(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.size
    nb = K // 64
    xq = np.zeros(max(nb * 64, 1), dtype=np.int16)
    xs = np.zeros(max(nb, 1), dtype=np.float32)
    oracle().orc_quant_x(_p(x), K, _p(xq), _p(xs))
    return xq[: nb * 64], xs[:nb]


def lane_sums(mant: np.ndarray, xq: np.ndarray):
    M, K = mant.shape
    lanes = np.zeros((M, K // 64, 4), dtype=np.int32)
    oracle().orc_lane_sums(_p(np.ascontiguousarray(mant)), _p(np.ascontiguousarray(xq, dtype=np.int16)), M, K,
                           _p(lanes))
    return lanes


def gemv_neon(x, mant, exps):
    """Board-build bfp8_gemv: returns (y, xq, xscale, lanes)."""
    mant = np.ascontiguousarray(mant)
    exps = np.ascontiguousarray(exps)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = mant.shape
    nb = K // 64
    y = np.zeros(M, dtype=np.float32)
    xq = np.zeros(max(nb * 64, 1), dtype=np.int16)
    xs = np.zeros(max(nb, 1), dtype=np.float32)
    lanes = np.zeros((M, max(nb, 1), 4), dtype=np.int32)
    small = K <= 4096
    oracle().orc_gemv_neon(_p(y), _p(x), _p(mant), _p(exps), M, K, _p(xq) if small else None,
                           _p(xs) if small else None, _p(lanes) if small else None)
    return y, xq[: nb * 64], xs[:nb], lanes[:, :nb]


def gemv_float(x, mant, exps):
    mant = np.ascontiguousarray(mant)
    M, K = mant.shape
    y = np.zeros(M, dtype=np.float32)
    oracle().orc_gemv_float(_p(y), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(mant),
                            _p(np.ascontiguousarray(exps)), M, K)
    return y


def gemv_f64(mant, exps, xq, xscale):
    M, K = mant.shape
    y = np.zeros(M, dtype=np.float64)
    oracle().orc_gemv_f64(_p(y), _p(np.ascontiguousarray(mant)), _p(np.ascontiguousarray(exps)),
                          _p(np.ascontiguousarray(xq, dtype=np.int16)),
                          _p(np.ascontiguousarray(xscale, dtype=np.float32)), M, K)
    return y


def argmax(logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return oracle().orc_argmax(_p(logits), logits.size)


def topk(logits, k):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(max(k, 1), dtype=np.int32)
    sc = np.zeros(max(k, 1), dtype=np.float32)
    n = oracle().orc_topk(_p(logits), logits.size, k, _p(ids), _p(sc))
    return ids[:n], sc[:n]


def neon_mul(a, b):
    return oracle().orc_neon_mul(a, b)


def neon_add(a, b):
    return oracle().orc_neon_add(a, b)


# ---- the reference's own host build (oracle/_ref) ---------------------------------
def ref_available() -> bool:
    return REF_KERNELS.exists() and REF_SAMPLING.exists()


_refk = _refs = None


def ref_kernels() -> ctypes.CDLL:
    global _refk
    if _refk is None:
        lib = ctypes.CDLL(str(REF_KERNELS))
        lib.init_kernels.argtypes = []
        lib.bfp8_gemv.argtypes = [c_void_p] * 4 + [c_int] * 2
        lib.bfp8_gemv.restype = None
        lib.lm_head_argmax.argtypes = [c_void_p, c_void_p, c_int, c_int]
        lib.lm_head_argmax.restype = c_int
        lib.init_kernels()
        _refk = lib
    return _refk


def ref_sampling() -> ctypes.CDLL:
    global _refs
    if _refs is None:
        lib = ctypes.CDLL(str(REF_SAMPLING))
        lib.lm_head_topk.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]
        lib.lm_head_topk.restype = c_int
        lib.sample_from_topk.argtypes = [c_void_p, c_void_p, c_int, c_float, c_int, c_float, c_void_p]
        lib.sample_from_topk.restype = c_int
        _refs = lib
    return _refs


def ref_gemv_float(x, mant, exps):
    """The reference's host bfp8_gemv (float path, 04/qwen_kernels_opt.c:311-325)."""
    mant = np.ascontiguousarray(mant)
    M, K = mant.shape
    y = np.zeros(M, dtype=np.float32)
    ref_kernels().bfp8_gemv(_p(y), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(mant),
                            _p(np.ascontiguousarray(exps)), M, K)
    return y


def bf16_column(logits_bf16_bits: np.ndarray):
    """An embedding table with hidden = 1 whose row t is the bf16 pattern
    logits_bf16_bits[t]; with h = [1.0] the reference's dot product is
    0 + 1.0*value, i.e. the logit itself."""
    return np.ascontiguousarray(logits_bf16_bits, dtype=np.uint16).reshape(-1, 1)


def ref_topk(logits_bf16_bits, k):
    table = bf16_column(logits_bf16_bits)
    h = np.ones(1, dtype=np.float32)
    ids = np.zeros(max(k, 1), dtype=np.int32)
    sc = np.zeros(max(k, 1), dtype=np.float32)
    n = ref_sampling().lm_head_topk(_p(h), _p(table), table.shape[0], 1, k, _p(ids), _p(sc))
    return ids[:n], sc[:n]


def ref_argmax(logits_bf16_bits):
    table = bf16_column(logits_bf16_bits)
    h = np.ones(1, dtype=np.float32)
    return ref_kernels().lm_head_argmax(_p(h), _p(table), table.shape[0], 1)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


# ---- bf16 tied-embedding lm_head and the sampler ------------------------------------
def bf16_dot(h, row, tail):
    h = np.ascontiguousarray(h, dtype=np.float32)
    row = np.ascontiguousarray(row, dtype=np.uint16)
    return oracle().orc_bf16_dot(_p(h), _p(row), row.size, int(tail))


def bf16_logits(h, table, tail):
    """Board-build scores of every row (tail: 0 = lm_head_argmax's rule,
    1 = lm_head_topk's)."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    table = np.ascontiguousarray(table, dtype=np.uint16)
    V, H = table.shape
    out = np.zeros(V, dtype=np.float32)
    oracle().orc_bf16_logits(_p(h), _p(table), V, H, int(tail), _p(out))
    return out


def sample_from_topk(ids, scores, temperature, top_k, top_p, state):
    """Returns (chosen id, new state)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    st = np.array([state], dtype=np.uint32)
    r = oracle().orc_sample_from_topk(_p(ids), _p(scores), ids.size, temperature, top_k, top_p, _p(st))
    return r, int(st[0])


def ref_sample_from_topk(ids, scores, temperature, top_k, top_p, state):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    st = np.array([state], dtype=np.uint32)
    r = ref_sampling().sample_from_topk(_p(ids), _p(scores), ids.size, temperature, top_k, top_p, _p(st))
    return r, int(st[0])


def f32_to_bf16_bits(x):
    """Round-to-nearest-even bf16 bits of float32 values (test data only)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)
