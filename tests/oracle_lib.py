"""ctypes access to the checkers: oracle/liboracle.so (the C restatement) and
oracle/_ref/*.so (the reference's own C sources built for the host).

Test infrastructure only.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
# ORACLE_LIB_UNDER_TEST: another build of the same sources (the sanitizer run)
ORACLE = Path(os.environ.get("ORACLE_LIB_UNDER_TEST") or ROOT / "oracle" / "liboracle.so")
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
        lib.orc_gemv_fallback.argtypes = [vp, vp, vp, vp, i, i, i]
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


def gemv_fallback(x, mant, exps, pairwise=True):
    """The engine's numpy fallback (04/qwen_real_engine.py:1230-1238) in numpy's
    summation order: pairwise (numpy >= 1.9) or sequential (numpy 1.8.2)."""
    mant = np.ascontiguousarray(mant, dtype=np.int8)
    M, K = mant.shape
    y = np.zeros(M, dtype=np.float32)
    oracle().orc_gemv_fallback(_p(y), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(mant),
                               _p(np.ascontiguousarray(exps, dtype=np.uint8)), M, K, int(bool(pairwise)))
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


# ---- decode runtime kernels ---------------------------------------------------------
_RT_BOUND = False


def _rt():
    global _RT_BOUND
    lib = oracle()
    if not _RT_BOUND:
        vp, i, f = c_void_p, c_int, c_float
        lib.orc_exp_neon.argtypes = [f]
        lib.orc_exp_neon.restype = f
        lib.orc_swiglu.argtypes = [vp, vp, vp, i]
        lib.orc_add_residual.argtypes = [vp, vp, i]
        lib.orc_rmsnorm.argtypes = [vp, vp, vp, i, f]
        lib.orc_conv1d_silu.argtypes = [vp, vp, vp, vp, i]
        lib.orc_qk_l2norm.argtypes = [vp, vp, i, i]
        lib.orc_gdn_gates.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i]
        lib.orc_gdn_step.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i]
        lib.orc_rmsnorm_gated.argtypes = [vp, vp, vp, vp, i, i, f]
        lib.orc_forward_linear_layer.argtypes = [vp, vp]
        lib.orc_forward_mlp.argtypes = [vp, vp]
        lib.orc_forward_token.argtypes = [i, vp, vp, vp, vp, vp, vp, vp, vp, i]
        lib.orc_forward_token.restype = i
        lib.orc_set_cr_libm.argtypes = [i]
        _RT_BOUND = True
    return lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def exp_neon(x):
    return _rt().orc_exp_neon(float(x))


def swiglu(gate, up):
    g, u = _f32(gate), _f32(up)
    y = np.zeros_like(g)
    _rt().orc_swiglu(_p(y), _p(g), _p(u), g.size)
    return y


def add_residual(x, res):
    x, r = _f32(x).copy(), _f32(res)
    _rt().orc_add_residual(_p(x), _p(r), x.size)
    return x


def rmsnorm(x, w, eps=1e-6):
    x, w = _f32(x), _f32(w)
    y = np.zeros_like(x)
    _rt().orc_rmsnorm(_p(y), _p(x), _p(w), x.size, eps)
    return y


def conv1d_silu(x, state, weight):
    """Returns (y, new state); state [3][C], weight [C][4]."""
    x, st, w = _f32(x), _f32(state).copy(), _f32(weight)
    y = np.zeros_like(x)
    _rt().orc_conv1d_silu(_p(y), _p(x), _p(st), _p(w), x.size)
    return y, st


def qk_l2norm(q, k, H, D):
    q, k = _f32(q).copy(), _f32(k).copy()
    _rt().orc_qk_l2norm(_p(q), _p(k), H, D)
    return q, k


def gdn_gates(x, wa, wb, nea, dt):
    H, K = wa.shape
    a = np.zeros(H, dtype=np.float32)
    b = np.zeros(H, dtype=np.float32)
    _rt().orc_gdn_gates(_p(a), _p(b), _p(_f32(x)), _p(_f32(wa)), _p(_f32(wb)), _p(_f32(nea)), _p(_f32(dt)), H, K)
    return a, b


def gdn_step(S, q, k, v, alpha, beta, H, D):
    """S: logical state [H][D][D] (row = input index i, column = output j).
    Returns (out, new S)."""
    S = _f32(S).copy()
    out = np.zeros(H * D, dtype=np.float32)
    _rt().orc_gdn_step(_p(out), _p(S), _p(_f32(q)), _p(_f32(k)), _p(_f32(v)), _p(_f32(alpha)), _p(_f32(beta)), H, D)
    return out, S


def rmsnorm_gated(x, z, w, H, D, eps=1e-6):
    x, z, w = _f32(x), _f32(z), _f32(w)
    y = np.zeros_like(x)
    _rt().orc_rmsnorm_gated(_p(y), _p(x), _p(z), _p(w), H, D, eps)
    return y


def gdn_state_to_blocked(S, H, D):
    """The reference's internal gdn state layout: block (jg, ig) of 16 floats,
    state[h][((jg*ng + ig)*4 + l)*4 + t] = S[h][4ig+t][4jg+l]."""
    S = np.asarray(S, dtype=np.float32).reshape(H, D // 4, 4, D // 4, 4)  # h, ig, t, jg, l
    return np.ascontiguousarray(S.transpose(0, 3, 1, 4, 2)).reshape(-1)


def gdn_state_from_blocked(B, H, D):
    B = np.asarray(B, dtype=np.float32).reshape(H, D // 4, D // 4, 4, 4)  # h, jg, ig, l, t
    return np.ascontiguousarray(B.transpose(0, 2, 4, 1, 3)).reshape(H, D, D)


def ref_runtime():
    """The reference host build's runtime kernels (scalar paths)."""
    lib = ref_kernels()
    vp, i, f = c_void_p, c_int, c_float
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
    return lib


class LinearPlan(ctypes.Structure):
    """Field-for-field mirror of LinearLayerPlan (04/qwen_kernels_opt.c:866-901)."""
    _fields_ = [(n, t) for n, t in [
        ("in_ln_w", c_void_p), ("mant_qkv", c_void_p), ("exp_qkv", c_void_p), ("M_qkv", c_int), ("K_qkv", c_int),
        ("conv_w", c_void_p), ("conv_s", c_void_p), ("wa", c_void_p), ("wb", c_void_p), ("nea", c_void_p),
        ("dt", c_void_p), ("state", c_void_p), ("mant_z", c_void_p), ("exp_z", c_void_p), ("M_z", c_int),
        ("K_z", c_int), ("norm_w", c_void_p), ("mant_o", c_void_p), ("exp_o", c_void_p), ("M_o", c_int),
        ("K_o", c_int), ("post_ln_w", c_void_p), ("mant_gate", c_void_p), ("exp_gate", c_void_p),
        ("M_gate", c_int), ("K_gate", c_int), ("mant_up", c_void_p), ("exp_up", c_void_p), ("M_up", c_int),
        ("K_up", c_int), ("mant_down", c_void_p), ("exp_down", c_void_p), ("M_down", c_int), ("K_down", c_int)]]


class MlpPlan(ctypes.Structure):
    """Field-for-field mirror of MlpPlan (04/qwen_kernels_opt.c:903-917)."""
    _fields_ = [("post_ln_w", c_void_p), ("mant_gate", c_void_p), ("exp_gate", c_void_p), ("M_gate", c_int),
                ("K_gate", c_int), ("mant_up", c_void_p), ("exp_up", c_void_p), ("M_up", c_int), ("K_up", c_int),
                ("mant_down", c_void_p), ("exp_down", c_void_p), ("M_down", c_int), ("K_down", c_int)]


class cr_libm:
    """Context: the oracle's expf / log1pf become exp / log1p in double rounded
    once to float (the definition the GPU implements)."""

    def __enter__(self):
        _rt().orc_set_cr_libm(1)
        return self

    def __exit__(self, *exc):
        _rt().orc_set_cr_libm(0)


def forward_mlp(plan, h):
    """orc_forward_mlp on a copy of h; plan is a ctypes MlpPlan (states are
    the host buffers the plan points at)."""
    h = _f32(h).copy()
    _rt().orc_forward_mlp(ctypes.addressof(plan), _p(h))
    return h


def forward_linear_layer(plan, h):
    """orc_forward_linear_layer on a copy of h; updates the plan's conv and
    recurrent state buffers in place (blocked state layout converted)."""
    h = _f32(h).copy()
    _rt().orc_forward_linear_layer(ctypes.addressof(plan), _p(h))
    return h


def forward_token(token_id, lin_plans, mlp_plans, is_full, final_norm_w, embed, vocab=65536):
    h = np.zeros(1024, dtype=np.float32)
    isf = np.ascontiguousarray(is_full, dtype=np.int32)
    best = _rt().orc_forward_token(int(token_id), _p(h), ctypes.addressof(lin_plans), ctypes.addressof(mlp_plans),
                                   _p(isf), _p(_f32(final_norm_w)), _p(embed), None, None, vocab)
    return best, h
