"""Regenerate the golden fixtures under tests/golden/.

    make -C oracle all ref          # builds oracle/liboracle.so and oracle/_ref/*.so
    python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):

  tb_gemv_core_legacy.npz
      The two bit-exact legacy-mode cases of the reference's RTL testbench
      (02/tb_gemv_core.v:401-403): stimulus re-derived from its LCG
      (seed = seed*1103515245 + 12345, 32-bit; xq = $signed(seed[15:0]) >>> 1,
      wq = $signed(seed[15:8]), we = e_lo + seed[7:0] % (e_hi-e_lo+1);
      02/tb_gemv_core.v:202-217) and the testbench's golden block dots
      dots[m][b] = sum_{i<64} wq*xq (02/tb_gemv_core.v:150-158), computed here
      by brute force in int64.

  ref_float_path.npz
      Outputs of the reference's own bfp8_gemv built for the host
      (oracle/_ref: the float path, 04/qwen_kernels_opt.c:311-325) on seeded
      inputs, including a K > 4096 case (the path the board build takes there).

  ref_topk.npz
      Outputs of the reference's own lm_head_topk (04/qwen_sampling.c:283-353)
      and lm_head_argmax (04/qwen_kernels_opt.c:401-506, host loop) on crafted
      logit vectors: an embedding table with hidden = 1 whose rows are bf16
      patterns and h = [1.0] makes each score exactly the row's value, so any
      bf16-representable logit vector (ties, NaN, -inf, -0, huge negatives)
      can be fed through the reference's selection code.

  oracle_neon.npz
      Regression vectors of the C restatement's board-build path (y, xq,
      xscale, lane sums) on seeded inputs -- produced by oracle/, so they pin
      only against later changes, not against the reference.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import oracle_lib as ol  # noqa: E402


def lcg_stimulus(K: int, M: int, seed: int, e_lo: int, e_hi: int):
    s = seed & 0xFFFFFFFF
    nb = K // 64

    def step():
        nonlocal s
        s = (s * 1103515245 + 12345) & 0xFFFFFFFF
        return s

    xq = np.empty(K, dtype=np.int16)
    for i in range(K):
        v = step() & 0xFFFF
        v = v - 0x10000 if v & 0x8000 else v
        xq[i] = v >> 1  # arithmetic shift of the signed 16-bit value
    wq = np.empty(M * K, dtype=np.int8)
    for i in range(M * K):
        v = (step() >> 8) & 0xFF
        wq[i] = v - 0x100 if v & 0x80 else v
    we = np.empty(M * nb, dtype=np.uint8)
    for i in range(M * nb):
        we[i] = e_lo + (step() & 0xFF) % (e_hi - e_lo + 1)
    return xq, wq.reshape(M, K), we.reshape(M, nb)


def tb_cases():
    out = {}
    for name, (K, M, seed) in {"k128_m3": (128, 3, 0x12345678), "k1024_m8": (1024, 8, 0x0BADF00D)}.items():
        xq, wq, we = lcg_stimulus(K, M, seed, 118, 130)
        dots = (wq.reshape(M, K // 64, 64).astype(np.int64) * xq.reshape(K // 64, 64).astype(np.int64)).sum(-1)
        out[f"{name}_xq"], out[f"{name}_wq"], out[f"{name}_we"] = xq, wq, we
        out[f"{name}_dots"] = dots.astype(np.int64)
    np.savez_compressed(HERE / "tb_gemv_core_legacy.npz", **out)


def float_path_cases():
    rng = np.random.default_rng(20261201)
    out = {}
    for name, (M, K) in {"m6_k128": (6, 128), "m7_k192": (7, 192), "m64_k1024": (64, 1024),
                         "m5_k4160": (5, 4160), "m3_k100": (3, 100)}.items():
        mant = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        exps = rng.integers(118, 131, size=(M, K // 64), dtype=np.uint8)
        x = rng.standard_normal(K).astype(np.float32)
        y = ol.ref_gemv_float(x, mant, exps)
        out[f"{name}_mant"], out[f"{name}_exps"], out[f"{name}_x"], out[f"{name}_y"] = mant, exps, x, y
    np.savez_compressed(HERE / "ref_float_path.npz", **out)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    return (np.asarray(v, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def topk_cases():
    rng = np.random.default_rng(7)
    cases = {}
    # many ties: 1000 logits from 37 distinct values
    vals = rng.standard_normal(37).astype(np.float32)
    cases["ties1000"] = f32_to_bf16_bits(vals[rng.integers(0, 37, 1000)])
    # odd vocabulary and specials: NaN, -inf, +-0, the largest bf16 magnitudes, values <= -1e30
    sp = f32_to_bf16_bits(rng.standard_normal(1001).astype(np.float32))
    special = {3: 0x7FC0, 10: 0xFF80, 11: 0x8000, 12: 0x0000, 40: 0x7F7F, 41: 0xFF7F, 500: 0xF2F0, 999: 0x7F80}
    for i, b in special.items():
        sp[i] = b
    cases["special1001"] = sp
    # the self-test's big shape: 65536 logits
    cases["vocab65536"] = f32_to_bf16_bits((rng.standard_normal(65536) * 3).astype(np.float32))
    # no candidate at all
    cases["allnan64"] = np.full(64, 0x7FC0, dtype=np.uint16)
    # only huge negatives (<= -1e30 but > -FLT_MAX): top-k keeps them, argmax returns 0
    cases["hugeneg128"] = f32_to_bf16_bits(-np.float32(1e31) * (1 + rng.random(128).astype(np.float32)))
    # equal maxima in both halves: the lower id must win
    eq = f32_to_bf16_bits(rng.standard_normal(256).astype(np.float32) * 0.1)
    eq[[30, 200]] = f32_to_bf16_bits(np.float32([5.0, 5.0]))
    cases["eqmax256"] = eq
    out = {}
    for name, bits in cases.items():
        out[f"{name}_bits"] = bits
        out[f"{name}_argmax"] = np.int32(ol.ref_argmax(bits))
        for k in (1, 40, 64):
            ids, sc = ol.ref_topk(bits, k)
            out[f"{name}_k{k}_ids"], out[f"{name}_k{k}_scores"] = ids, sc
    np.savez_compressed(HERE / "ref_topk.npz", **out)


def oracle_neon_cases():
    rng = np.random.default_rng(424242)
    out = {}
    for name, (M, K) in {"m6_k128": (6, 128), "m7_k256": (7, 256), "m64_k1024": (64, 1024)}.items():
        mant = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        exps = rng.integers(122, 131, size=(M, K // 64), dtype=np.uint8)
        exps[0, 0] = 5  # a subnormal EXP_SCALE block
        x = rng.standard_normal(K).astype(np.float32)
        x[::37] *= 20.0
        y, xq, xs, lanes = ol.gemv_neon(x, mant, exps)
        out.update({f"{name}_mant": mant, f"{name}_exps": exps, f"{name}_x": x, f"{name}_y": y,
                    f"{name}_xq": xq, f"{name}_xscale": xs, f"{name}_lanes": lanes})
    np.savez_compressed(HERE / "oracle_neon.npz", **out)


if __name__ == "__main__":
    if not ol.ref_available():
        sys.exit("oracle/_ref not built: run `make -C oracle ref` (needs the reference sources)")
    tb_cases()
    float_path_cases()
    topk_cases()
    oracle_neon_cases()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
