"""GPU checks of the weight-image loader: a synthetic image in the exporter's
format (tensors at 64-byte aligned offsets, BFP8 = mantissa plane then
exponent plane padded to 8 with 127, raw fp32 / bf16 arrays) is written to a
file, mapped read-only as the engine maps it, preloaded, and then

  * every BFP8 tensor's device planes unpack to the image's planes, byte for byte;
  * bfp8_gemv on the engine's slicing of the image (mant = raw[:M*K],
    exps = raw[M*K:]) equals the oracle bit for bit;
  * the PL core's per-row stream (exponents then mantissas per row) packs to
    the same device planes as the SoA planes."""
import ctypes
import json
import mmap
import sys

import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


SHAPES = [("layers.0.linear_attn.in_proj_qkv.weight", 6144, 1024), ("layers.0.mlp.down_proj.weight", 1024, 3584),
          ("layers.3.self_attn.k_proj.weight", 512, 1024), ("odd.weight", 3, 128), ("wide.weight", 64, 4096)]


@pytest.fixture(scope="module")
def image(tmp_path_factory):
    rng = np.random.default_rng(31)
    d = tmp_path_factory.mktemp("weights")
    parts, tensors, off = [], {}, 0

    def put(name, data, meta):
        nonlocal off
        pad = (-off) % 64
        parts.append(b"\0" * pad)
        off += pad
        meta.update(file_offset=off, byte_size=len(data))
        tensors[name] = meta
        parts.append(data)
        off += len(data)

    put("embed_tokens.weight", rng.integers(0, 2 ** 16, 300 * 64, dtype=np.uint16).tobytes(),
        {"dtype": "bfloat16", "shape": [300, 64], "type": "raw_bf16"})
    put("norm.weight", rng.standard_normal(1024).astype(np.float32).tobytes(),
        {"dtype": "float32", "shape": [1024], "type": "raw_fp32"})
    planes = {}
    for name, M, K in SHAPES:
        m = rng.integers(-128, 128, M * K, dtype=np.int8)
        e = rng.integers(118, 131, M * K // 64, dtype=np.uint8)
        pad = (-e.size) % 8
        put(name, m.tobytes() + e.tobytes() + bytes([127] * pad),
            {"dtype": "bfp8_soa", "shape": [M, K], "type": "block64_bfp8", "mantissa_bytes": M * K,
             "exponent_bytes": e.size + pad})
        planes[name] = (m, e, M, K)
    parts.append(b"\0" * ((-off) % 64))
    blob = b"".join(parts)
    (d / "w.bin").write_bytes(blob)
    (d / "w.json").write_text(json.dumps({"tensors": tensors, "total_binary_bytes": len(blob)}))
    f = open(d / "w.bin", "rb")
    mm = mmap.mmap(f.fileno(), 0, prot=mmap.PROT_READ)
    raw = np.frombuffer(mm, dtype=np.uint8)
    yield raw, tensors, planes, d / "w.json"
    # the mapping goes with its last numpy view (closing it here would fail
    # while pytest still holds the fixture value)
    f.close()


def test_preload_then_engine_slicing(gpu, image):
    import torch

    qk = gpu
    lib = qk.load()
    raw, tensors, planes, manifest = image
    lib.bfp8_cache_clear()
    say("preload")
    n = lib.qwen_weights_preload(raw.ctypes.data, raw.size, str(manifest).encode())
    assert n == len(SHAPES), lib.bfp8_last_error()
    for name, M, K in SHAPES:
        m, e, _, _ = planes[name]
        mg, eg = ctypes.c_void_p(), ctypes.c_void_p()
        Mo, Ko = ctypes.c_int(), ctypes.c_int()
        assert lib.qwen_weights_find(name.encode(), ctypes.byref(mg), ctypes.byref(eg), ctypes.byref(Mo),
                                     ctypes.byref(Ko)) == 0
        assert (Mo.value, Ko.value) == (M, K)
        ms = torch.empty(M * K, dtype=torch.int8, device="cuda")
        es = torch.empty(M * K // 64, dtype=torch.uint8, device="cuda")
        qk.check(lib.bfp8_dev_unpack(ms.data_ptr(), es.data_ptr(), mg.value, eg.value, M, K, None))
        torch.cuda.synchronize()
        assert np.array_equal(ms.cpu().numpy(), m) and np.array_equal(es.cpu().numpy(), e), name
        # the engine's slicing of the mapped image, 04/qwen_real_engine.py:834-846
        t = tensors[name]
        sl = raw[t["file_offset"]: t["file_offset"] + t["byte_size"]]
        mant, exps = sl[: M * K].view(np.int8), sl[M * K: M * K + M * K // 64]
        x = np.random.default_rng(M + K).standard_normal(K).astype(np.float32)
        y = np.empty(M, dtype=np.float32)
        say("gemv", name)
        lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, mant.ctypes.data, exps.ctypes.data, M, K)
        want = ol.gemv_neon(x, m.reshape(M, K), e.reshape(M, K // 64))[0]
        assert np.array_equal(y.view(np.uint32), np.asarray(want, dtype=np.float32).view(np.uint32)), name
    assert lib.qwen_weights_find(b"norm.weight", None, None, None, None) < 0  # raw tensors are not GEMV planes
    lib.bfp8_cache_clear()
    assert lib.qwen_weights_find(SHAPES[0][0].encode(), None, None, None, None) < 0


def test_preload_rejects_a_truncated_image(gpu, image):
    lib = gpu.load()
    raw, tensors, planes, manifest = image
    assert lib.qwen_weights_preload(raw.ctypes.data, raw.size - 64, str(manifest).encode()) < 0
    assert b"outside" in lib.bfp8_last_error()


def test_row_stream_packs_like_the_soa_planes(gpu):
    import torch

    qk = gpu
    lib = qk.load()
    rng = np.random.default_rng(32)
    for M, K in ((3584, 1024), (130, 192), (1, 64)):
        nb = K // 64
        m = rng.integers(-128, 128, (M, K), dtype=np.int8)
        e = rng.integers(0, 256, (M, nb), dtype=np.uint8)
        stream = np.concatenate([e, m.view(np.uint8)], axis=1)  # per row: exponents, then mantissas
        say("pack_rows", M, K)
        sd = torch.from_numpy(np.ascontiguousarray(stream).reshape(-1)).cuda()
        md = torch.from_numpy(m.reshape(-1)).cuda()
        ed = torch.from_numpy(e.reshape(-1)).cuda()
        gm1 = torch.empty(lib.bfp8_dev_mant_bytes(M, K), dtype=torch.uint8, device="cuda")
        ge1 = torch.empty(lib.bfp8_dev_exps_bytes(M, K), dtype=torch.uint8, device="cuda")
        gm2, ge2 = torch.empty_like(gm1), torch.empty_like(ge1)
        qk.check(lib.bfp8_dev_pack_rows(gm1.data_ptr(), ge1.data_ptr(), sd.data_ptr(), M, K, None))
        qk.check(lib.bfp8_dev_pack(gm2.data_ptr(), ge2.data_ptr(), md.data_ptr(), ed.data_ptr(), M, K, None))
        torch.cuda.synchronize()
        assert torch.equal(gm1, gm2) and torch.equal(ge1, ge2), (M, K)
