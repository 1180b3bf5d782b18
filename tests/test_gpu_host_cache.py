"""The host-pointer ABI's weight cache: bfp8_gemv keeps a device copy of
weights that live in read-only memory (the engine's PROT_READ mmap of its
image, 04/qwen_real_engine.py:745-751), keyed by address and shape.  When
the memory at that address is replaced (a model reload mapped at the same
address) the copy is converted again from the new contents, and writable
buffers are re-read on every call."""
import ctypes
import mmap
import os
import sys

import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu
F32 = np.float32


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def _libc():
    libc = ctypes.CDLL(None, use_errno=True)
    libc.mmap.restype = ctypes.c_void_p
    libc.mmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_long]
    libc.munmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    return libc


def test_replaced_mapping_at_the_same_address_is_converted_again(gpu, tmp_path):
    qk = gpu
    M, K = 640, 1024
    images = []
    for i in range(2):
        mant, exps = qk.synth_planes(M, K, 300 + i, 124, 130)
        p = tmp_path / f"image{i}.bin"
        with open(p, "wb") as f:
            f.write(mant.tobytes())
            f.write(exps.tobytes())
        images.append((p, mant, exps))
    size = M * K + M * (K // 64)
    x = qk.synth_normal(K, 99)
    libc = _libc()
    MAP_PRIVATE, MAP_FIXED = 0x02, 0x10
    fds = [os.open(str(p), os.O_RDONLY) for p, _, _ in images]
    addr = libc.mmap(None, size, mmap.PROT_READ, MAP_PRIVATE, fds[0], 0)
    assert addr not in (None, ctypes.c_void_p(-1).value)
    lib = qk.load()
    y = np.empty(M, dtype=F32)
    try:
        for rnd, img in enumerate((0, 0, 1, 1, 0)):
            if rnd > 0 and img != (0, 0, 1, 1, 0)[rnd - 1]:
                got = libc.mmap(addr, size, mmap.PROT_READ, MAP_PRIVATE | MAP_FIXED, fds[img], 0)
                assert got == addr
            say("cached mapping round", rnd, "image", img)
            lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, addr, addr + M * K, M, K)
            y_ref = ol.gemv_neon(x, images[img][1], images[img][2])[0]
            assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), (rnd, img)
    finally:
        libc.munmap(addr, size)
        for fd in fds:
            os.close(fd)
        lib.bfp8_cache_clear()


def test_a_full_device_uploads_per_call(gpu, tmp_path):
    """A device that cannot hold another cached copy (rehearsed with
    bfp8_debug_device_limit at what the library holds) is recoverable:
    bfp8_gemv on read-only weights, which it would cache, converts them into
    its per-call buffers instead -- the oracle's result, nothing more held, no
    abort -- and caches them once the device has room again; an entry point
    with an error channel (bfp8_lm_head_topk) returns 0 with the reason while
    the device is full and the oracle's top-k afterwards."""
    qk = gpu
    lib = qk.load()
    M, K = 640, 1024
    mant, exps = qk.synth_planes(M, K, 4242, 124, 130)
    path = tmp_path / "image.bin"
    path.write_bytes(mant.tobytes() + exps.tobytes())
    size = M * K + M * (K // 64)
    x = qk.synth_normal(K, 4243)
    y_ref = ol.gemv_neon(x, mant, exps)[0]
    libc = _libc()
    fd = os.open(str(path), os.O_RDONLY)
    addr = libc.mmap(None, size, mmap.PROT_READ, 0x02, fd, 0)
    assert addr not in (None, ctypes.c_void_p(-1).value)
    y = np.empty(M, dtype=F32)
    lib.bfp8_cache_clear()
    try:
        say("full device: per-call buffers of the shape first (writable planes)")
        lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, mant.ctypes.data, exps.ctypes.data, M, K)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        held = lib.bfp8_device_bytes()
        lib.bfp8_debug_device_limit(held)
        try:
            say("full device: read-only planes, not cached")
            y.fill(np.nan)
            lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, addr, addr + M * K, M, K)
            assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
            assert lib.bfp8_device_bytes() == held
            say("full device: lm_head beyond the per-call buffers")
            V, H, k = 16384, 1024, 40
            lm, le = qk.synth_planes(V, H, 4244, 122, 128)
            h = qk.synth_normal(H, 4245)
            ids = np.full(k, -1, dtype=np.int32)
            sc = np.zeros(k, dtype=F32)
            n = lib.bfp8_lm_head_topk(h.ctypes.data, lm.ctypes.data, le.ctypes.data, V, H, k, ids.ctypes.data,
                                      sc.ctypes.data)
            assert n == 0 and b"device memory" in lib.bfp8_last_error()
        finally:
            lib.bfp8_debug_device_limit(0)
        say("room again: cached, and the lm_head runs")
        y.fill(np.nan)
        lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, addr, addr + M * K, M, K)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        assert lib.bfp8_device_bytes() > held
        n = lib.bfp8_lm_head_topk(h.ctypes.data, lm.ctypes.data, le.ctypes.data, V, H, k, ids.ctypes.data,
                                  sc.ctypes.data)
        ids_ref, sc_ref = ol.topk(ol.gemv_neon(h, lm, le)[0], k)
        assert n == k and np.array_equal(ids, ids_ref) and np.array_equal(sc.view(np.uint32), sc_ref.view(np.uint32))
    finally:
        libc.munmap(addr, size)
        os.close(fd)
        lib.bfp8_cache_clear()
