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
