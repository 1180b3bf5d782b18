"""The no-alloc lm_head entry point (bfp8_dev_lm_head_topk_noalloc) against
bfp8_dev_lm_head_topk on the same inputs, through the C ABI: two calls in a
row, the second with a smaller input (and another path: odd vocabulary,
k above 64), each identical to the allocating entry point and to the
oracle; sizes above the fixed scratch are rejected with an error.  Named to be
collected last: it must pass after every other GPU test and alone."""
import sys

import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu
F32 = np.float32


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def run_entry(qk, fn, dm, xsp, xs, k):
    import torch

    kk = min(k, dm.M)
    ids = torch.full((kk,), -7, dtype=torch.int32, device="cuda")
    sc = torch.zeros(kk, dtype=torch.float32, device="cuda")
    cnt = torch.full((2,), -7, dtype=torch.int32, device="cuda")
    rc = fn(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), cnt.data_ptr() + 4, xsp.data_ptr(), xs.data_ptr(),
            dm.mant.data_ptr(), dm.exps.data_ptr(), dm.M, dm.K, k, torch.cuda.current_stream().cuda_stream)
    qk.check(rc, fn.__name__)
    torch.cuda.synchronize()
    n = int(cnt[0].item())
    return ids.cpu().numpy()[:n], sc.cpu().numpy()[:n].view(np.uint32), int(cnt[1].item())


def test_no_alloc_lm_head_matches_the_allocating_entry(gpu):
    qk = gpu
    import torch

    lib = qk.load()
    cases = [(65536, 1024, 40, 11), (4099, 512, 100, 12)]  # the second call smaller, general path
    for V, H, k, seed in cases:
        r = np.random.default_rng(seed)
        mant = r.integers(-128, 128, size=(V, H), dtype=np.int8)
        exps = r.integers(120, 131, size=(V, H // 64), dtype=np.uint8)
        x = r.standard_normal(H).astype(F32)
        dm = qk.DeviceMatrix.from_soa(mant, exps)
        _, xs, xsp = qk.quantize(torch.from_numpy(x).cuda())
        say("no-alloc lm_head", V, H, k)
        got = run_entry(qk, lib.bfp8_dev_lm_head_topk_noalloc, dm, xsp, xs, k)
        want = run_entry(qk, lib.bfp8_dev_lm_head_topk, dm, xsp, xs, k)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]) and got[2] == want[2]
        y = ol.gemv_neon(x, mant, exps)[0]
        ids_ref, sc_ref = ol.topk(y, k)
        assert np.array_equal(got[0], ids_ref) and np.array_equal(got[1], sc_ref.view(np.uint32))
        assert got[2] == ol.argmax(y)
    # beyond the scratch: rejected before any launch
    big = qk.DeviceMatrix.synth(262146, 64, 3, 122, 128)
    _, xs, xsp = qk.quantize(torch.zeros(64, device="cuda"))
    ids = torch.empty(4, dtype=torch.int32, device="cuda")
    rc = lib.bfp8_dev_lm_head_topk_noalloc(ids.data_ptr(), ids.data_ptr(), ids.data_ptr(), ids.data_ptr(),
                                           xsp.data_ptr(), xs.data_ptr(), big.mant.data_ptr(), big.exps.data_ptr(),
                                           262146, 64, 4, None)
    assert rc == qk.BFP8_EINVAL and b"262144" in lib.bfp8_last_error()


def test_no_alloc_lm_head_allocates_nothing(gpu):
    """On a stream the library has never seen (the allocating entry would
    reserve that stream's scratch there; HIP has used it once), a call of the
    no-alloc entry leaves the device's free memory exactly as it was, and its
    result is the oracle's."""
    qk = gpu
    import torch

    lib = qk.load()
    V, H, k = 65536, 1024, 40
    r = np.random.default_rng(13)
    mant = r.integers(-128, 128, size=(V, H), dtype=np.int8)
    exps = r.integers(120, 131, size=(V, H // 64), dtype=np.uint8)
    x = r.standard_normal(H).astype(F32)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    _, xs, xsp = qk.quantize(torch.from_numpy(x).cuda())
    ids = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    sc = torch.zeros(k, dtype=torch.float32, device="cuda")
    cnt = torch.full((2,), -7, dtype=torch.int32, device="cuda")
    fresh = torch.cuda.Stream()
    with torch.cuda.stream(fresh):  # HIP's own first use of the stream, outside the measured call
        ids.fill_(-7)
    torch.cuda.synchronize()
    say("no-alloc lm_head free memory", V, H, k)
    free0 = torch.cuda.mem_get_info()[0]
    rc = lib.bfp8_dev_lm_head_topk_noalloc(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), cnt.data_ptr() + 4,
                                           xsp.data_ptr(), xs.data_ptr(), dm.mant.data_ptr(), dm.exps.data_ptr(),
                                           V, H, k, fresh.cuda_stream)
    qk.check(rc, "bfp8_dev_lm_head_topk_noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    y = ol.gemv_neon(x, mant, exps)[0]
    ids_ref, sc_ref = ol.topk(y, k)
    n = int(cnt[0].item())
    assert n == k and int(cnt[1].item()) == ol.argmax(y)
    assert np.array_equal(ids.cpu().numpy()[:n], ids_ref)
    assert np.array_equal(sc.cpu().numpy()[:n].view(np.uint32), sc_ref.view(np.uint32))
