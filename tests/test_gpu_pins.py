"""Hand-worked cases on the GPU, through the C ABI: the blocks that pin the
oracle's quantizer rounding order and unfused epilogue (tests/test_oracle.py)
give the same results on the device, and the engine's numpy fallback
(04/qwen_real_engine.py:1230-1238) matches the oracle's restatement of it in
both of numpy's summation orders."""
import sys

import numpy as np
import pytest

import oracle_lib as ol
from test_oracle import QUANT_ORDER_AMAX, QUANT_ORDER_X, epilogue_case

pytestmark = pytest.mark.gpu
F32 = np.float32


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def test_quantizer_rounding_order_on_the_gpu(gpu):
    qk = gpu
    import torch

    x = np.zeros(128, dtype=F32)
    x[0], x[1] = QUANT_ORDER_AMAX, QUANT_ORDER_X
    x[64:] = np.linspace(-3, 3, 64, dtype=F32)
    say("quantizer rounding order")
    xq, xs, _ = qk.quantize(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    xq_ref, xs_ref = ol.quant_x(x)
    assert xq.cpu().numpy()[1] == 2872
    assert np.array_equal(xq.cpu().numpy(), xq_ref) and np.array_equal(xs.cpu().numpy(), xs_ref)


def test_unfused_epilogue_on_the_gpu(gpu):
    """Both the device GEMV and the host bfp8_gemv give 2^24 where a fused
    multiply-add would give 2^24 + 2."""
    qk = gpu
    import torch

    mant, exps, x, _ = epilogue_case()
    say("unfused epilogue")
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    _, xs, xsp = qk.quantize(torch.from_numpy(x).cuda())
    y = qk.gemv(dm, xsp, xs)
    torch.cuda.synchronize()
    assert list(y.cpu().numpy()) == [2.0 ** 24, 2.0 ** 24]
    assert list(qk.Bfp8Kernels().gemv_bfp8(x, mant, exps, 2, 128)) == [2.0 ** 24, 2.0 ** 24]


@pytest.mark.parametrize("M,K", [(7, 64), (300, 1024), (1024, 3584), (65, 8320), (3, 0)])
@pytest.mark.parametrize("pairwise", [True, False])
def test_numpy_fallback_matches_the_oracle(gpu, M, K, pairwise):
    qk = gpu
    rng = np.random.default_rng(M + K + pairwise)
    mant = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    exps = rng.integers(0, 140, size=(M, K // 64), dtype=np.uint8)  # subnormal scales included
    x = (rng.standard_normal(K) * 10.0 ** rng.uniform(-6, 6, K)).astype(F32)
    say("numpy fallback", M, K, pairwise)
    y = qk.Bfp8Kernels().gemv_fallback(x, mant, exps, M, K, pairwise)
    y_ref = ol.gemv_fallback(x, mant, exps, pairwise)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))


def test_numpy_fallback_device_entry_and_argument_checks(gpu):
    qk = gpu
    import torch

    lib = qk.load()
    M, K = 513, 2048
    rng = np.random.default_rng(3)
    mant = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    exps = rng.integers(118, 136, size=(M, K // 64), dtype=np.uint8)
    x = rng.standard_normal(K).astype(F32)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    xd = torch.from_numpy(x).cuda()
    y = torch.empty(M, dtype=torch.float32, device="cuda")
    say("numpy fallback device entry")
    qk.check(lib.bfp8_dev_gemv_fallback(y.data_ptr(), xd.data_ptr(), dm.mant.data_ptr(), dm.exps.data_ptr(), M, K, 1,
                                        torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ol.gemv_fallback(x, mant, exps, True).view(np.uint32))
    assert lib.bfp8_dev_gemv_fallback(y.data_ptr(), xd.data_ptr(), dm.mant.data_ptr(), dm.exps.data_ptr(), M, 100, 1,
                                      None) == qk.BFP8_EINVAL
