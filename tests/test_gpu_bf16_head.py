"""GPU parity of the bf16 tied-embedding lm_head and the sampler.

lm_head_argmax (libqwen_kernels.so) and lm_head_topk / sample_from_topk
(libqwen_sampling.so) are called through their C ABI with host pointers, as
the reference engine and chat front end call them; the device-level entry
points are checked on the same inputs.  Scores are compared bit for bit with
the oracle's restatement of the board build's dot products."""
import ctypes
import sys

import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu
F32 = np.float32


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def same_f32(a, b):
    a = np.asarray(a, dtype=F32).reshape(-1)
    b = np.asarray(b, dtype=F32).reshape(-1)
    return bool(np.all((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))))


def table_and_h(vocab, hidden, seed, scale=0.05):
    rng = np.random.default_rng(seed)
    table = ol.f32_to_bf16_bits(rng.standard_normal((vocab, hidden), dtype=F32) * F32(scale))
    h = rng.standard_normal(hidden, dtype=F32)
    return np.ascontiguousarray(table), h


def host_topk(qk, h, table, k):
    smp = qk.load_sampling()
    ids = (ctypes.c_int * max(k, 1))()
    sc = (ctypes.c_float * max(k, 1))()
    n = smp.lm_head_topk(h.ctypes.data, table.ctypes.data, table.shape[0], table.shape[1], k, ids, sc)
    return np.array(ids[:n], dtype=np.int32), np.array(sc[:n], dtype=F32)


@pytest.fixture(scope="module")
def head_case():
    table, h = table_and_h(65536, 1024, 2024)
    return table, h, ol.bf16_logits(h, table, tail=0), ol.bf16_logits(h, table, tail=1)


def test_bf16_scores_bit_exact_full_vocab(gpu, head_case):
    qk = gpu
    import torch

    table, h, logits0, logits1 = head_case
    say("bf16 scores 65536x1024")
    lib = qk.load()
    t = torch.from_numpy(table.view(np.int16)).cuda()
    hd = torch.from_numpy(h).cuda()
    out = torch.empty(65536, dtype=torch.float32, device="cuda")
    for tail, ref in ((0, logits0), (1, logits1)):
        qk.check(lib.bf16_dev_lm_head(None, None, None, None, out.data_ptr(), hd.data_ptr(), t.data_ptr(),
                                      65536, 1024, 0, tail, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert same_f32(out.cpu().numpy(), ref), tail


def test_lm_head_argmax_and_topk_host_abi(gpu, head_case):
    qk = gpu
    table, h, logits0, logits1 = head_case
    lib = qk.load()
    say("lm_head_argmax host")
    assert lib.lm_head_argmax(h.ctypes.data, table.ctypes.data, 65536, 1024) == ol.argmax(logits0)
    for k in (1, 40, 64):
        say("lm_head_topk host", k)
        ids, sc = host_topk(qk, h, table, k)
        r_ids, r_sc = ol.topk(logits1, k)
        assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc), k


def test_ties_ragged_vocab_and_tail_rules(gpu):
    """Duplicated rows (ties broken by the lower id), a vocabulary that is not
    a multiple of 64, and hidden % 8 != 0, where lm_head_argmax drops the
    trailing elements and lm_head_topk adds them; hidden sizes above one
    512-byte row slice and up to the 4096 limit."""
    qk = gpu
    lib = qk.load()
    for vocab, hidden in ((1000, 1000), (4099, 1003), (130, 5), (64, 8), (1500, 1100), (3000, 2048), (300, 4096)):
        table, h = table_and_h(vocab, hidden, vocab + hidden)
        if vocab > 40:
            l1 = ol.bf16_logits(h, table, tail=1)
            top = np.argsort(-l1, kind="stable")[:10]
            for src in top:
                for dst in ((int(src) * 7 + 3) % vocab, (int(src) + vocab // 2) % vocab):
                    table[dst] = table[src]
        l0 = ol.bf16_logits(h, table, tail=0)
        l1 = ol.bf16_logits(h, table, tail=1)
        say("bf16 ragged", vocab, hidden)
        assert lib.lm_head_argmax(h.ctypes.data, table.ctypes.data, vocab, hidden) == ol.argmax(l0)
        for k in (1, 17, 64):
            ids, sc = host_topk(qk, h, table, k)
            r_ids, r_sc = ol.topk(l1, k)
            assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc), (vocab, hidden, k)


def test_nan_inf_hidden_state_and_invalid_arguments(gpu):
    qk = gpu
    lib = qk.load()
    table, h = table_and_h(512, 64, 77)
    h[3] = np.nan               # every score NaN: no candidate, argmax 0
    assert lib.lm_head_argmax(h.ctypes.data, table.ctypes.data, 512, 64) == ol.argmax(ol.bf16_logits(h, table, 0))
    assert host_topk(qk, h, table, 40)[0].size == 0
    h[3] = np.inf
    l1 = ol.bf16_logits(h, table, 1)
    ids, sc = host_topk(qk, h, table, 40)
    r_ids, r_sc = ol.topk(l1, 40)
    assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc)
    smp = qk.load_sampling()
    out = (ctypes.c_int * 4)()
    scs = (ctypes.c_float * 4)()
    assert smp.lm_head_topk(h.ctypes.data, table.ctypes.data, 512, 64, 0, out, scs) == 0
    assert smp.lm_head_topk(h.ctypes.data, table.ctypes.data, 0, 64, 4, out, scs) == 0
    assert smp.lm_head_topk(h.ctypes.data, table.ctypes.data, 512, 64, 65, out, scs) == 0   # above the fused limit
    assert lib.lm_head_argmax(h.ctypes.data, table.ctypes.data, 0, 64) == 0


def test_sampler_host_abi_matches_oracle(gpu):
    qk = gpu
    smp = qk.load_sampling()
    rng = np.random.default_rng(99)
    say("sampler host abi")
    for trial in range(120):
        n = int(rng.integers(1, 65))
        sc = np.sort(rng.standard_normal(n).astype(F32) * F32(rng.choice([0.1, 1.0, 8.0])))[::-1].copy()
        if trial % 4 == 0:
            rng.shuffle(sc)
        ids = rng.permutation(70000)[:n].astype(np.int32)
        temp = float(rng.choice([0.0, 0.3, 0.7, 1.0, 2.5]))
        top_k = int(rng.choice([0, 1, 5, 40]))
        top_p = float(rng.choice([0.0, 0.5, 0.9, 1.0]))
        state = int(rng.integers(0, 2**32))
        want = ol.sample_from_topk(ids, sc, temp, top_k, top_p, state)
        st = ctypes.c_uint(state)
        got = smp.sample_from_topk(ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                   sc.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n, temp, top_k, top_p,
                                   ctypes.byref(st))
        assert (got, st.value) == want, trial


def test_device_topk_then_sample_chain(gpu, head_case):
    """lm_head top-64 and the draw stay on the device (the sampler reads the
    candidate count the merge wrote); the xorshift32 state advances on the
    device across draws."""
    qk = gpu
    import torch

    table, h, _, logits1 = head_case
    lib = qk.load()
    s = torch.cuda.current_stream().cuda_stream
    t = torch.from_numpy(table.view(np.int16)).cuda()
    hd = torch.from_numpy(h).cuda()
    ids = torch.empty(64, dtype=torch.int32, device="cuda")
    sc = torch.empty(64, dtype=torch.float32, device="cuda")
    cnt = torch.empty(2, dtype=torch.int32, device="cuda")
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    rng_dev = torch.from_numpy(np.array([0x9E3779B9], dtype=np.uint32).view(np.int32)).cuda()
    work = torch.empty(64 * 2, dtype=torch.int32, device="cuda")
    r_ids, r_sc = ol.topk(logits1, 64)
    state = 0x9E3779B9
    say("device topk + sample chain")
    for draw in range(5):
        qk.check(lib.bf16_dev_lm_head(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), cnt.data_ptr() + 4, None,
                                      hd.data_ptr(), t.data_ptr(), 65536, 1024, 64, 1, s))
        qk.check(lib.bfp8_dev_sample_from_topk(out.data_ptr(), ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), 64,
                                               0.8, 40, 0.9, rng_dev.data_ptr(), work.data_ptr(), s))
        torch.cuda.synchronize()
        want, state = ol.sample_from_topk(r_ids, r_sc, 0.8, 40, 0.9, state)
        assert int(out.item()) == want, draw
        assert int(rng_dev.cpu().numpy().view(np.uint32)[0]) == state
        assert int(cnt[1].item()) == ol.argmax(logits1)
