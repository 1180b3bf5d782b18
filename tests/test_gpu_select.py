"""GPU parity of the lm_head selections over the reference's whole argument
range and of the sampler for any candidate count.

The reference's lm_head_topk returns min(k, vocab) entries for any k
(04/qwen_sampling.c:283-353; its self-test asks for k = vocab + 50, :953),
bfp8_gemv defines the odd last row (04/qwen_kernels_opt.c:279-306) and the
float path above K = 4096 (:311-325), and sample_from_topk takes any n
(:384-529).  Each case runs through the C ABI and is compared with the
oracle: ids identical, scores bit for bit."""
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
    return a.size == b.size and bool(np.all((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))))


def planes(V, H, seed, lo=-128, hi=128):
    r = np.random.default_rng(seed)
    mant = r.integers(lo, hi, size=(V, H), dtype=np.int8)
    exps = r.integers(120, 131, size=(V, max(H // 64, 1)), dtype=np.uint8)[:, : H // 64].copy()
    x = r.standard_normal(H).astype(F32)
    return mant, exps, x


def ref_logits(x, mant, exps):
    """bfp8_gemv's outputs: the quantized path up to K = 4096 (an odd last row
    in the scalar order), the float path above, zeros without a whole block."""
    V, H = mant.shape
    if H // 64 == 0:
        return np.zeros(V, dtype=F32)
    if H > 4096:
        return ol.gemv_float(x, mant, exps)
    return ol.gemv_neon(x, mant, exps)[0]


@pytest.mark.parametrize("V,H,k", [(4099, 1024, 40), (3001, 1024, 1), (3000, 1024, 65), (3000, 512, 200),
                                   (3000, 1024, 3050), (2049, 256, 64), (1001, 4160, 10), (500, 32, 7)])
def test_bfp8_lm_head_host_any_arguments(gpu, V, H, k):
    """Odd vocabularies, k above 64 and above the vocabulary, K above 4096 and
    below one block: bfp8_lm_head_topk / bfp8_lm_head_argmax take the general
    path (the plain GEMV's scores, then the selection)."""
    qk = gpu
    kk = qk.Bfp8Kernels()
    mant, exps, x = planes(V, H, V * 7 + H + k)
    y = ref_logits(x, mant, exps)
    say("bfp8 lm_head host", V, H, k)
    ids, sc = kk.lm_head_topk(x, mant, exps, V, H, k)
    ids_ref, sc_ref = ol.topk(y, k)
    assert ids.size == min(k, V)
    assert np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref), (V, H, k)
    assert kk.lm_head_argmax(x, mant, exps, V, H) == ol.argmax(y)


def test_bfp8_lm_head_odd_vocab_with_ties(gpu):
    """Equal scores across the odd last row and paired rows: ids ascending
    among equals, whichever epilogue order produced the score."""
    qk = gpu
    kk = qk.Bfp8Kernels()
    V, H = 2049, 128
    mant, exps, x = planes(V, H, 31, -1, 2)
    mant[V - 1] = mant[5]
    exps[V - 1] = exps[5]
    y = ref_logits(x, mant, exps)
    say("bfp8 lm_head odd vocab ties")
    for k in (1, 40, 64, 100):
        ids, sc = kk.lm_head_topk(x, mant, exps, V, H, k)
        ids_ref, sc_ref = ol.topk(y, k)
        assert np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref), k


@pytest.mark.parametrize("V,k", [(4099, 40), (65536, 100), (3000, 3050), (4097, 1)])
def test_bfp8_lm_head_device_any_arguments(gpu, V, k):
    """bfp8_dev_lm_head_topk on the caller's stream over the general range."""
    qk = gpu
    import torch

    H = 1024
    mant, exps, x = planes(V, H, V + k)
    y = ref_logits(x, mant, exps)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    _, xs, xsp = qk.quantize(torch.from_numpy(x).cuda())
    say("bfp8 lm_head device", V, k)
    ids, sc, cnt, am = qk.lm_head_topk(dm, xsp, xs, k)
    torch.cuda.synchronize()
    ids_ref, sc_ref = ol.topk(y, k)
    n = int(cnt.item())
    assert n == ids_ref.size
    assert np.array_equal(ids.cpu().numpy()[:n], ids_ref) and same_f32(sc.cpu().numpy()[:n], sc_ref)
    assert int(am.item()) == ol.argmax(y)


@pytest.mark.parametrize("k,ties", [(65, False), (200, False), (65586, False), (200, True), (65586, True)])
def test_k_above_64_at_the_full_vocabulary(gpu, k, ties):
    """k = 65, 200 and vocab + 50 over 65536 rows (bfp8_dev_lm_head_topk: the
    scores, then the selection of 4096-key blocks sorted in LDS and ranked
    against each other): ids and scores bit-exact against the oracle, the
    count and argmax too; with mantissas in {-1, 0, 1} many scores are equal
    and ids ascend among them."""
    qk = gpu
    import torch

    V, H = 65536, 1024
    mant, exps, x = planes(V, H, 6500 + k + ties, *((-1, 2) if ties else (-128, 128)))
    y = ref_logits(x, mant, exps)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    _, xs, xsp = qk.quantize(torch.from_numpy(x).cuda())
    say("k above 64 at 65536 rows", k, ties)
    ids, sc, cnt, am = qk.lm_head_topk(dm, xsp, xs, k)
    torch.cuda.synchronize()
    ids_ref, sc_ref = ol.topk(y, k)
    n = int(cnt.item())
    assert n == ids_ref.size == min(k, V)
    assert np.array_equal(ids.cpu().numpy()[:n], ids_ref) and same_f32(sc.cpu().numpy()[:n], sc_ref)
    assert int(am.item()) == ol.argmax(y)


@pytest.mark.parametrize("k", [40, 100])
def test_top_k_on_a_second_stream_and_the_host_entry(gpu, k):
    """Scratch is per stream: a device-level top-k queued on a second stream
    (not waited for) and the host entry bfp8_lm_head_topk (the library's own
    stream) right after it, then two device-level top-ks on two streams, each
    over its own lm_head, all against the oracle.  k = 40 takes the fused
    per-tile lists and the merge, k = 100 the scores and the selection."""
    qk = gpu
    import torch

    V, H = 65536, 1024
    kk = qk.Bfp8Kernels()
    mats = [planes(V, H, 9100 + i) for i in range(3)]
    refs = [ol.topk(ref_logits(x, mant, exps), k) for mant, exps, x in mats]
    dms = [qk.DeviceMatrix.from_soa(mant, exps) for mant, exps, _ in mats]
    xq = [qk.quantize(torch.from_numpy(x).cuda()) for _, _, x in mats]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    say("two streams", V, H, k)
    for rep in range(3):
        with torch.cuda.stream(s2):
            d0 = qk.lm_head_topk(dms[0], xq[0][2], xq[0][1], k)
        mant, exps, x = mats[1]
        ids_h, sc_h = kk.lm_head_topk(x, mant, exps, V, H, k)  # the library's stream, while s2 runs
        with torch.cuda.stream(s1):
            d1 = qk.lm_head_topk(dms[2], xq[2][2], xq[2][1], k)
        with torch.cuda.stream(s2):
            d2 = qk.lm_head_topk(dms[0], xq[0][2], xq[0][1], k)
        torch.cuda.synchronize()
        assert np.array_equal(ids_h, refs[1][0]) and same_f32(sc_h, refs[1][1]), rep
        for (ids, sc, cnt, _), (ids_ref, sc_ref) in ((d0, refs[0]), (d1, refs[2]), (d2, refs[0])):
            n = int(cnt.item())
            assert n == ids_ref.size, rep
            assert np.array_equal(ids.cpu().numpy()[:n], ids_ref) and same_f32(sc.cpu().numpy()[:n], sc_ref), rep


@pytest.mark.parametrize("case", ["odd_vocab", "k100", "k4160"])
def test_plan_with_a_general_lm_head(gpu, case):
    """A sweep plan whose lm_head item is outside the fused launch's range runs
    it as a plain GEMV into the plan's scores buffer and selects at the end;
    the other items are unaffected.  Run twice with fresh activations."""
    qk = gpu
    import torch

    V, H, k = {"odd_vocab": (4099, 1024, 40), "k100": (8192, 1024, 100), "k4160": (2000, 4160, 16)}[case]
    mant, exps, _ = planes(V, H, 77)
    g_shapes = [(640, 1024), (1025, 2048)]
    gm = [planes(M, K, 80 + i) for i, (M, K) in enumerate(g_shapes)]
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    gdm = [qk.DeviceMatrix.from_soa(m, e) for m, e, _ in gm]
    hx = torch.empty(H, dtype=torch.float32, device="cuda")
    gx = [torch.empty(K, dtype=torch.float32, device="cuda") for _, K in g_shapes]
    ys = [torch.empty(M, dtype=torch.float32, device="cuda") for M, _ in g_shapes]
    items = [{"mat": gdm[0], "x": gx[0], "y": ys[0]}, {"mat": dm, "x": hx, "topk": k},
             {"mat": gdm[1], "x": gx[1], "y": ys[1]}]
    plan = qk.SweepPlan(items)
    try:
        for run in range(2):
            r = np.random.default_rng(1000 * run + 5)
            xh = r.standard_normal(H).astype(F32)
            xg = [r.standard_normal(K).astype(F32) for _, K in g_shapes]
            hx.copy_(torch.from_numpy(xh))
            for t, v in zip(gx, xg):
                t.copy_(torch.from_numpy(v))
            say("plan general lm_head", case, run)
            plan.run()
            torch.cuda.synchronize()
            ids, sc, cnt = plan.topk_out
            n = int(cnt[0].item())
            y = ref_logits(xh, mant, exps)
            ids_ref, sc_ref = ol.topk(y, k)
            assert n == ids_ref.size
            assert np.array_equal(ids.cpu().numpy()[:n], ids_ref) and same_f32(sc.cpu().numpy()[:n], sc_ref)
            assert int(cnt[1].item()) == ol.argmax(y)
            for (m, e, _), v, yt in zip(gm, xg, ys):
                assert same_f32(yt.cpu().numpy(), ref_logits(v, m, e))
    finally:
        plan.close()


# ---- the bf16 tied-embedding lm_head -------------------------------------------------------------
def bf16_table(vocab, hidden, seed, scale=0.05):
    rng = np.random.default_rng(seed)
    table = ol.f32_to_bf16_bits(rng.standard_normal((vocab, hidden), dtype=F32) * F32(scale))
    return np.ascontiguousarray(table), rng.standard_normal(hidden, dtype=F32)


def host_topk(qk, h, table, k):
    smp = qk.load_sampling()
    ids = (ctypes.c_int * max(k, 1))()
    sc = (ctypes.c_float * max(k, 1))()
    n = smp.lm_head_topk(h.ctypes.data, table.ctypes.data, table.shape[0], table.shape[1], k, ids, sc)
    return np.array(ids[:n], dtype=np.int32), np.array(sc[:n], dtype=F32)


@pytest.mark.parametrize("vocab,hidden,k", [(3000, 1024, 65), (3000, 1003, 200), (3000, 64, 3050), (700, 5003, 40),
                                            (600, 8192, 100), (65536, 1024, 128)])
def test_bf16_lm_head_any_k_and_hidden(gpu, vocab, hidden, k):
    """lm_head_topk for k above 64 (up to past the vocabulary) and hidden above
    4096 (h read from global memory), lm_head_argmax at the same sizes."""
    qk = gpu
    lib = qk.load()
    table, h = bf16_table(vocab, hidden, vocab + hidden + k)
    l0 = ol.bf16_logits(h, table, tail=0)
    l1 = ol.bf16_logits(h, table, tail=1)
    say("bf16 any k / hidden", vocab, hidden, k)
    assert lib.lm_head_argmax(h.ctypes.data, table.ctypes.data, vocab, hidden) == ol.argmax(l0)
    ids, sc = host_topk(qk, h, table, k)
    r_ids, r_sc = ol.topk(l1, k)
    assert ids.size == min(k, vocab)
    assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc), (vocab, hidden, k)


def test_bf16_scalar_tail_keeps_subnormals(gpu):
    """lm_head_topk adds the hidden % 8 trailing products in scalar IEEE
    arithmetic (04/qwen_sampling.c:201-204): with the vector part zero and
    subnormal tail products the scores are subnormal, not flushed."""
    qk = gpu
    vocab, hidden = 500, 1027
    table, h = bf16_table(vocab, hidden, 123)
    h[:1024] = 0.0
    h[1024:] = np.array([3e-30, -2e-30, 5e-31], dtype=F32)
    tw = ol.f32_to_bf16_bits(np.random.default_rng(5).standard_normal((vocab, 3)).astype(F32) * F32(1e-9))
    table[:, 1024:] = tw
    l1 = ol.bf16_logits(h, table, tail=1)
    assert np.any((l1 != 0) & (np.abs(l1) < np.finfo(F32).tiny)), "the case must reach subnormal scores"
    say("bf16 subnormal tail")
    ids, sc = host_topk(qk, h, table, 64)
    r_ids, r_sc = ol.topk(l1, 64)
    assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc)
    # the device entry with every score written out
    import torch

    lib = qk.load()
    lg = torch.empty(vocab, dtype=torch.float32, device="cuda")
    t = torch.from_numpy(table.view(np.int16)).cuda()
    hd = torch.from_numpy(h).cuda()
    qk.check(lib.bf16_dev_lm_head(None, None, None, None, lg.data_ptr(), hd.data_ptr(), t.data_ptr(), vocab, hidden,
                                  0, 1, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert same_f32(lg.cpu().numpy(), l1)


@pytest.mark.parametrize("layout", ["rows", "tiles"])
def test_bf16_device_lm_head_k_above_64(gpu, layout):
    """bf16_dev_lm_head / bf16_dev_lm_head_tiles with k = 300 on the caller's
    stream: the scores, then the sort of all keys."""
    qk = gpu
    import torch

    lib = qk.load()
    vocab, hidden, k = 9000, 1024, 300
    table, h = bf16_table(vocab, hidden, 4242)
    tail = 1 if layout == "rows" else 0
    logits = ol.bf16_logits(h, table, tail=tail)
    s = torch.cuda.current_stream().cuda_stream
    t = torch.from_numpy(table.view(np.int16)).cuda()
    hd = torch.from_numpy(h).cuda()
    ids = torch.empty(k, dtype=torch.int32, device="cuda")
    sc = torch.empty(k, dtype=torch.float32, device="cuda")
    cnt = torch.empty(2, dtype=torch.int32, device="cuda")
    say("bf16 device k=300", layout)
    if layout == "rows":
        qk.check(lib.bf16_dev_lm_head(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), cnt.data_ptr() + 4, None,
                                      hd.data_ptr(), t.data_ptr(), vocab, hidden, k, 1, s))
    else:
        tt = torch.empty(lib.bf16_dev_tiles_bytes(vocab, hidden) // 2, dtype=torch.int16, device="cuda")
        qk.check(lib.bf16_dev_tile_table(tt.data_ptr(), t.data_ptr(), vocab, hidden, s))
        qk.check(lib.bf16_dev_lm_head_tiles(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), cnt.data_ptr() + 4, None,
                                            hd.data_ptr(), tt.data_ptr(), vocab, hidden, k, s))
    torch.cuda.synchronize()
    r_ids, r_sc = ol.topk(logits, k)
    assert int(cnt[0].item()) == k
    assert np.array_equal(ids.cpu().numpy(), r_ids) and same_f32(sc.cpu().numpy(), r_sc)
    assert int(cnt[1].item()) == ol.argmax(logits)


# ---- the sampler ---------------------------------------------------------------------------------
@pytest.mark.parametrize("n,shuffled", [(5000, False), (5000, True), (20000, True), (4097, True)])
def test_sampler_any_candidate_count(gpu, n, shuffled):
    """sample_from_topk over n > 4096 candidates, sorted and unsorted (the
    unsorted list ordered by (score desc, id asc) on a copy); some scores
    repeated so that the id order among equals matters."""
    qk = gpu
    smp = qk.load_sampling()
    rng = np.random.default_rng(n + shuffled)
    sc = np.sort(rng.standard_normal(n).astype(F32))[::-1].copy()
    sc[10:20] = sc[10]
    sc[n // 2: n // 2 + 7] = sc[n // 2]
    ids = rng.permutation(200000)[:n].astype(np.int32)
    if shuffled:
        perm = rng.permutation(n)
        sc, ids = sc[perm].copy(), ids[perm].copy()
    say("sampler n", n, shuffled)
    for temp, top_k, top_p in ((0.0, 0, 1.0), (0.8, 0, 1.0), (1.0, 0, 0.95), (0.7, 3000, 0.9), (2.0, 0, 0.0)):
        state = int(rng.integers(0, 2**32))
        want = ol.sample_from_topk(ids, sc, temp, top_k, top_p, state)
        st = ctypes.c_uint(state)
        got = smp.sample_from_topk(ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                   sc.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n, temp, top_k, top_p,
                                   ctypes.byref(st))
        assert (got, st.value) == want, (n, shuffled, temp, top_k, top_p)


def test_device_sampler_clamps_the_count(gpu):
    """bfp8_dev_sample_from_topk reads the candidate count from the device and
    clamps it to the capacity n (above: n; negative: no candidate, -1)."""
    qk = gpu
    import torch

    lib = qk.load()
    s = torch.cuda.current_stream().cuda_stream
    n = 300
    rng = np.random.default_rng(8)
    sc = rng.standard_normal(n).astype(F32)
    ids = np.arange(1000, 1000 + n, dtype=np.int32)
    d_ids, d_sc = torch.from_numpy(ids).cuda(), torch.from_numpy(sc).cuda()
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    work = torch.empty(2 * n, dtype=torch.int32, device="cuda")
    for cnt_val, want_n in ((n + 50, n), (n, n), (120, 120), (-3, 0)):
        cnt = torch.tensor([cnt_val], dtype=torch.int32, device="cuda")
        state = 0x1234567
        rng_dev = torch.from_numpy(np.array([state], dtype=np.uint32).view(np.int32)).cuda()
        say("device sampler count", cnt_val)
        qk.check(lib.bfp8_dev_sample_from_topk(out.data_ptr(), d_ids.data_ptr(), d_sc.data_ptr(), cnt.data_ptr(), n,
                                               0.9, 0, 1.0, rng_dev.data_ptr(), work.data_ptr(), s))
        torch.cuda.synchronize()
        if want_n == 0:
            assert int(out.item()) == -1
        else:
            want, st = ol.sample_from_topk(ids[:want_n], sc[:want_n], 0.9, 0, 1.0, state)
            assert int(out.item()) == want
            assert int(rng_dev.cpu().numpy().view(np.uint32)[0]) == st
