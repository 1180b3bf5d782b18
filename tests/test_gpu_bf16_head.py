"""GPU parity of the bf16 tied-embedding lm_head and the sampler.

lm_head_argmax (libqwen_kernels.so) and lm_head_topk / sample_from_topk
(libqwen_sampling.so) are called through their C ABI with host pointers, as
the reference engine and chat front end call them; the device-level entry
points are checked on the same inputs.  Scores are compared bit for bit with
the oracle's restatement of the board build's dot products."""
import ctypes
import mmap
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


def tile_layout(table):
    """The lm_head's tile layout: rows in groups of 16, nT = 4 * ceil(vocab /
    64) groups (rows past vocab zero); element e = 8c + j of row 16T + r, with
    c = 4q + cc, q = 2p + s and j = 4 hi + g, at uint16 offset
    (((p * nT + T) * 2 + s) * 64 + 4r + g) * 8 + 2 cc + hi."""
    vocab, hidden = table.shape
    nT = 4 * -(-vocab // 64)
    pad = np.zeros((nT * 16, hidden), dtype=np.uint16)
    pad[:vocab] = table
    # e = 64p + 32s + 8cc + 4hi + g: axes (T, r, p, s, cc, hi, g) -> (p, T, s, r, g, cc, hi)
    return pad.reshape(nT, 16, hidden // 64, 2, 4, 2, 4).transpose(2, 0, 3, 1, 6, 4, 5).reshape(-1)


def readonly_view(path, arr):
    """arr's bytes in a file mapped PROT_READ, as the engine maps its image."""
    arr.tofile(path)
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, prot=mmap.PROT_READ)
    return np.frombuffer(mm, dtype=arr.dtype).reshape(arr.shape)


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


def test_random_tables_against_the_oracle(gpu):
    """Eight seeded row-major tables: hidden 1-4,096 (any remainder mod 8),
    vocabularies up to 40 M elements in all, k in 1-64, half of the tables
    drawn from three values so that equal scores are common: argmax (tail
    dropped) and top-k (tail added) identical, scores bit-exact."""
    qk = gpu
    lib = qk.load()
    rng = np.random.default_rng(5150)
    for i in range(8):
        hidden = int(rng.integers(1, 4097))
        vocab = int(rng.integers(1, 40_000_000 // hidden + 1))
        k = int(rng.integers(1, 65))
        seed = int(rng.integers(0, 2**31))
        table, h = table_and_h(vocab, hidden, seed)
        if i % 2:
            r = np.random.default_rng(seed + 1)
            vals = ol.f32_to_bf16_bits(np.array([-0.05, 0.0, 0.05], dtype=F32))
            table = np.ascontiguousarray(vals[r.integers(0, 3, size=(vocab, hidden))])
        say("bf16 random", vocab, hidden, k, seed)
        l0 = ol.bf16_logits(h, table, tail=0)
        l1 = ol.bf16_logits(h, table, tail=1)
        assert lib.lm_head_argmax(h.ctypes.data, table.ctypes.data, vocab, hidden) == ol.argmax(l0), (vocab, hidden)
        ids, sc = host_topk(qk, h, table, k)
        r_ids, r_sc = ol.topk(l1, k)
        assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc), (vocab, hidden, k, seed)


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


def test_tile_layout_and_tiled_lm_head(gpu, head_case):
    """bf16_dev_tile_table writes the documented layout byte for byte, and the
    tile kernel's scores, top-64 and argmax equal the oracle's bit for bit:
    the full vocabulary, a ragged one with duplicated rows (ties), a
    single-tile one and NaN / inf hidden states."""
    qk = gpu
    import torch

    lib = qk.load()
    s = torch.cuda.current_stream().cuda_stream
    assert lib.bf16_dev_tiles_bytes(65536, 1024) == 65536 * 1024 * 2
    assert lib.bf16_dev_tiles_bytes(1000, 1024) == 1024 * 1024 * 2
    assert lib.bf16_dev_tiles_bytes(1000, 1000) == 0 and lib.bf16_dev_tiles_bytes(0, 1024) == 0
    table, h, logits0, _ = head_case
    cases = [(table, h, logits0)]
    for vocab, seed in ((1000, 5), (64, 6), (4099, 7)):
        t2, h2 = table_and_h(vocab, 1024, seed)
        l2 = ol.bf16_logits(h2, t2, tail=0)
        for src in np.argsort(-l2, kind="stable")[:8]:
            t2[(int(src) * 7 + 3) % vocab] = t2[src]
        cases.append((t2, h2, ol.bf16_logits(h2, t2, tail=0)))
    # equal scores (every row the same, or three distinct rows): ties broken by
    # the row alone, the selection's histogram bins refined down to the row bits
    row = table[:1]
    t_eq = np.ascontiguousarray(np.repeat(row, 5000, axis=0))
    cases.append((t_eq, h, ol.bf16_logits(h, t_eq, tail=0)))
    t3 = np.ascontiguousarray(table[np.random.default_rng(9).integers(0, 3, 9000)])
    cases.append((t3, h, ol.bf16_logits(h, t3, tail=0)))
    hn = h.copy()
    hn[5] = np.inf
    cases.append((table, hn, ol.bf16_logits(hn, table, tail=0)))
    hn = h.copy()
    hn[700] = np.nan
    cases.append((table, hn, ol.bf16_logits(hn, table, tail=0)))
    for tb, hv, ref in cases:
        vocab = tb.shape[0]
        say("bf16 tiles", vocab, "nonfinite" if not np.all(np.isfinite(hv)) else "")
        t = torch.from_numpy(tb.view(np.int16)).cuda()
        tiles = torch.empty(lib.bf16_dev_tiles_bytes(vocab, 1024) // 2, dtype=torch.int16, device="cuda")
        qk.check(lib.bf16_dev_tile_table(tiles.data_ptr(), t.data_ptr(), vocab, 1024, s))
        hd = torch.from_numpy(hv).cuda()
        logits = torch.empty(vocab, dtype=torch.float32, device="cuda")
        ids = torch.empty(64, dtype=torch.int32, device="cuda")
        sc = torch.empty(64, dtype=torch.float32, device="cuda")
        cnt = torch.empty(2, dtype=torch.int32, device="cuda")
        qk.check(lib.bf16_dev_lm_head_tiles(None, None, None, None, logits.data_ptr(), hd.data_ptr(),
                                            tiles.data_ptr(), vocab, 1024, 0, s))
        torch.cuda.synchronize()
        assert np.array_equal(tiles.cpu().numpy().view(np.uint16), tile_layout(tb)), vocab
        assert same_f32(logits.cpu().numpy(), ref), vocab
        for k in (1, 40, 64):
            qk.check(lib.bf16_dev_lm_head_tiles(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(), cnt.data_ptr() + 4,
                                                None, hd.data_ptr(), tiles.data_ptr(), vocab, 1024, k, s))
            torch.cuda.synchronize()
            r_ids, r_sc = ol.topk(ref, k)
            n = int(cnt[0].item())
            assert n == r_ids.size, (vocab, k)
            assert np.array_equal(ids[:n].cpu().numpy(), r_ids) and same_f32(sc[:n].cpu().numpy(), r_sc), (vocab, k)
            assert int(cnt[1].item()) == ol.argmax(ref), (vocab, k)
    assert lib.bf16_dev_tile_table(tiles.data_ptr(), t.data_ptr(), 64, 1000, s) != 0
    assert lib.bf16_dev_lm_head_tiles(None, None, None, None, logits.data_ptr(), hd.data_ptr(), tiles.data_ptr(),
                                      64, 1000, 0, s) != 0


def test_host_lm_head_on_a_readonly_table_uses_the_cached_tiles(gpu, head_case, tmp_path):
    """A read-only table (the engine's PROT_READ image) is cached on the device
    in the tile layout: lm_head_argmax / lm_head_topk keep the oracle's
    results on the first call (conversion) and on later calls (cache hit),
    and after bfp8_cache_clear."""
    qk = gpu
    lib = qk.load()
    table, h, logits0, logits1 = head_case
    ro = readonly_view(tmp_path / "embed.bin", table)
    lib.bfp8_cache_clear()
    try:
        for rep in range(2):
            say("read-only table host lm_head", rep)
            assert lib.lm_head_argmax(h.ctypes.data, ro.ctypes.data, 65536, 1024) == ol.argmax(logits0)
            for k in (1, 64):
                ids, sc = host_topk(qk, h, ro, k)
                r_ids, r_sc = ol.topk(logits1, k)
                assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc), (rep, k)
        t2, h2 = table_and_h(1000, 1024, 8)
        ro2 = readonly_view(tmp_path / "embed2.bin", t2)
        say("read-only ragged table")
        l2 = ol.bf16_logits(h2, t2, tail=1)
        assert lib.lm_head_argmax(h2.ctypes.data, ro2.ctypes.data, 1000, 1024) == ol.argmax(l2)
        ids, sc = host_topk(qk, h2, ro2, 64)
        r_ids, r_sc = ol.topk(l2, 64)
        assert np.array_equal(ids, r_ids) and same_f32(sc, r_sc)
    finally:
        lib.bfp8_cache_clear()
