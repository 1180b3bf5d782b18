"""GPU parity: the HIP kernels against the CPU oracle, bit for bit.

Shapes are the real ones (3584x1024, 1024x3584, 65536x1024, the 24-layer
sweep, B=16); inputs come from the library's seeded generators and are fed
identically to the GPU and to the oracle.  Floats are compared as bit
patterns (NaN compared as NaN: the reference's NEON default-NaN payload is
not reproduced)."""
import os
import sys
import tempfile

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
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


def mismatch(a, b):
    a = np.asarray(a, dtype=F32).reshape(-1)
    b = np.asarray(b, dtype=F32).reshape(-1)
    bad = np.nonzero(~((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))))[0]
    return f"{bad.size} mismatches, first {bad[:5]}: {a[bad[:5]]} vs {b[bad[:5]]}"


def encode_xsplit(xq):
    """The split-activation layout (bfp8_layout.h) built from int16 xq."""
    xq = np.asarray(xq, dtype=np.int32)
    nb = xq.size // 64
    xl = ((xq & 0xFF) ^ 0x80) - 0x80
    xh = (xq - xl) >> 8
    out = np.zeros((nb, 4, 8), dtype=np.uint32)
    for k in range(64):
        q, i = k & 3, k >> 2
        d, p = i >> 2, i & 3
        out[:, q, d] |= (xh[k::64].astype(np.uint32) & 0xFF) << (8 * p)
        out[:, q, 4 + d] |= (xl[k::64].astype(np.uint32) & 0xFF) << (8 * p)
    return out.reshape(-1).view(np.int32)


def decode_xsplit(words, nb):
    w = np.asarray(words, dtype=np.int32).view(np.uint32)[: nb * 32].reshape(nb, 4, 8)
    xq = np.zeros(nb * 64, dtype=np.int32)
    for k in range(64):
        q, i = k & 3, k >> 2
        d, p = i >> 2, i & 3
        h = ((w[:, q, d] >> (8 * p)) & 0xFF).astype(np.int32)
        l = ((w[:, q, 4 + d] >> (8 * p)) & 0xFF).astype(np.int32)
        h = (h ^ 0x80) - 0x80
        l = (l ^ 0x80) - 0x80
        xq[k::64] = 256 * h + l
    return xq


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    return torch


def run_gemv_dev(qk, torch, mant, exps, x, lanes=True):
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=F32)).cuda()
    xq, xs, xsp = qk.quantize(xt)
    if lanes:
        y, ln = qk.gemv(dm, xsp, xs, lane_sums=True)
    else:
        y, ln = qk.gemv(dm, xsp, xs), None
    torch.cuda.synchronize()
    return (y.cpu().numpy(), xq.cpu().numpy(), xs.cpu().numpy(), xsp.cpu().numpy(),
            None if ln is None else ln.cpu().numpy())


# ---- quantizer -------------------------------------------------------------------------------

def test_gpu_ready_on_the_gpu_box(gpu):
    """init_kernels() then bfp8_gpu_ready(): 1 on a gfx950 device with this
    library's code object loaded (the check an engine makes to keep the GPU
    path)."""
    lib = gpu.load()
    lib.init_kernels()
    assert lib.bfp8_gpu_ready() == 1, lib.bfp8_last_error()

def test_quantize_bit_exact_with_special_values(gpu, torch_mod):
    qk, torch = gpu, torch_mod
    rng = np.random.default_rng(11)
    K = 4096
    x = (rng.standard_normal(K) * np.repeat(10.0 ** rng.uniform(-12, 12, K // 64), 64)).astype(F32)
    x[0:64] = 0.0
    x[64:128] = F32(1e-20)
    x[128:192] = np.nextafter(F32(0), F32(1)) * np.arange(64, dtype=F32)  # subnormals only
    x[192] = 16384.0
    x[193:200] = [2.5, 3.5, -2.5, -3.5, 0.5, 1.5, 16383.5]
    x[260] = np.nan
    x[330] = np.inf
    x[400] = -np.inf
    x[470:480] = -F32(0.0)
    x[600] = F32(1.5e-38)  # subnormal next to normals
    say("quantize K=4096 specials")
    xt = torch.from_numpy(x).cuda()
    xq, xs, xsp = qk.quantize(xt)
    torch.cuda.synchronize()
    xq_ref, xs_ref = ol.quant_x(x)
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    assert same_f32(xs.cpu().numpy(), xs_ref)
    assert np.array_equal(decode_xsplit(xsp.cpu().numpy(), K // 64), xq_ref.astype(np.int32))


@pytest.mark.parametrize("K", [64, 1024, 2048, 3584])
def test_quantize_random_scales(gpu, torch_mod, K):
    qk, torch = gpu, torch_mod
    rng = np.random.default_rng(K)
    for trial in range(20):
        x = (rng.standard_normal(K) * 10.0 ** rng.uniform(-30, 30)).astype(F32)
        xq, xs, _ = qk.quantize(torch.from_numpy(x).cuda())
        xq_ref, xs_ref = ol.quant_x(x)
        assert np.array_equal(xq.cpu().numpy(), xq_ref), trial
        assert same_f32(xs.cpu().numpy(), xs_ref), trial


# ---- layout converter -------------------------------------------------------------------------
@pytest.mark.parametrize("M,K", [(1, 64), (65, 192), (3584, 1024), (1024, 3584), (3, 100)])
def test_pack_unpack_round_trip(gpu, torch_mod, M, K):
    qk, torch = gpu, torch_mod
    mant, exps = qk.synth_planes(M, K, 1000 + M, 0, 255)
    say("pack/unpack", M, K)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    ms, es = dm.unpack()
    torch.cuda.synchronize()
    nb = K // 64
    assert np.array_equal(es.cpu().numpy(), exps[:, :nb])
    back = ms.cpu().numpy()
    assert np.array_equal(back[:, : nb * 64], mant[:, : nb * 64])


def test_gpu_synth_matches_host_synth(gpu, torch_mod):
    qk, torch = gpu, torch_mod
    M, K = 1000, 1024
    say("synth planes")
    dm = qk.DeviceMatrix.synth(M, K, 77, 124, 130)
    ms, es = dm.unpack()
    mant, exps = qk.synth_planes(M, K, 77, 124, 130)
    assert np.array_equal(ms.cpu().numpy(), mant) and np.array_equal(es.cpu().numpy(), exps)


# ---- GEMV at the configured shapes -----------------------------------------------------------------
def test_known_answer_279616_on_gpu(gpu, torch_mod):
    """All-0x01 weights and xq = 0x1111: every block sums to 279616."""
    qk, torch = gpu, torch_mod
    M, K = 3584, 1024
    mant = np.ones((M, K), dtype=np.int8)
    exps = np.full((M, K // 64), 134, dtype=np.uint8)
    say("KAT 279616")
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    xsp = torch.from_numpy(encode_xsplit(np.full(K, 0x1111, dtype=np.int16))).cuda()
    xs = torch.ones(K // 64, dtype=torch.float32, device="cuda")
    y, lanes = qk.gemv(dm, xsp, xs, lane_sums=True)
    ln = lanes.cpu().numpy()
    assert (ln == 16 * 0x1111).all() and (ln.sum(-1) == 279616).all()
    assert (y.cpu().numpy() == F32(279616 * 16)).all()


@pytest.mark.parametrize("M,K,elo,ehi,seed", [
    (3584, 1024, 124, 130, 1),   # single GEMV, batch 1
    (1024, 3584, 124, 130, 2),   # down projection
    (6144, 1024, 124, 130, 3),   # in-projection stand-in
    (1024, 2048, 124, 130, 4),   # out-projection stand-in
    (40000, 1024, 122, 128, 5),  # 625 row tiles: the persistent streaming kernel
    (2048, 4096, 124, 130, 6),   # K = 4096: the widest block slice (16 blocks)
])
def test_gemv_configured_shapes(gpu, torch_mod, M, K, elo, ehi, seed):
    qk, torch = gpu, torch_mod
    mant, exps = qk.synth_planes(M, K, seed, elo, ehi)
    x = qk.synth_swiglu(K, seed + 50) if K == 3584 else qk.synth_normal(K, seed + 50)
    say("gemv", M, K)
    y, xq, xs, _, lanes = run_gemv_dev(qk, torch, mant, exps, x)
    y_ref, xq_ref, xs_ref, lanes_ref = ol.gemv_neon(x, mant, exps)
    assert np.array_equal(xq, xq_ref) and same_f32(xs, xs_ref)
    assert np.array_equal(lanes, lanes_ref)
    assert same_f32(y, y_ref), mismatch(y, y_ref)


def test_gate_up_down_chain(gpu, torch_mod):
    """Down projection chained after gate+up: three GEMVs on one stream."""
    qk, torch = gpu, torch_mod
    gate = qk.synth_planes(3584, 1024, 21, 124, 130)
    up = qk.synth_planes(3584, 1024, 22, 124, 130)
    down = qk.synth_planes(1024, 3584, 23, 124, 130)
    xh = qk.synth_normal(1024, 24)
    xd = qk.synth_swiglu(3584, 25, 0.01, 20.0)
    say("gate/up/down chain")
    kk = qk.Bfp8Kernels()
    for (m, e), x in ((gate, xh), (up, xh), (down, xd)):
        y = kk.gemv_bfp8(x, m, e, m.shape[0], m.shape[1])
        y_ref, *_ = ol.gemv_neon(x, m, e)
        assert same_f32(y, y_ref), mismatch(y, y_ref)


@pytest.mark.parametrize("M,K", [(1, 64), (7, 64), (65, 1024), (129, 3584), (3, 100), (5, 1000), (2, 63), (9, 4096)])
def test_odd_rows_ragged_k_and_flushed_exponents(gpu, torch_mod, M, K):
    qk, torch = gpu, torch_mod
    rng = np.random.default_rng(M * 7919 + K)
    mant = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    exps = rng.integers(0, 256, size=(M, max(K // 64, 0)), dtype=np.uint8)
    if exps.size:
        exps[:, 0] = rng.integers(0, 8, size=M)  # subnormal EXP_SCALE
    x = (rng.standard_normal(K) * 1e-3).astype(F32)
    if K >= 128:
        x[64:128] = 0.0
    say("odd/ragged", M, K)
    y = qk.Bfp8Kernels().gemv_bfp8(x, mant, exps, M, K)
    y_ref, *_ = ol.gemv_neon(x, mant, exps)
    assert same_f32(y, y_ref), mismatch(y, y_ref)


@pytest.mark.parametrize("case", ["m5_k4160"])
def test_float_path_above_4096_matches_reference_build(gpu, torch_mod, case):
    """K > 4096 takes the reference's float path; the fixture holds the output
    of the reference's own host build."""
    qk = gpu
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_float_path.npz"))
    x, mant, exps, y_fix = (d[f"{case}_{k}"] for k in ("x", "mant", "exps", "y"))
    say("float path", mant.shape)
    y = qk.Bfp8Kernels().gemv_bfp8(x, mant, exps, *mant.shape)
    assert same_f32(y, y_fix), mismatch(y, y_fix)
    mant2, exps2 = qk.synth_planes(33, 8192, 5, 0, 255)
    x2 = qk.synth_normal(8192, 6)
    y2 = qk.Bfp8Kernels().gemv_bfp8(x2, mant2, exps2, 33, 8192)
    assert same_f32(y2, ol.gemv_float(x2, mant2, exps2))


def test_nan_and_inf_activations(gpu, torch_mod):
    qk, torch = gpu, torch_mod
    M, K = 64, 256
    mant, exps = qk.synth_planes(M + 1, K, 31, 124, 130)
    x = qk.synth_normal(K, 32)
    x[5] = np.nan
    x[70] = np.inf
    say("nan/inf")
    y = qk.Bfp8Kernels().gemv_bfp8(x, mant, exps, M + 1, K)
    y_ref, *_ = ol.gemv_neon(x, mant, exps)
    assert same_f32(y, y_ref), mismatch(y, y_ref)


# ---- host-pointer boundary -------------------------------------------------------------------------
def test_writable_weights_follow_their_contents(gpu, torch_mod):
    qk = gpu
    M, K = 256, 1024
    mant, exps = qk.synth_planes(M, K, 41, 124, 130)
    x = qk.synth_normal(K, 42)
    kk = qk.Bfp8Kernels()
    say("writable weights")
    y1 = kk.gemv_bfp8(x, mant, exps, M, K)
    mant[:, :] = np.roll(mant, 1, axis=0)
    y2 = kk.gemv_bfp8(x, mant, exps, M, K)
    assert same_f32(y2, ol.gemv_neon(x, mant, exps)[0]) and not same_f32(y1, y2)


def test_read_only_mapped_weights_are_cached(gpu, torch_mod):
    """The engine's weights are a PROT_READ mmap (04/qwen_real_engine.py:745-751)."""
    qk = gpu
    M, K = 3584, 1024
    mant, exps = qk.synth_planes(M, K, 43, 124, 130)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "w.bin")
        with open(path, "wb") as f:
            f.write(mant.tobytes())
            f.write(exps.tobytes())
        raw = np.memmap(path, dtype=np.uint8, mode="r")
        mm = raw[: M * K].view(np.int8)
        ee = raw[M * K: M * K + M * K // 64]
        kk = qk.Bfp8Kernels()
        say("read-only mmap weights")
        for seed in (44, 45, 46):
            x = qk.synth_normal(K, seed)
            y = kk.gemv_bfp8(x, mm, ee, M, K)
            assert same_f32(y, ol.gemv_neon(x, mant, exps)[0])
        del raw, mm, ee
    kk.lib.bfp8_cache_clear()


def test_profiler_slots_untouched_by_direct_calls(gpu, torch_mod):
    """As in the reference (QP_TIME appears only inside the forward loop,
    04/qwen_kernels_opt.c:943-1047), a bfp8_gemv called from the host books
    nothing; the forward's slots are checked in test_gpu_runtime."""
    qk = gpu
    kk = qk.Bfp8Kernels()
    lib = kk.lib
    lib.qwen_prof_reset()
    lib.qwen_prof_enable(1)
    mant, exps = qk.synth_planes(128, 1024, 47, 124, 130)
    kk.gemv_bfp8(qk.synth_normal(1024, 48), mant, exps, 128, 1024)
    lib.qwen_prof_enable(0)
    assert all(lib.qwen_prof_get(i) == 0.0 for i in range(lib.qwen_prof_count()))


# ---- fused lm_head -------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lm_head_case(gpu):
    qk = gpu
    V, H = 65536, 1024
    mant, exps = qk.synth_planes(V, H, 500, 122, 128)
    x = qk.synth_normal(H, 501)
    y_ref, *_ = ol.gemv_neon(x, mant, exps)
    return mant, exps, x, y_ref


@pytest.mark.parametrize("k", [1, 40, 64])
def test_lm_head_topk_fused(gpu, torch_mod, lm_head_case, k):
    qk, torch = gpu, torch_mod
    mant, exps, x, y_ref = lm_head_case
    say("lm_head fused top-k", k)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    _, xs, xsp = qk.quantize(torch.from_numpy(x).cuda())
    for rep in range(3):  # repeated launches reuse the partials workspace
        ids, sc, cnt, am = qk.lm_head_topk(dm, xsp, xs, k)
        torch.cuda.synchronize()
        ids_ref, sc_ref = ol.topk(y_ref, k)
        n = int(cnt.item())
        assert n == ids_ref.size
        assert np.array_equal(ids.cpu().numpy()[:n], ids_ref), rep
        assert same_f32(sc.cpu().numpy()[:n], sc_ref)
        assert int(am.item()) == ol.argmax(y_ref)


def test_lm_head_host_api_and_ties(gpu, torch_mod, lm_head_case):
    qk = gpu
    mant, exps, x, y_ref = lm_head_case
    mant = mant.copy()
    exps = exps.copy()
    top = np.argsort(-y_ref, kind="stable")[:50]
    # duplicate the best rows elsewhere (both lower and higher ids): equal logits
    for j, src in enumerate(top[:20]):
        for dst in (int(src) ^ 0x8000, (int(src) + 12345) % 65536):
            mant[dst] = mant[src]
            exps[dst] = exps[src]
    y2, *_ = ol.gemv_neon(x, mant, exps)
    assert len(np.unique(y2[np.argsort(-y2, kind="stable")[:40]])) < 40  # ties present
    kk = qk.Bfp8Kernels()
    say("lm_head host api with ties")
    for k in (40, 64):
        ids, sc = kk.lm_head_topk(x, mant, exps, 65536, 1024, k)
        ids_ref, sc_ref = ol.topk(y2, k)
        assert np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref)
    assert kk.lm_head_argmax(x, mant, exps, 65536, 1024) == ol.argmax(y2)


def test_lm_head_small_vocab_and_invalid_arguments(gpu, torch_mod):
    qk = gpu
    kk = qk.Bfp8Kernels()
    mant, exps = qk.synth_planes(100, 128, 60, 124, 130)
    x = qk.synth_normal(128, 61)
    y_ref, *_ = ol.gemv_neon(x, mant, exps)
    say("lm_head small vocab")
    ids, sc = kk.lm_head_topk(x, mant, exps, 100, 128, 64)
    ids_ref, sc_ref = ol.topk(y_ref, 64)
    assert np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref)
    ids, _ = kk.lm_head_topk(x, mant, exps, 30, 128, 64)  # k > vocab -> min(k, vocab)
    assert np.array_equal(ids, ol.topk(y_ref[:30], 64)[0])
    # an odd vocabulary: the last row in the scalar order of the odd-M tail
    y99, *_ = ol.gemv_neon(x, mant[:99], exps[:99])
    ids, sc = kk.lm_head_topk(x, mant, exps, 99, 128, 40)
    ids_ref, sc_ref = ol.topk(y99, 40)
    assert np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref)
    assert kk.lm_head_argmax(x, mant, exps, 99, 128) == ol.argmax(y99)
    ids, sc = kk.lm_head_topk(x, mant, exps, 100, 128, 65)  # k above the fused launch's 64
    ids_ref, sc_ref = ol.topk(y_ref, 65)
    assert ids.size == 65 and np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref)
    assert kk.lm_head_topk(x, mant, exps, 100, 128, 0)[0].size == 0
    assert kk.lm_head_topk(x, mant, exps, 0, 128, 5)[0].size == 0
    assert kk.lm_head_argmax(x, mant, exps, 0, 128) == -1


def test_random_lm_heads_against_the_oracle(gpu, torch_mod):
    """Eight seeded lm_heads: even vocabularies of 2-140,000 rows, hidden 64-1,024
    (whole blocks), k in 1-64, half of them with mantissas in {-1, 0, 1} so that
    equal scores are common: ids (ties broken by the lower id), scores bit-exact
    and the argmax against the restatement."""
    qk = gpu
    kk = qk.Bfp8Kernels()
    rng = np.random.default_rng(9091)
    for i in range(8):
        V = int(rng.integers(1, 70001)) * 2
        H = int(rng.integers(1, 17)) * 64
        k = int(rng.integers(1, 65))
        seed = int(rng.integers(0, 2**31))
        r = np.random.default_rng(seed)
        lo, hi = (-1, 2) if i % 2 else (-128, 128)
        mant = r.integers(lo, hi, size=(V, H), dtype=np.int8)
        exps = r.integers(120, 131, size=(V, H // 64), dtype=np.uint8)
        x = r.standard_normal(H).astype(F32)
        say("random lm_head", V, H, k, seed)
        y_ref, *_ = ol.gemv_neon(x, mant, exps)
        ids, sc = kk.lm_head_topk(x, mant, exps, V, H, k)
        ids_ref, sc_ref = ol.topk(y_ref, k)
        assert np.array_equal(ids, ids_ref) and same_f32(sc, sc_ref), (V, H, k, seed)
        assert kk.lm_head_argmax(x, mant, exps, V, H) == ol.argmax(y_ref), (V, H, seed)


@pytest.mark.parametrize("other", ["small", "queue"])
@pytest.mark.parametrize("k", [2, 5, 40, 64])
def test_lm_head_one_tile_holds_the_best(gpu, torch_mod, k, other):
    """One 64-row tile's exponents sit 8 above the others', so most of the best
    rows share its partial list: the merge's threshold selection keeps reading
    that list past the entries it loads up front.  Stand-alone merge (16
    wavefronts), then in a plan with another GEMV: folded into the second
    launch (4 wavefronts; a 128 x 256 GEMV, too narrow for the single launch)
    or in the single launch (epoch-tagged keys; a 256 x 1024 GEMV); ids,
    scores, count and argmax against the restatement."""
    qk, torch = gpu, torch_mod
    V, H = 65536, 1024
    mant, exps = qk.synth_planes(V, H, 910, 122, 128)
    exps = exps.copy()
    exps[64 * 517:64 * 518] += 8
    x = qk.synth_normal(H, 911)
    y_ref, *_ = ol.gemv_neon(x, mant, exps)
    ids_ref, sc_ref = ol.topk(y_ref, k)
    assert np.sum((ids_ref >= 64 * 517) & (ids_ref < 64 * 518)) >= min(k, 20)
    say("lm_head one tile holds the best", k, other)
    dm = qk.DeviceMatrix.from_soa(mant, exps)
    xt = torch.from_numpy(x).cuda()
    _, xs, xsp = qk.quantize(xt)
    ids, sc, cnt, am = qk.lm_head_topk(dm, xsp, xs, k)
    torch.cuda.synchronize()
    assert int(cnt.item()) == k and int(am.item()) == ol.argmax(y_ref)
    assert np.array_equal(ids.cpu().numpy(), ids_ref) and same_f32(sc.cpu().numpy(), sc_ref)
    OM, OK = (128, 256) if other == "small" else (256, 1024)
    sm, se = qk.synth_planes(OM, OK, 912, 124, 130)
    xo = qk.synth_normal(OK, 913)
    items = [{"mat": dm, "x": xt, "topk": k},
             {"mat": qk.DeviceMatrix.from_soa(sm, se), "x": torch.from_numpy(xo).cuda(),
              "y": torch.empty(OM, dtype=torch.float32, device="cuda")}]
    plan = qk.SweepPlan(items)
    assert plan.kernel_name(0) == ("bfp8_gemv_head_kernel" if other == "small" else "bfp8_sweep_kernel")
    for rep in range(2):
        plan.run()
        torch.cuda.synchronize()
        ids, sc, cnt = plan.topk_out
        assert int(cnt[0].item()) == k and int(cnt[1].item()) == ol.argmax(y_ref), rep
        assert np.array_equal(ids.cpu().numpy(), ids_ref) and same_f32(sc.cpu().numpy(), sc_ref), rep
        assert same_f32(items[1]["y"].cpu().numpy(), ol.gemv_neon(xo, sm, se)[0]), rep
    plan.close()


def test_small_plan_one_tile_per_workgroup(gpu, torch_mod):
    """A plan without an lm_head and with few row tiles runs its GEMVs one tile
    per 16-wavefront workgroup; an odd-M item adds the tail-row kernel and a
    K > 4096 item the float path."""
    qk, torch = gpu, torch_mod
    shapes = [(3584, 1024), (1024, 3584), (1023, 2048), (130, 64), (2048, 4096), (64, 4160)]
    items, refs = [], []
    for j, (M, K) in enumerate(shapes):
        dm = qk.DeviceMatrix.synth(M, K, 4242 + j, 124, 130)
        x = qk.synth_swiglu(K, 4300 + j) if K == 3584 else qk.synth_normal(K, 4300 + j)
        items.append({"mat": dm, "x": torch.from_numpy(x).cuda(), "y": torch.empty(M, dtype=torch.float32, device="cuda")})
        refs.append((M, K, 4242 + j, x))
    plan = qk.SweepPlan(items)
    assert plan.kernel_name(1) == "bfp8_gemv_wide_grouped_kernel"
    say("small plan")
    for rep in range(2):
        for it in items:
            it["y"].fill_(np.nan)
        plan.run()
        torch.cuda.synchronize()
        for it, (M, K, seed, x) in zip(items, refs):
            mant, exps = qk.synth_planes(M, K, seed, 124, 130)
            y_ref = ol.gemv_neon(x, mant, exps)[0] if K <= 4096 else ol.gemv_float(x, mant, exps)
            assert same_f32(it["y"].cpu().numpy(), y_ref), (rep, M, K, mismatch(it["y"].cpu().numpy(), y_ref))
    plan.close()


ROWS_CASES = {
    "one": [(3584, 1024)],                              # 16-row sub-tiles
    "one_ragged_odd": [(1023, 1000)],                   # 4-row sub-tiles, XCD-paired grid of 256
    "one_8_rows": [(1500, 2048)],                       # 8-row sub-tiles (375 four-row groups > 256)
    "one_4_rows_down": [(1024, 3584)],                  # the down projection's shape
    "one_4_rows_unpaired": [(999, 3584)],               # 250 workgroups: no XCD pairing
    "pair_shared_x": [(3584, 1024), (3584, 1024)],      # two 16-row sub-tiles per workgroup
    "pair_ragged_odd": [(4001, 1000), (4001, 1000)],
    "pair_4_rows": [(512, 1024), (512, 1024)],          # the k / v projections' shape
    "pair_4_rows_odd_split": [(499, 1088), (523, 1088)],  # 125 + 131 groups, paired grid
}


@pytest.mark.parametrize("case", list(ROWS_CASES))
def test_plan_rows_kernel_paths(gpu, torch_mod, case):
    """Plans of one GEMV, or of two reading the same activation, run on the
    16-row kernel, which quantizes the activation itself: odd M adds the
    tail-row kernel (reading the records the launch left), a ragged K uses its
    K / 64 whole blocks, GEMVs with few rows use sub-tiles of 8 or 4 rows (one
    workgroup per CU at most; 4-row sub-tiles sharing a 128-byte line on one
    XCD when the grid is a multiple of 16), and more 16-row workgroups than CUs
    put two sub-tiles in each workgroup (the pairs; the ragged pair ends in a
    half-used one)."""
    qk, torch = gpu, torch_mod
    shapes = ROWS_CASES[case]
    K = shapes[0][1]
    x = qk.synth_normal(K, 5150)
    xd = torch.from_numpy(x).cuda()
    items, refs = [], []
    for j, (M, K) in enumerate(shapes):
        dm = qk.DeviceMatrix.synth(M, K, 5100 + j, 124, 130)
        items.append({"mat": dm, "x": xd, "y": torch.empty(M, dtype=torch.float32, device="cuda")})
        refs.append((M, K, 5100 + j))
    plan = qk.SweepPlan(items)
    assert plan.kernel_name(1) == "rt_rows_gemv_kernel"
    say("rows plan", case)
    for rep in range(2):
        for it in items:
            it["y"].fill_(np.nan)
        plan.run()
        torch.cuda.synchronize()
        for it, (M, K, seed) in zip(items, refs):
            mant, exps = qk.synth_planes(M, K, seed, 124, 130)
            y_ref = ol.gemv_neon(x, mant, exps)[0]
            assert same_f32(it["y"].cpu().numpy(), y_ref), (rep, M, K, mismatch(it["y"].cpu().numpy(), y_ref))
    plan.close()


def _special_blocks(K, seed, inf=False):
    """An activation whose first blocks take every branch of the block
    quantizer (04/qwen_kernels_opt.c:182-205): zeros, negative zeros, a block
    at and one just above the 1e-20 amax threshold, NaN, exact .5 ties,
    subnormals, values of 1e33; then blocks of seven decades.
    With `inf`, block 5 holds an inf (its scale is inf, so y is all inf/NaN)."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(K) * np.float32(10.0) ** rng.integers(-6, 4, size=K)).astype(F32)
    blk = lambda b: slice(64 * b, 64 * b + 64)
    x[blk(0)] = 0.0
    x[blk(1)] = -0.0
    t = np.float32(1e-20)
    x[blk(2)] = rng.uniform(-1, 1, 64).astype(F32) * t
    x[64 * 2] = t                                          # amax == 1e-20: not above, a zero record
    x[blk(3)] = rng.uniform(-1, 1, 64).astype(F32) * t
    x[64 * 3] = np.nextafter(t, np.float32(1.0))           # just above: quantized
    x[64 * 4 + 3] = np.nan
    x[64 * 4 + 40] = np.nan
    if inf:
        x[64 * 5 + 7] = np.inf                             # xscale inf, every other product 0
    x[blk(6)] = (rng.integers(-64, 64, 64) + 0.5).astype(F32)
    x[64 * 6] = 16384.0                                    # q = 1: the .5 values are ties
    x[blk(7)] = (rng.standard_normal(64) * np.float32(1e-39)).astype(F32)
    x[64 * 7 + 9] = 1e-3
    x[blk(8)] = (rng.uniform(-1, 1, 64) * np.float32(3e33)).astype(F32)  # huge amax, y still finite
    return x


@pytest.mark.parametrize("M,K,inf", [(1024, 3584, False), (3584, 1024, False), (1500, 2048, False),
                                     (999, 1000, False), (999, 1000, True)])
def test_rows_kernel_quantizes_special_blocks(gpu, torch_mod, M, K, inf):
    """The 16-row kernel's block quantizer (16 lanes per block, four elements
    per lane) on special blocks, at each sub-tile size, twice in a row."""
    qk, torch = gpu, torch_mod
    x = _special_blocks(K, 6100 + M, inf)
    dm = qk.DeviceMatrix.synth(M, K, 6000 + M, 118, 136)
    y = torch.empty(M, dtype=torch.float32, device="cuda")
    plan = qk.SweepPlan([{"mat": dm, "x": torch.from_numpy(x).cuda(), "y": y}])
    assert plan.kernel_name(1) == "rt_rows_gemv_kernel"
    mant, exps = qk.synth_planes(M, K, 6000 + M, 118, 136)
    y_ref = ol.gemv_neon(x, mant, exps)[0]
    say("rows special blocks", M, K)
    for rep in range(2):
        y.fill_(np.nan)
        plan.run()
        torch.cuda.synchronize()
        assert same_f32(y.cpu().numpy(), y_ref), (rep, mismatch(y.cpu().numpy(), y_ref))
    plan.close()


@pytest.mark.parametrize("shape", ["alone", "alone_65536", "alone_1536_tiles", "alone_ragged_2049_tiles", "alone_k1",
                                   "with_small_gemv", "ragged_2049_tiles", "queue_gemv", "queue_ragged_2049_tiles",
                                   "queue_k1", "queue_small_vocab"])
def test_plan_lm_head_merge_paths(gpu, torch_mod, shape):
    """A plan's lm_head merge runs in the merging workgroup of the single
    launch (with a 2048 x 1024 GEMV: the 2049-tile vocabulary gives some
    workgroups three lm_head tiles, a 64-tile one leaves most workgroups to
    start from the queue, and k = 1), as the stand-alone merge kernel after
    the per-tile lists (a lone lm_head: 256 and 1024 tiles, 1536 in the wide
    form that reads eight passes of list heads, a ragged 2049 tiles, and
    k = 1), or folded into workgroup 0 of the second launch (another GEMV too
    narrow for the single launch, here 128 x 256); a 2049-tile ragged
    vocabulary takes several passes over the list heads.  Later runs use new
    activations written in place: every activation is quantized again (no
    stale records)."""
    qk, torch = gpu, torch_mod
    V, H, k = {"alone": (16384, 1024, 64), "alone_65536": (65536, 1024, 40), "alone_1536_tiles": (98304, 1024, 40),
               "alone_ragged_2049_tiles": (131074, 1024, 40), "alone_k1": (65536, 1024, 1),
               "with_small_gemv": (65536, 1024, 40), "ragged_2049_tiles": (131074, 1024, 40),
               "queue_gemv": (65536, 1024, 40), "queue_ragged_2049_tiles": (131074, 1024, 40),
               "queue_k1": (65536, 1024, 1), "queue_small_vocab": (4096, 512, 64)}[shape]
    say("plan lm_head", shape, V, H, k)
    lm = qk.DeviceMatrix.synth(V, H, 777, 122, 128)
    xl = qk.synth_normal(H, 778)
    items = [{"mat": lm, "x": torch.from_numpy(xl).cuda(), "topk": k}]
    small = None
    if not shape.startswith("alone"):
        small = (128, 256, 779) if not shape.startswith("queue") else (2048, 1024, 779)
        SM, SK, sseed = small
        xs = qk.synth_normal(SK, 780)
        items.append({"mat": qk.DeviceMatrix.synth(SM, SK, sseed, 124, 130), "x": torch.from_numpy(xs).cuda(),
                      "y": torch.empty(SM, dtype=torch.float32, device="cuda")})
    plan = qk.SweepPlan(items)
    if shape.startswith("alone"):  # per-tile lists, then the merge kernel (its wide form past 1024 lists)
        merge = "bfp8_topk_merge_kernel" if V <= 65536 else "bfp8_topk_merge_wide_kernel"
        assert plan.kernel_name(0) == "bfp8_gemv_head_kernel" and plan.kernel_name(1) == merge
    elif shape.startswith("queue"):
        assert plan.kernel_name(0) == "bfp8_sweep_kernel"
    else:
        assert plan.kernel_name(0) == "bfp8_gemv_head_kernel"
    mant, exps = qk.synth_planes(V, H, 777, 122, 128)
    for rep in range(3):
        if rep > 0:  # new activations, same device buffers
            xl = qk.synth_normal(H, 778 + 100 * rep)
            items[0]["x"].copy_(torch.from_numpy(xl))
            if small:
                xs = qk.synth_normal(small[1], 780 + 100 * rep)
                items[1]["x"].copy_(torch.from_numpy(xs))
        y_ref, *_ = ol.gemv_neon(xl, mant, exps)
        ids_ref, sc_ref = ol.topk(y_ref, k)
        plan.run()
        torch.cuda.synchronize()
        ids, sc, cnt = plan.topk_out
        assert int(cnt[0].item()) == k and int(cnt[1].item()) == ol.argmax(y_ref), rep
        assert np.array_equal(ids.cpu().numpy(), ids_ref) and same_f32(sc.cpu().numpy(), sc_ref), rep
        if small:
            sm, se = qk.synth_planes(*small, 124, 130)
            assert same_f32(items[1]["y"].cpu().numpy(), ol.gemv_neon(xs, sm, se)[0]), rep
    plan.close()


@pytest.mark.parametrize("other_k", [0, 2048, 1984])
def test_plan_lm_head_quantizes_special_blocks(gpu, torch_mod, other_k):
    """The launch that streams the lm_head quantizes its activation itself (16
    lanes per block, four elements per lane) and, with another GEMV in the
    plan, that GEMV's activation: in LDS in the single launch (K = 2048), as
    one-block tasks of the two-launch path (K = 1984, whose 31 blocks the
    single launch does not take).  Special blocks in both (zeros, -0, the
    1e-20 threshold, NaN, .5 ties, subnormals, 1e33): top-k, argmax and y
    against the oracle."""
    qk, torch = gpu, torch_mod
    V, H, k = 16384, 1024, 40
    with_other = other_k > 0
    say("plan lm_head special blocks", other_k)
    xl = _special_blocks(H, 6301)
    items = [{"mat": qk.DeviceMatrix.synth(V, H, 6300, 118, 136), "x": torch.from_numpy(xl).cuda(), "topk": k}]
    if with_other:
        xo = _special_blocks(other_k, 6303)
        items.append({"mat": qk.DeviceMatrix.synth(1000, other_k, 6302, 118, 136), "x": torch.from_numpy(xo).cuda(),
                      "y": torch.empty(1000, dtype=torch.float32, device="cuda")})
    plan = qk.SweepPlan(items)
    if with_other:
        assert plan.kernel_name(0) == ("bfp8_sweep_kernel" if other_k == 2048 else "bfp8_gemv_head_kernel")
    mant, exps = qk.synth_planes(V, H, 6300, 118, 136)
    y_ref, *_ = ol.gemv_neon(xl, mant, exps)
    ids_ref, sc_ref = ol.topk(y_ref, k)
    for rep in range(2):
        plan.run()
        torch.cuda.synchronize()
        ids, sc, cnt = plan.topk_out
        assert int(cnt[0].item()) == k and int(cnt[1].item()) == ol.argmax(y_ref), rep
        assert np.array_equal(ids.cpu().numpy(), ids_ref) and same_f32(sc.cpu().numpy(), sc_ref), rep
        if with_other:
            om, oe = qk.synth_planes(1000, other_k, 6302, 118, 136)
            y_o = items[1]["y"].cpu().numpy()
            assert same_f32(y_o, ol.gemv_neon(xo, om, oe)[0]), (rep, mismatch(y_o, ol.gemv_neon(xo, om, oe)[0]))
    plan.close()


# ---- batch and sweep ---------------------------------------------------------------------------------
def _random_cases(seed, n, kmax, k_whole):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.choice([rng.integers(1, 40), rng.integers(40, 1500)]))
        K = int(rng.integers(1, kmax // 64 + 1)) * 64 if (k_whole or i % 2 == 0) else int(rng.integers(1, kmax + 1))
        out.append((M, K, int(rng.integers(0, 2**31))))
    return out


def _random_planes(M, K, seed):
    rng = np.random.default_rng(seed)
    mant = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    exps = rng.integers(0, 256, size=(M, max(K // 64, 0)), dtype=np.uint8)
    x = (rng.standard_normal(K) * np.float32(10.0) ** rng.integers(-4, 3)).astype(F32)
    x[rng.random(K) < 0.02] = 0.0
    return rng, mant, exps, x


def test_random_shapes_against_the_oracle(gpu, torch_mod):
    """24 seeded shapes: 1-1,499 rows (odd and even), K up to 4,096 whole
    blocks or ragged, every exponent byte, mantissa -128 included, activations
    spanning seven decades with zeros: y bit-exact against the NEON-order
    restatement."""
    qk = gpu
    for M, K, seed in _random_cases(4242, 24, 4096, False):
        _, mant, exps, x = _random_planes(M, K, seed)
        say("random gemv", M, K, seed)
        y = qk.Bfp8Kernels().gemv_bfp8(x, mant, exps, M, K)
        y_ref, *_ = ol.gemv_neon(x, mant, exps)
        assert same_f32(y, y_ref), (M, K, seed, mismatch(y, y_ref))


def test_random_batches_against_the_oracle(gpu, torch_mod):
    """Six seeded batched calls: 1-16 vectors, 1-1,499 rows, K whole blocks up
    to 4,096; each vector bit-exact against the restatement."""
    qk = gpu
    for M, K, seed in _random_cases(777, 6, 4096, True):
        rng, mant, exps, _ = _random_planes(M, K, seed)
        B = int(rng.integers(1, 17))
        X = np.stack([_random_planes(1, K, seed + 1 + b)[3] for b in range(B)])
        say("random batch", B, M, K, seed)
        Y = qk.Bfp8Kernels().gemv_batch(X, mant, exps, M, K)
        for b in range(B):
            y_ref, *_ = ol.gemv_neon(X[b], mant, exps)
            assert same_f32(Y[b], y_ref), (B, M, K, seed, b, mismatch(Y[b], y_ref))


@pytest.mark.parametrize("kind", ["any", "queue"])
def test_random_plans_against_the_oracle(gpu, torch_mod, kind):
    """Six seeded plans of 1-10 GEMVs (1-4,999 rows; K whole blocks up to 4,096
    or ragged; some sharing an activation tensor), most with one fused lm_head
    (even vocabularies up to 140,000, hidden 64-1,024, k in 1-64) at a random
    place in the list: every y bit-exact, the top-k and argmax identical, on
    two runs.  "queue": shapes the single launch takes (even M up to 9,998, K
    a multiple of 512, hidden 512 or 1,024), so that the tile queue, its
    LDS quantization and its in-launch merge see random plans."""
    qk, torch = gpu, torch_mod
    rng = np.random.default_rng(31337 if kind == "any" else 4711)
    for p in range(6):
        items, refs = [], []
        for j in range(int(rng.integers(1, 11))):
            if kind == "queue":
                M = int(rng.integers(1, 5000)) * 2
                K = int(rng.integers(1, 9)) * 512
            else:
                M = int(rng.integers(1, 5000))
                K = int(rng.integers(1, 65)) * 64 if rng.random() < 0.8 else int(rng.integers(64, 4097))
            seed = int(rng.integers(0, 2**31))
            if refs and refs[-1][1] == K and rng.random() < 0.5:
                xd, x = items[-1]["x"], refs[-1][3]  # the same activation tensor
            else:
                x = qk.synth_normal(K, seed + 1)
                xd = torch.from_numpy(x).cuda()
            items.append({"mat": qk.DeviceMatrix.synth(M, K, seed, 124, 130), "x": xd,
                          "y": torch.empty(M, dtype=torch.float32, device="cuda")})
            refs.append((M, K, seed, x))
        head = None
        if rng.random() < 0.7:
            V, H, k = int(rng.integers(1, 70001)) * 2, int(rng.integers(1, 17)) * 64, int(rng.integers(1, 65))
            if kind == "queue":
                H = int(rng.choice([512, 1024]))
            seed = int(rng.integers(0, 2**31))
            x = qk.synth_normal(H, seed + 1)
            pos = int(rng.integers(0, len(items) + 1))
            items.insert(pos, {"mat": qk.DeviceMatrix.synth(V, H, seed, 122, 128),
                               "x": torch.from_numpy(x).cuda(), "topk": k})
            head = (V, H, k, seed, x)
        say("random plan", kind, p, [(M, K) for M, K, *_ in refs], head[:3] if head else None)
        plan = qk.SweepPlan(items)
        if kind == "queue" and (head or sum((M + 63) // 64 for M, *_ in refs) > 384):
            assert plan.kernel_name(0) == "bfp8_sweep_kernel", p
        for rep in range(2):
            for it in items:
                if "y" in it:
                    it["y"].fill_(np.nan)
            plan.run()
            torch.cuda.synchronize()
            ys = [it["y"].cpu().numpy() for it in items if "y" in it]
            for y, (M, K, seed, x) in zip(ys, refs):
                mant, exps = qk.synth_planes(M, K, seed, 124, 130)
                y_ref = ol.gemv_neon(x, mant, exps)[0]
                assert same_f32(y, y_ref), (p, rep, M, K, seed, mismatch(y, y_ref))
            if head:
                V, H, k, seed, x = head
                mant, exps = qk.synth_planes(V, H, seed, 122, 128)
                y_ref = ol.gemv_neon(x, mant, exps)[0]
                ids_ref, sc_ref = ol.topk(y_ref, k)
                ids, sc, cnt = plan.topk_out
                n = int(cnt[0].item())
                assert n == ids_ref.size and int(cnt[1].item()) == ol.argmax(y_ref), (p, rep, V, H, k)
                assert np.array_equal(ids.cpu().numpy()[:n], ids_ref), (p, rep, V, H, k)
                assert same_f32(sc.cpu().numpy()[:n], sc_ref), (p, rep, V, H, k)
        plan.close()


@pytest.mark.parametrize("M", [3584, 65536])
def test_batch16_matches_sixteen_single_calls(gpu, torch_mod, M):
    qk, torch = gpu, torch_mod
    K, B = 1024, 16
    mant, exps = qk.synth_planes(M, K, 70 + M, 124, 130)
    X = np.stack([qk.synth_normal(K, 700 + b) for b in range(B)])
    say("batch16", M)
    Y = qk.Bfp8Kernels().gemv_batch(X, mant, exps, M, K)
    for b in range(B):
        y_ref, *_ = ol.gemv_neon(X[b], mant, exps)
        assert same_f32(Y[b], y_ref), (b, mismatch(Y[b], y_ref))


@pytest.mark.parametrize("B,M,K", [(8, 131, 512), (11, 64, 4096), (16, 1000, 1088), (12, 1000, 960), (16, 32769, 960),
                                   (9, 33000, 64), (12, 500, 64), (10, 3, 128)])
def test_batch_scale_edges(gpu, torch_mod, B, M, K):
    """Batches of 8-16 vectors (the matrix-core kernels) whose block scales
    span the float range: every exponent byte 0-255 across rows and blocks,
    vectors scaled by 10^-40 .. 10^35 (subnormal to huge block scales, so that
    2^(e-134) * xscale underflows or overflows for some blocks while the
    reference's two products do not), zero blocks and single huge elements.
    Each vector bit-exact against the restatement.  The last two shapes have
    513 and 516 tiles (the LDS-ring kernel for K <= 1024: an odd last row, a
    last workgroup with idle tile slots, a single block)."""
    qk = gpu
    rng = np.random.default_rng(B * 1000 + M)
    nb = K // 64
    mant = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    exps = ((np.arange(M)[:, None] * 7 + np.arange(nb)[None, :] * 29) % 256).astype(np.uint8)
    X = np.empty((B, K), dtype=F32)
    for b in range(B):
        with np.errstate(over="ignore", under="ignore"):
            X[b] = (rng.standard_normal(K) * 10.0 ** (-40 + 5 * (b % 16))).astype(F32)
        X[b, (b % nb) * 64:(b % nb) * 64 + 64] = 0.0      # a zero block
        X[b, rng.integers(0, K)] = F32(3.0e38) if b % 3 == 0 else F32(-1.0e-42)
    say("batch scale edges", B, M, K)
    Y = qk.Bfp8Kernels().gemv_batch(X, mant, exps, M, K)
    for b in range(B):
        y_ref, *_ = ol.gemv_neon(X[b], mant, exps)
        assert same_f32(Y[b], y_ref), (B, M, K, b, mismatch(Y[b], y_ref))


@pytest.mark.parametrize("B,M,K", [(8, 200, 1000), (16, 1000, 1105), (12, 3584, 4095), (8, 40000, 1000), (13, 301, 1000)])
def test_batch_ragged_k(gpu, torch_mod, B, M, K):
    """Batches of 8-16 vectors (the matrix-core kernel) with K not a multiple
    of 64: the trailing K % 64 elements are dropped, as in the single-vector
    path; each vector bit-exact against the restatement."""
    qk = gpu
    mant, exps = qk.synth_planes(M, K, 90 + B, 124, 130)
    X = np.stack([qk.synth_normal(K, 900 + b) for b in range(B)])
    say("batch ragged K", B, M, K)
    Y = qk.Bfp8Kernels().gemv_batch(X, mant, exps, M, K)
    for b in range(B):
        y_ref, *_ = ol.gemv_neon(X[b], mant, exps)
        assert same_f32(Y[b], y_ref), (B, M, K, b, mismatch(Y[b], y_ref))


def test_batch_odd_sizes(gpu, torch_mod):
    qk = gpu
    M, K, B = 129, 2048, 5
    mant, exps = qk.synth_planes(M, K, 80, 124, 130)
    X = np.stack([qk.synth_normal(K, 800 + b) for b in range(B)])
    say("batch5 odd M")
    Y = qk.Bfp8Kernels().gemv_batch(X, mant, exps, M, K)
    for b in range(B):
        assert same_f32(Y[b], ol.gemv_neon(X[b], mant, exps)[0]), b


@pytest.mark.parametrize("with_head", [True, False])
def test_sweep_plan_24_layers_and_lm_head(gpu, torch_mod, with_head):
    """The full synthetic decode sweep in one plan: 24 x {gate, up, down, in, out}
    plus the fused lm_head (or without it: every tile from the queue), in the
    single launch, every output bit-exact, three runs in a row (the second
    with new activations written in place; the runs take the plan's two
    ticket-counter sets in turn, so the third depends on the second having
    zeroed the first's)."""
    qk, torch = gpu, torch_mod
    shapes = [(3584, 1024), (3584, 1024), (1024, 3584), (6144, 1024), (1024, 2048)]
    items, refs = [], []
    say("sweep plan build")
    for layer in range(24):
        for j, (M, K) in enumerate(shapes):
            seed = 10_000 + layer * 10 + j
            dm = qk.DeviceMatrix.synth(M, K, seed, 124, 130)
            x = qk.synth_swiglu(K, seed + 5) if K == 3584 else qk.synth_normal(K, seed + 5)
            items.append({"mat": dm, "x": torch.from_numpy(x).cuda(),
                          "y": torch.empty(M, dtype=torch.float32, device="cuda")})
            refs.append((M, K, seed, x))
    lm = qk.DeviceMatrix.synth(65536, 1024, 99_999, 122, 128)
    xl = qk.synth_normal(1024, 99_998)
    items.insert(0, {"mat": lm, "x": torch.from_numpy(xl).cuda(), "topk": 40})
    plan = qk.SweepPlan(items if with_head else items[1:])
    assert plan.kernel_name(0) == "bfp8_sweep_kernel"
    for rep in range(3):
        say("sweep plan run", with_head, rep)
        if rep == 1:  # new activations in the same buffers: no record of the last run may be read
            for i, (it, (M, K, seed, x)) in enumerate(zip(items[1:], refs)):
                x = qk.synth_swiglu(K, seed + 7) if K == 3584 else qk.synth_normal(K, seed + 7)
                it["x"].copy_(torch.from_numpy(x))
                refs[i] = (M, K, seed, x)
            xl = qk.synth_normal(1024, 99_997)
            items[0]["x"].copy_(torch.from_numpy(xl))
        for it in items[1:]:
            it["y"].fill_(np.nan)
        plan.run()
        torch.cuda.synchronize()
        for it, (M, K, seed, x) in zip(items[1:], refs):
            mant, exps = qk.synth_planes(M, K, seed, 124, 130)
            y_ref, *_ = ol.gemv_neon(x, mant, exps)
            assert same_f32(it["y"].cpu().numpy(), y_ref), (M, K, seed)
        if not with_head:
            continue
        mant, exps = qk.synth_planes(65536, 1024, 99_999, 122, 128)
        y_ref, *_ = ol.gemv_neon(xl, mant, exps)
        ids, sc, am = plan.topk_result()  # raises on an invalid (count -1) run
        ids_ref, sc_ref = ol.topk(y_ref, 40)
        assert ids.numel() == 40 and am == ol.argmax(y_ref)
        assert np.array_equal(ids.cpu().numpy(), ids_ref) and same_f32(sc.cpu().numpy(), sc_ref)
    plan.close()
