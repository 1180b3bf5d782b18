"""GPU parity of the decode runtime and the forward loop against the oracle.

The reference's runtime symbols (rmsnorm, swiglu, add_residual,
causal_conv1d_update_silu, qk_l2norm, gdn_gates, gdn_recurrent_step,
rmsnorm_gated) and its forward loop (forward_mlp, forward_linear_layer,
forward_token_c) are called through the C ABI with host pointers, as the
engine calls them (04/qwen_real_engine.py:1090-1170, :1258-1270).

Bit for bit wherever no libm call is involved.  Steps that call expf /
log1pf (gdn_gates, rmsnorm_gated, the scalar tails of swiglu and conv1d) are
compared bit for bit with the oracle in its correctly-rounded libm mode (the
definition the GPU implements) and within 2 ulp of the oracle on the host C
library.  gdn states are held in the reference's blocked layout on the GPU
side and converted for the oracle's logical layout.  NaN compares as NaN."""
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


def same(a, b):
    a = np.asarray(a, dtype=F32).reshape(-1)
    b = np.asarray(b, dtype=F32).reshape(-1)
    return a.shape == b.shape and bool(np.all((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))))


def ulp_gap(a, b):
    """Largest distance in units in the last place (ordered float bits); NaN
    against NaN counts as 0, NaN against a number as 2**32."""
    a = np.asarray(a, dtype=F32).reshape(-1)
    b = np.asarray(b, dtype=F32).reshape(-1)
    if a.size == 0:
        return 0

    def ordered(x):
        u = x.view(np.int32).astype(np.int64)
        return np.where(u < 0, -(u & 0x7FFFFFFF), u)
    gap = np.abs(ordered(a) - ordered(b))
    na, nb = np.isnan(a), np.isnan(b)
    gap = np.where(na & nb, 0, np.where(na | nb, 2 ** 32, gap))
    return int(gap.max())


def ptr(a):
    return a.ctypes.data


def normal(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(F32)


# ---- single kernels ----------------------------------------------------------------------------
def test_rmsnorm_and_add_residual(gpu):
    lib = gpu.load()
    rng = np.random.default_rng(11)
    for n in (1024, 1027, 3, 1, 4097, 9001):
        x, w = normal(rng, n, 3.0), normal(rng, n, 0.1)
        say("rmsnorm", n)
        y = np.empty(n, dtype=F32)
        lib.rmsnorm(ptr(y), ptr(x), ptr(w), n, 1e-6)
        assert same(y, ol.rmsnorm(x, w, 1e-6)), n
        r = normal(rng, n)
        xr = x.copy()
        lib.add_residual(ptr(xr), ptr(r), n)
        assert same(xr, ol.add_residual(x, r)), n
    # zeros (scale 1/sqrt(eps)), eps 0 with a tiny sum of squares, subnormal and huge inputs
    for x, eps in ((np.zeros(1024, F32), 1e-6), (np.full(8, 1e-20, F32), 0.0),
                   (np.full(7, 3e-39, F32), 1e-6), (np.full(1024, 3e18, F32), 1e-6)):
        w = normal(rng, x.size, 0.1)
        y = np.empty_like(x)
        lib.rmsnorm(ptr(y), ptr(x), ptr(w), x.size, eps)
        assert same(y, ol.rmsnorm(x, w, eps)), (x[0], eps)


def test_swiglu_vector_part_and_tail(gpu):
    lib = gpu.load()
    rng = np.random.default_rng(12)
    for n in (3584, 3587, 2):
        g, u = normal(rng, n, 4.0), normal(rng, n)
        if n >= 8:
            g[:8] = [np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-40, -95.0, 120.0]
        say("swiglu", n)
        y = np.empty(n, dtype=F32)
        lib.swiglu(ptr(y), ptr(g), ptr(u), n)
        with ol.cr_libm():
            assert same(y, ol.swiglu(g, u)), n
        want = ol.swiglu(g, u)
        nv = n & ~3
        assert same(y[:nv], want[:nv]) and ulp_gap(y[nv:], want[nv:]) <= 2, n


def test_conv1d_state_update(gpu):
    lib = gpu.load()
    rng = np.random.default_rng(13)
    for C in (6144, 6147, 5):
        st = normal(rng, 3 * C)
        w = normal(rng, 4 * C, 0.5)
        st_gpu = st.copy()
        st_ref = st.copy()
        for step in range(3):
            x = normal(rng, C, 2.0)
            say("conv1d", C, step)
            y = np.empty(C, dtype=F32)
            lib.causal_conv1d_update_silu(ptr(y), ptr(x), ptr(st_gpu), ptr(w), C)
            with ol.cr_libm():
                y_ref, st_ref = ol.conv1d_silu(x, st_ref, w)
            assert same(y, y_ref) and same(st_gpu, st_ref), (C, step)


def test_qk_l2norm(gpu):
    lib = gpu.load()
    rng = np.random.default_rng(14)
    for H, D in ((16, 128), (3, 130), (2, 6), (1, 3)):
        q, k = normal(rng, H * D), normal(rng, H * D)
        if H == 16:
            k[:D] = 0.0  # a zero head: scale 1/sqrt(1e-6)
        say("qk_l2norm", H, D)
        qg, kg = q.copy(), k.copy()
        lib.qk_l2norm(ptr(qg), ptr(kg), H, D)
        qr, kr = ol.qk_l2norm(q, k, H, D)
        assert same(qg, qr) and same(kg, kr), (H, D)


def gate_inputs(rng, H, K):
    return (normal(rng, K), normal(rng, H * K, 0.03).reshape(H, K), normal(rng, H * K, 0.03).reshape(H, K),
            (-rng.uniform(0.2, 3.0, H)).astype(F32), rng.uniform(-2, 2, H).astype(F32))


def test_gdn_gates(gpu):
    lib = gpu.load()
    rng = np.random.default_rng(15)
    for H, K in ((16, 1024), (5, 1026), (3, 2)):
        x, wa, wb, nea, dt = gate_inputs(rng, H, K)
        wa[0] *= 300.0  # softplus far into both tails
        wb[1] *= 300.0
        say("gdn_gates", H, K)
        a = np.empty(H, dtype=F32)
        b = np.empty(H, dtype=F32)
        lib.gdn_gates(ptr(a), ptr(b), ptr(x), ptr(wa), ptr(wb), ptr(nea), ptr(dt), H, K)
        with ol.cr_libm():
            ar, br = ol.gdn_gates(x, wa, wb, nea, dt)
        assert same(a, ar) and same(b, br), (H, K)
        ah, bh = ol.gdn_gates(x, wa, wb, nea, dt)
        assert ulp_gap(a, ah) <= 2 and ulp_gap(b, bh) <= 2, (H, K)


def test_gdn_recurrent_step_blocked_state(gpu):
    """head_dim 128 (columns kept in registers), 64, and 132 (generic path),
    three steps each on an evolving state."""
    lib = gpu.load()
    rng = np.random.default_rng(16)
    for H, D in ((16, 128), (4, 64), (3, 132)):
        S = normal(rng, H * D * D, 0.1).reshape(H, D, D)
        blocked = ol.gdn_state_to_blocked(S, H, D)
        for step in range(3):
            q, k, v = normal(rng, H * D, 0.1), normal(rng, H * D, 0.1), normal(rng, H * D)
            alpha = rng.uniform(0.5, 1.0, H).astype(F32)
            beta = rng.uniform(0.0, 1.0, H).astype(F32)
            say("gdn_step", H, D, step)
            out = np.empty(H * D, dtype=F32)
            lib.gdn_recurrent_step(ptr(out), ptr(blocked), ptr(q), ptr(k), ptr(v), ptr(alpha), ptr(beta), H, D)
            out_ref, S = ol.gdn_step(S, q, k, v, alpha, beta, H, D)
            assert same(out, out_ref), (H, D, step)
            assert same(ol.gdn_state_from_blocked(blocked, H, D), S), (H, D, step)


def test_rmsnorm_gated(gpu):
    lib = gpu.load()
    rng = np.random.default_rng(17)
    for H, D in ((16, 128), (3, 130), (2, 3)):
        x, z, w = normal(rng, H * D), normal(rng, H * D, 3.0), normal(rng, D, 0.5)
        z[:4] = [np.inf, -np.inf, -100.0, 1e-40][:4]
        say("rmsnorm_gated", H, D)
        y = np.empty(H * D, dtype=F32)
        lib.rmsnorm_gated(ptr(y), ptr(x), ptr(z), ptr(w), H, D, 1e-6)
        with ol.cr_libm():
            assert same(y, ol.rmsnorm_gated(x, z, w, H, D, 1e-6)), (H, D)
        assert ulp_gap(y, ol.rmsnorm_gated(x, z, w, H, D, 1e-6)) <= 4, (H, D)


# ---- the forward loop ---------------------------------------------------------------------------
class Model:
    """Synthetic model-shaped weights in the engine's layout: BFP8 planes
    (mantissas [M][K] int8, exponents [M][K/64]) and float parameters.  The
    GEMV weights are shared by every layer of a kind (the forward caches them
    by address either way); states and norms are per layer."""

    SHAPES = {"qkv": (6144, 1024), "z": (2048, 1024), "o": (1024, 2048), "gate": (3584, 1024),
              "up": (3584, 1024), "down": (1024, 3584)}

    def __init__(self, seed, n_layers=24, full=(3, 7, 11, 15, 19, 23), embed=True):
        rng = np.random.default_rng(seed)
        self.keep = []
        self.planes = {}
        for name, (M, K) in self.SHAPES.items():
            m = rng.integers(-127, 128, size=M * K, dtype=np.int8)
            e = rng.integers(122, 127, size=M * (K // 64), dtype=np.uint8)
            self.planes[name] = (m, e, M, K)
        self.is_full = np.array([1 if l in full else 0 for l in range(n_layers)], dtype=np.int32)
        n_lin = int((self.is_full == 0).sum())
        self.gpu_lin = (ol_plan_types()[0] * max(n_lin, 1))()
        self.ref_lin = (ol.LinearPlan * max(n_lin, 1))()
        self.gpu_mlp = (ol_plan_types()[1] * n_layers)()
        self.ref_mlp = (ol.MlpPlan * n_layers)()
        self.gpu_states, self.ref_states = [], []
        li = 0
        for l in range(n_layers):
            post = self._f(normal(rng, 1024, 0.1))
            if self.is_full[l]:
                for plan in (self.gpu_mlp[l], self.ref_mlp[l]):
                    plan.post_ln_w = ptr(post)
                    self._gemvs(plan, ("gate", "up", "down"))
                continue
            in_ln, norm_w = self._f(normal(rng, 1024, 0.1)), self._f(normal(rng, 128, 0.5))
            conv_w = self._f(normal(rng, 6144 * 4, 0.5))
            wa, wb = self._f(normal(rng, 16 * 1024, 0.03)), self._f(normal(rng, 16 * 1024, 0.03))
            nea = self._f((-rng.uniform(0.2, 3.0, 16)).astype(F32))
            dt = self._f(rng.uniform(-2, 2, 16).astype(F32))
            conv0 = normal(rng, 3 * 6144, 0.5)
            S0 = normal(rng, 16 * 128 * 128, 0.05).reshape(16, 128, 128)
            gst = (self._f(conv0.copy()), self._f(ol.gdn_state_to_blocked(S0, 16, 128)))
            rst = (self._f(conv0.copy()), self._f(S0.reshape(-1).copy()))
            self.gpu_states.append(gst)
            self.ref_states.append(rst)
            for plan, (cs, rs) in ((self.gpu_lin[li], gst), (self.ref_lin[li], rst)):
                plan.in_ln_w, plan.conv_w, plan.conv_s = ptr(in_ln), ptr(conv_w), ptr(cs)
                plan.wa, plan.wb, plan.nea, plan.dt, plan.state = ptr(wa), ptr(wb), ptr(nea), ptr(dt), ptr(rs)
                plan.norm_w, plan.post_ln_w = ptr(norm_w), ptr(post)
                self._gemvs(plan, ("qkv", "z", "o", "gate", "up", "down"))
            li += 1
        self.final_w = self._f(normal(rng, 1024, 0.1))
        if embed:
            self.embed = ol.f32_to_bf16_bits(normal(rng, 65536 * 1024, 0.05)).reshape(65536, 1024)

    def _f(self, a):
        a = np.ascontiguousarray(a, dtype=F32)
        self.keep.append(a)
        return a

    def _gemvs(self, plan, names):
        for name in names:
            m, e, M, K = self.planes[name]
            setattr(plan, "mant_" + name, ptr(m))
            setattr(plan, "exp_" + name, ptr(e))
            setattr(plan, "M_" + name, M)
            setattr(plan, "K_" + name, K)

    def states_match(self, n=None):
        return states_match(self.gpu_states[:n], self.ref_states[:n])


def states_match(gpu_states, ref_states):
    for (gc, gs), (rc, rs) in zip(gpu_states, ref_states):
        if not (same(gc, rc) and same(ol.gdn_state_from_blocked(gs, 16, 128), rs.reshape(16, 128, 128))):
            return False
    return True


def ol_plan_types():
    import qwen_kernels_gpu as qk
    return qk.LinearLayerPlan, qk.MlpPlan


@pytest.fixture(scope="module")
def model(gpu):
    m = Model(2025)
    yield m
    # the forward's caches are keyed by host addresses: drop them with the buffers
    gpu.load().bfp8_cache_clear()


@pytest.fixture
def fresh_cache(gpu):
    """Drops the forward's device copies after a test that frees its model."""
    yield
    gpu.load().bfp8_cache_clear()


def test_plan_struct_layouts(gpu):
    assert ctypes.sizeof(gpu.LinearLayerPlan) == ctypes.sizeof(ol.LinearPlan) == 224
    assert ctypes.sizeof(gpu.MlpPlan) == ctypes.sizeof(ol.MlpPlan) == 80


def test_forward_mlp_bit_exact(gpu, model):
    lib = gpu.load()
    rng = np.random.default_rng(21)
    l = int(np.nonzero(model.is_full)[0][0])
    h0 = normal(rng, 1024, 2.0)
    h = h0.copy()
    want = h0.copy()
    for step in range(2):
        say("forward_mlp", step)
        lib.forward_mlp(ctypes.addressof(model.gpu_mlp[l]), ptr(h))
        want = ol.forward_mlp(model.ref_mlp[l], want)
        assert same(h, want), step


def test_forward_linear_layer_bit_exact(gpu, model):
    lib = gpu.load()
    rng = np.random.default_rng(22)
    h = normal(rng, 1024, 2.0)
    want = h.copy()
    with ol.cr_libm():
        for step in range(3):
            say("forward_linear_layer", step)
            lib.forward_linear_layer(ctypes.addressof(model.gpu_lin[0]), ptr(h))
            want = ol.forward_linear_layer(model.ref_lin[0], want)
            assert same(h, want), step
            gc, gs = model.gpu_states[0]
            rc, rs = model.ref_states[0]
            assert same(gc, rc) and same(ol.gdn_state_from_blocked(gs, 16, 128), rs.reshape(16, 128, 128)), step


def test_forward_linear_layer_exact_fallbacks(gpu, fresh_cache):
    """Inputs that send the fused kernels' scalar chains to their exact paths
    (the float fast path applies only to normal operands and results): head 0's
    z rows are zero (silu(0), gated products of zero), head 1's k is zero (its
    L2 scale of a zero sum), heads 2 and 3 have zero gate rows (softplus and
    sigmoid of 0), dt of head 4 is zero, h holds zeros and subnormals, and a
    second step runs on h = 0 (the rms scale of a zero sum, all-zero blocks).
    Bit-exact against the oracle with correctly rounded libm."""
    lib = gpu.load()
    lib.bfp8_cache_clear()
    m = Model(2027, n_layers=1, full=(), embed=False)
    by_addr = {a.ctypes.data: a for a in m.keep}
    plan = m.gpu_lin[0]
    mz, _, _, _ = m.planes["z"]
    mz.reshape(2048, 1024)[0:128] = 0
    mq, _, _, _ = m.planes["qkv"]
    kch = slice(2048 + 128, 2048 + 256)  # head 1's k channels
    mq.reshape(6144, 1024)[kch] = 0
    for conv in (m.gpu_states[0][0], m.ref_states[0][0]):
        conv.reshape(3, 6144)[:, kch] = 0
    by_addr[plan.wa].reshape(16, 1024)[2] = 0
    by_addr[plan.wb].reshape(16, 1024)[3] = 0
    by_addr[plan.dt][4] = 0
    rng = np.random.default_rng(23)
    h = normal(rng, 1024, 2.0)
    h[:64] = 0
    h[64:72] = np.float32(1e-40)
    want = h.copy()
    with ol.cr_libm():
        for step in range(2):
            if step == 1:
                h[:] = 0
                want[:] = 0
            say("forward_linear_layer fallbacks", step)
            lib.forward_linear_layer(ctypes.addressof(plan), ptr(h))
            want = ol.forward_linear_layer(m.ref_lin[0], want)
            assert same(h, want), (step, np.nonzero(h.view(np.uint32) != want.view(np.uint32))[0][:8])
            assert m.states_match(), step


def test_forward_token_c_with_callback(gpu, fresh_cache, tmp_path):
    """24 layers (18 linear-attention, 6 full-attention whose attention is a
    host callback that edits h), final norm, bf16 lm_head argmax; four tokens,
    states carried over, the last two with the table read-only (cached in the
    tile layout); the library is re-entered from the callback."""
    lib = gpu.load()
    m = Model(2026)
    seen = []

    def cb_body(layer, hp, ctx):
        h = np.ctypeslib.as_array(ctypes.cast(hp, ctypes.POINTER(ctypes.c_float)), shape=(1024,))
        seen.append(layer)
        h += np.float32(0.01 * (layer + 1))
        h[layer] = np.float32(-1.5)

    def gpu_cb(layer, hp, ctx):
        cb_body(layer, hp, ctx)
        x = np.ones(1024, dtype=F32)
        lib.add_residual(ptr(x), hp, 1024)  # re-entry while the forward is suspended

    cb_gpu = gpu.FULL_ATTN_CALLBACK(gpu_cb)
    cb_ref = gpu.FULL_ATTN_CALLBACK(cb_body)
    rt = ol._rt()
    rt.orc_forward_token.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, gpu.FULL_ATTN_CALLBACK,
                                     ctypes.c_void_p, ctypes.c_int]
    # a read-only mapping of the table (the engine's PROT_READ image) is
    # cached in the lm_head's tile layout, so the embedding row is read
    # from that layout too
    m.embed.tofile(tmp_path / "embed.bin")
    with open(tmp_path / "embed.bin", "rb") as f:
        ro = np.frombuffer(mmap.mmap(f.fileno(), 0, prot=mmap.PROT_READ), dtype=np.uint16)
    with ol.cr_libm():
        for token, table in ((1234, m.embed), (70001, m.embed), (65535, ro), (40000, ro)):
            say("forward_token_c", token, "read-only table" if table is ro else "")
            h = np.zeros(1024, dtype=F32)
            got = lib.forward_token_c(token, ptr(h), ctypes.addressof(m.gpu_lin), ctypes.addressof(m.gpu_mlp),
                                      ptr(m.is_full), ptr(m.final_w), ptr(table), cb_gpu, None)
            h_ref = np.zeros(1024, dtype=F32)
            want = rt.orc_forward_token(token, ptr(h_ref), ctypes.addressof(m.ref_lin), ctypes.addressof(m.ref_mlp),
                                        ptr(m.is_full), ptr(m.final_w), ptr(table), cb_ref, None, 65536)
            assert got == want, token
            assert same(h, h_ref), token
            assert m.states_match(), token
    assert seen == [3, 7, 11, 15, 19, 23] * 8


def test_forward_state_resident_mode(gpu, fresh_cache):
    """Device-resident states: the caller's buffers are left alone until
    qwen_forward_sync_state; reset zeroes the device states."""
    lib = gpu.load()
    m = Model(2027, embed=False)
    rng = np.random.default_rng(23)
    prev = lib.qwen_forward_state_resident(1)
    try:
        h = normal(rng, 1024)
        want = h.copy()
        before = [(c.copy(), s.copy()) for c, s in m.gpu_states[:1]]
        with ol.cr_libm():
            for step in range(2):
                say("resident", step)
                lib.forward_linear_layer(ctypes.addressof(m.gpu_lin[0]), ptr(h))
                want = ol.forward_linear_layer(m.ref_lin[0], want)
                assert same(h, want), step
        gc, gs = m.gpu_states[0]
        assert same(gc, before[0][0]) and same(gs, before[0][1])  # untouched while resident
        lib.qwen_forward_sync_state()
        assert m.states_match(1)
        lib.qwen_forward_reset_state()
        lib.qwen_forward_sync_state()
        assert not gc.any() and not gs.any()
    finally:
        lib.qwen_forward_state_resident(prev)


def test_profiler_slots(gpu, model):
    lib = gpu.load()
    assert lib.qwen_prof_count() == 15
    names = [lib.qwen_prof_name(i).decode() for i in range(15)]
    assert names[0] == "bfp8_gemv" and names[2] == "gdn_recurrent_step" and names[14] == "forward_token_c"
    lib.qwen_prof_reset()
    lib.qwen_prof_enable(1)
    try:
        h = np.ones(1024, dtype=F32)
        lib.forward_linear_layer(ctypes.addressof(model.gpu_lin[1]), ptr(h))
    finally:
        lib.qwen_prof_enable(0)
    t = [lib.qwen_prof_get(i) for i in range(15)]
    # norms and swiglu run inside the GEMV launches (booked to bfp8_gemv)
    assert t[0] > 0 and t[2] > 0 and t[12] > 0 and t[14] == 0
