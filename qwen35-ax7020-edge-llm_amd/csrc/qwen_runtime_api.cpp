// qwen_runtime_api.cpp -- C ABI of the decode runtime (include/qwen_kernels.h):
// the reference's rmsnorm ... rmsnorm_gated on host pointers, and its compiled
// forward loop (forward_linear_layer, forward_mlp, forward_token_c) run on
// the GPU with weights, parameters and activations resident in HBM.  All
// arithmetic is in the HIP kernels (runtime_ftz.hip, bfp8_ftz.hip,
// bf16_head.hip); nothing here computes results on the CPU.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "host_internal.h"
#include "runtime_internal.h"

namespace qhost {
namespace {

// ---- host-pointer calls: one arena in, kernels, the same arena out --------------------
// Arguments are packed at 256-byte offsets into a pinned buffer, copied to the
// device in one transfer, and copied back in one transfer after the kernels.
struct HostCall {
    struct Arg {
        void* host;
        size_t bytes, off;
        bool out;
    };
    std::vector<Arg> args;
    size_t total = 0;
    // Registers an argument; returns its offset in the arena.
    size_t add(const void* p, size_t bytes, bool out) {
        const size_t off = total;
        args.push_back(Arg{const_cast<void*>(p), bytes, off, out});
        total += (bytes + 255) & ~(size_t)255;
        return off;
    }
    int upload() {
        int rc;
        if ((rc = g.rt_pin.reserve(total)) || (rc = g.rt_dev.reserve(total))) return rc;
        char* pin = static_cast<char*>(g.rt_pin.p);
        for (const Arg& a : args)
            if (a.bytes) memcpy(pin + a.off, a.host, a.bytes);
        HIP_OK(hipMemcpyAsync(g.rt_dev.p, pin, total, hipMemcpyHostToDevice, g.stream));
        return BFP8_OK;
    }
    template <class T>
    T* dev(size_t off) const {
        return reinterpret_cast<T*>(static_cast<char*>(g.rt_dev.p) + off);
    }
    int download() {
        HIP_OK(hipMemcpyAsync(g.rt_pin.p, g.rt_dev.p, total, hipMemcpyDeviceToHost, g.stream));
        HIP_OK(hipStreamSynchronize(g.stream));
        const char* pin = static_cast<const char*>(g.rt_pin.p);
        for (const Arg& a : args)
            if (a.out && a.bytes) memcpy(a.host, pin + a.off, a.bytes);
        return BFP8_OK;
    }
};

#define RT_CHECK(where, expr)                                                            \
    do {                                                                                 \
        int rc_ = (expr);                                                                \
        if (rc_ != BFP8_OK) fatal(where);                                                \
    } while (0)

#define RT_LAUNCH(expr)                                                                  \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess) {                                                          \
            set_error("%s: %s", #expr, hipGetErrorString(e_));                           \
            return BFP8_EHIP;                                                            \
        }                                                                                \
    } while (0)

// ---- the forward -----------------------------------------------------------------------
constexpr int kHidden = RT_HIDDEN, kConv = RT_CONV_CH, kHD = RT_HEADS * RT_HEAD_DIM, kMlp = 3584;
constexpr int kVocab = 65536, kLayers = 24;

// Device copies of parameters the forward reads (float vectors, bf16 tables,
// writable BFP8 planes), keyed by host address and size, kept until
// bfp8_cache_clear().
struct ParamKey {
    const void* p;
    size_t bytes;
    bool operator<(const ParamKey& o) const { return p != o.p ? p < o.p : bytes < o.bytes; }
};

struct DevState {
    DevBuf conv[2], rec;  // [3][6144] taps (the current one conv[cur]), [16][128*128] blocked state
    int cur = 0;
    float* host_conv;     // the caller's buffers
    float* host_rec;
    bool resident_used = false;  // advanced on the device while resident
    bool dirty = false;          // device copy newer than the caller's buffers
};

// One layer (linear-attention layer or MLP of a full-attention layer).
struct FwdLayer {
    bool linear;
    LinearLayerPlan lp;  // the plan it was built from
    MlpPlan mp;
    // parameters (device)
    const float *in_ln_w = nullptr, *conv_w = nullptr, *wa = nullptr, *wb = nullptr, *nea = nullptr,
                *dt = nullptr, *norm_w = nullptr, *post_ln_w = nullptr;
    DevState* st = nullptr;
    // GPU planes: linear = qkv, z, o, gate, up, down; MLP = gate, up, down
    DevWeights w[6];
};

struct Workspace {
    DevBuf buf;
    float *h, *h2;  // the hidden state ping-pongs between these (see RtRowsArgs::h_out)
    float *normed, *qkv, *z, *zsilu, *attn, *o, *gate, *up, *down;
    int* lm;        // [ids 1, scores 1, count, argmax]; directly after h2
    bool start_h2;  // a token's embedding goes to h2 (see result_out)
};

struct Forward {
    std::map<ParamKey, DevBuf> params;
    std::map<ParamKey, CachedWeights> planes;           // writable BFP8 planes
    std::map<std::vector<char>, std::unique_ptr<FwdLayer>> layers;
    std::map<std::pair<const float*, const float*>, std::unique_ptr<DevState>> states;  // by the caller's buffers
    Workspace ws{};
    bool ws_ready = false;
    int resident = 0;
};

Forward F;

int fwd_param(const void* p, size_t bytes, const void** out) {
    const ParamKey key{p, bytes};
    auto it = F.params.find(key);
    if (it == F.params.end()) {
        DevBuf d;
        int rc;
        if ((rc = d.reserve(bytes))) return rc;
        HIP_OK(hipMemcpy(d.p, p, bytes, hipMemcpyHostToDevice));
        it = F.params.emplace(key, d).first;
    }
    *out = it->second.p;
    return BFP8_OK;
}

template <class T>
int fwd_vec(const T* p, size_t n, const T** out) {
    const void* d;
    int rc = fwd_param(p, n * sizeof(T), &d);
    *out = static_cast<const T*>(d);
    return rc;
}

// GPU-layout planes: the shared read-only cache, else a forward-owned copy.
int fwd_planes(const int8_t* mant, const uint8_t* exps, int M, int K, DevWeights* out) {
    const size_t mb = (size_t)M * K, eb = (size_t)M * bfp8_nblocks(K);
    if (range_readonly_cached(mant, mb) && range_readonly_cached(exps, eb)) return weights_for(mant, exps, M, K, out);
    const ParamKey key{mant, mb};
    auto it = F.planes.find(key);
    if (it == F.planes.end()) {
        int rc;
        if ((rc = g.soa_m.reserve(mb)) || (rc = g.soa_e.reserve(eb))) return rc;
        HIP_OK(hipMemcpyAsync(g.soa_m.p, mant, mb, hipMemcpyHostToDevice, g.stream));
        HIP_OK(hipMemcpyAsync(g.soa_e.p, exps, eb, hipMemcpyHostToDevice, g.stream));
        CachedWeights cw;
        if ((rc = cw.mant.reserve(bfp8_gpu_mant_bytes(M, K))) || (rc = cw.exps.reserve(bfp8_gpu_exps_bytes(M, K))))
            return rc;
        HIP_OK(bfp8_launch_pack(cw.mant.as<uint8_t>(), cw.exps.as<uint8_t>(), g.soa_m.as<int8_t>(),
                                g.soa_e.as<uint8_t>(), M, K, g.stream));
        HIP_OK(hipStreamSynchronize(g.stream));
        it = F.planes.emplace(key, cw).first;
    }
    out->mant = it->second.mant.as<uint8_t>();
    out->exps = it->second.exps.as<uint8_t>();
    return BFP8_OK;
}

int ensure_workspace() {
    if (F.ws_ready) return BFP8_OK;
    Workspace& w = F.ws;
    const int nf[] = {kHidden, kHidden, kHidden, kConv, kHD, kHD, kHD, kHidden, kMlp, kMlp, kHidden};
    size_t total = 256;
    for (int n : nf) total += ((size_t)n * 4 + 255) & ~(size_t)255;
    int rc;
    if ((rc = w.buf.reserve(total))) return rc;
    char* p = w.buf.as<char>();
    auto take = [&](size_t bytes) {
        char* r = p;
        p += (bytes + 255) & ~(size_t)255;
        return r;
    };
    float** fl[] = {&w.h, &w.h2, &w.normed, &w.qkv, &w.z, &w.zsilu, &w.attn, &w.o, &w.gate, &w.up, &w.down};
    for (int i = 0; i < 11; ++i) {
        *fl[i] = reinterpret_cast<float*>(take((size_t)nf[i] * 4));
        if (i == 1) w.lm = reinterpret_cast<int*>(take(16));  // h2 is a multiple of 256 B
    }
    F.ws_ready = true;
    return BFP8_OK;
}

bool linear_shapes_ok(const LinearLayerPlan& p) {
    return p.M_qkv == kConv && p.K_qkv == kHidden && p.M_z == kHD && p.K_z == kHidden && p.M_o == kHidden &&
           p.K_o == kHD && p.M_gate == kMlp && p.K_gate == kHidden && p.M_up == kMlp && p.K_up == kHidden &&
           p.M_down == kHidden && p.K_down == kMlp;
}

bool mlp_shapes_ok(const MlpPlan& p) {
    return p.M_gate == kMlp && p.K_gate == kHidden && p.M_up == kMlp && p.K_up == kHidden && p.M_down == kHidden &&
           p.K_down == kMlp;
}

// Device state of a layer, keyed by the caller's conv-state buffer.  A new
// one starts from the caller's buffers.
int fwd_state(float* conv_s, float* state, DevState** out) {
    const std::pair<const float*, const float*> key{conv_s, state};
    auto it = F.states.find(key);
    if (it != F.states.end()) {
        *out = it->second.get();
        return BFP8_OK;
    }
    std::unique_ptr<DevState> st(new DevState());
    int rc;
    if ((rc = st->conv[0].reserve((size_t)3 * kConv * 4)) || (rc = st->conv[1].reserve((size_t)3 * kConv * 4)) ||
        (rc = st->rec.reserve((size_t)RT_HEADS * RT_HEAD_DIM * RT_HEAD_DIM * 4)))
        return rc;
    st->host_conv = conv_s;
    st->host_rec = state;
    HIP_OK(hipMemcpy(st->conv[0].p, conv_s, (size_t)3 * kConv * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(st->rec.p, state, (size_t)RT_HEADS * RT_HEAD_DIM * RT_HEAD_DIM * 4, hipMemcpyHostToDevice));
    *out = st.get();
    F.states[key] = std::move(st);
    return BFP8_OK;
}

int state_in(DevState* st) {
    HIP_OK(hipMemcpyAsync(st->conv[st->cur].p, st->host_conv, (size_t)3 * kConv * 4, hipMemcpyHostToDevice, g.stream));
    HIP_OK(hipMemcpyAsync(st->rec.p, st->host_rec, (size_t)RT_HEADS * RT_HEAD_DIM * RT_HEAD_DIM * 4,
                          hipMemcpyHostToDevice, g.stream));
    return BFP8_OK;
}

int state_out(DevState* st) {
    HIP_OK(hipMemcpyAsync(st->host_conv, st->conv[st->cur].p, (size_t)3 * kConv * 4, hipMemcpyDeviceToHost, g.stream));
    HIP_OK(hipMemcpyAsync(st->host_rec, st->rec.p, (size_t)RT_HEADS * RT_HEAD_DIM * RT_HEAD_DIM * 4,
                          hipMemcpyDeviceToHost, g.stream));
    return BFP8_OK;
}

std::vector<char> key_of(const void* p, size_t n, char tag) {
    std::vector<char> k(n + 1);
    k[0] = tag;
    memcpy(k.data() + 1, p, n);
    return k;
}

int fwd_linear_layer(const LinearLayerPlan* p, FwdLayer** out) {
    if (!linear_shapes_ok(*p)) {
        set_error("linear-layer plan shapes differ from the model's (qkv %dx%d, z %dx%d, o %dx%d, gate %dx%d, "
                  "up %dx%d, down %dx%d)", p->M_qkv, p->K_qkv, p->M_z, p->K_z, p->M_o, p->K_o, p->M_gate,
                  p->K_gate, p->M_up, p->K_up, p->M_down, p->K_down);
        return BFP8_EINVAL;
    }
    const std::vector<char> key = key_of(p, sizeof *p, 'L');
    auto it = F.layers.find(key);
    if (it != F.layers.end()) {
        *out = it->second.get();
        return BFP8_OK;
    }
    std::unique_ptr<FwdLayer> L(new FwdLayer());
    L->linear = true;
    L->lp = *p;
    int rc;
    const int8_t* m[6] = {p->mant_qkv, p->mant_z, p->mant_o, p->mant_gate, p->mant_up, p->mant_down};
    const uint8_t* e[6] = {p->exp_qkv, p->exp_z, p->exp_o, p->exp_gate, p->exp_up, p->exp_down};
    const int Ms[6] = {p->M_qkv, p->M_z, p->M_o, p->M_gate, p->M_up, p->M_down};
    const int Ks[6] = {p->K_qkv, p->K_z, p->K_o, p->K_gate, p->K_up, p->K_down};
    for (int i = 0; i < 6; ++i)
        if ((rc = fwd_planes(m[i], e[i], Ms[i], Ks[i], &L->w[i]))) return rc;
    if ((rc = fwd_vec(p->in_ln_w, kHidden, &L->in_ln_w)) || (rc = fwd_vec(p->conv_w, (size_t)kConv * 4, &L->conv_w)) ||
        (rc = fwd_vec(p->wa, (size_t)RT_HEADS * kHidden, &L->wa)) ||
        (rc = fwd_vec(p->wb, (size_t)RT_HEADS * kHidden, &L->wb)) || (rc = fwd_vec(p->nea, RT_HEADS, &L->nea)) ||
        (rc = fwd_vec(p->dt, RT_HEADS, &L->dt)) || (rc = fwd_vec(p->norm_w, RT_HEAD_DIM, &L->norm_w)) ||
        (rc = fwd_vec(p->post_ln_w, kHidden, &L->post_ln_w)) || (rc = fwd_state(p->conv_s, p->state, &L->st)))
        return rc;
    *out = L.get();
    F.layers.emplace(key, std::move(L));
    return BFP8_OK;
}

int fwd_mlp_layer(const MlpPlan* p, FwdLayer** out) {
    if (!mlp_shapes_ok(*p)) {
        set_error("MLP plan shapes differ from the model's (gate %dx%d, up %dx%d, down %dx%d)", p->M_gate, p->K_gate,
                  p->M_up, p->K_up, p->M_down, p->K_down);
        return BFP8_EINVAL;
    }
    const std::vector<char> key = key_of(p, sizeof *p, 'M');
    auto it = F.layers.find(key);
    if (it != F.layers.end()) {
        *out = it->second.get();
        return BFP8_OK;
    }
    std::unique_ptr<FwdLayer> L(new FwdLayer());
    L->linear = false;
    L->mp = *p;
    int rc;
    const int8_t* m[3] = {p->mant_gate, p->mant_up, p->mant_down};
    const uint8_t* e[3] = {p->exp_gate, p->exp_up, p->exp_down};
    const int Ms[3] = {p->M_gate, p->M_up, p->M_down};
    const int Ks[3] = {p->K_gate, p->K_up, p->K_down};
    for (int i = 0; i < 3; ++i)
        if ((rc = fwd_planes(m[i], e[i], Ms[i], Ks[i], &L->w[i]))) return rc;
    if ((rc = fwd_vec(p->post_ln_w, kHidden, &L->post_ln_w))) return rc;
    *out = L.get();
    F.layers.emplace(key, std::move(L));
    return BFP8_OK;
}

// Profiled step: while profiling, each step is synchronised and its wall time
// booked to its slot.
struct Step {
    int slot;
    double t0;
    explicit Step(int s) : slot(s), t0(g_prof_on ? now_ms() : 0.0) {}
    int done() {
        if (!g_prof_on) return BFP8_OK;
        HIP_OK(hipStreamSynchronize(g.stream));
        g_prof_ms[slot] += now_ms() - t0;
        return BFP8_OK;
    }
};

RtRowsGemv rows_gemv(const DevWeights& w, float* y, int M) {
    RtRowsGemv r{};
    r.mant = w.mant;
    r.exps = w.exps;
    r.y = y;
    r.M = M;
    r.pair_rows = M & ~1;
    return r;
}

int rows_step(const RtRowsArgs& a) {
    Step s(QP_GEMV);
    RT_LAUNCH(rt_launch_rows(a, g.stream));
    return s.done();
}

// The other buffer of the hidden state's ping-pong.
float* other_h(const float* h) { return h == F.ws.h ? F.ws.h2 : F.ws.h; }

// rmsnorm of *h (after adding res, if any) into y, in place (the final norm).
int norm_step(float* h, const float* res, const float* w, float* y) {
    Step s(QP_RMSNORM);
    RtNormArgs a{};
    a.h = h;
    a.res = res;
    a.w = w;
    a.y = y;
    a.n = kHidden;
    a.eps = 1e-6f;
    RT_LAUNCH(rt_launch_rmsnorm(a, g.stream));
    return s.done();
}

// The MLP half shared by both layer kinds (planes gud = gate, up, down):
// rmsnorm(h + res) -> gate, up in one launch; swiglu -> down in another.
// *h moves to the other buffer when a residual is added.  Leaves the down
// projection in ws.down, not yet added.
int mlp_steps(const FwdLayer& L, const DevWeights* gud, float** h, const float* res) {
    Workspace& w = F.ws;
    RtRowsArgs a{};
    a.g[0] = rows_gemv(gud[0], w.gate, kMlp);
    a.g[1] = rows_gemv(gud[1], w.up, kMlp);
    a.ngemv = 2;
    a.split = kMlp / 16;
    a.K = kHidden;
    a.mode = RT_ROWS_NORM;
    a.h = *h;
    a.res = res;
    a.w = L.post_ln_w;
    a.eps = 1e-6f;
    a.h_out = res ? other_h(*h) : nullptr;
    int rc;
    if ((rc = rows_step(a))) return rc;
    if (res) *h = a.h_out;
    RtRowsArgs d{};
    d.g[0] = rows_gemv(gud[2], w.down, kHidden);
    d.ngemv = 1;
    d.split = kHidden / 16;
    d.K = kMlp;
    d.mode = RT_ROWS_SWIGLU;
    d.gate = w.gate;
    d.up = w.up;
    return rows_step(d);
}

// forward_linear_layer on the device: *h the hidden state, res a pending
// residual to add first (null for none).  Leaves the MLP's down projection in
// ws.down.
int linear_steps(const FwdLayer& L, float** h, const float* res) {
    Workspace& w = F.ws;
    RtRowsArgs a{};
    a.g[0] = rows_gemv(L.w[0], w.qkv, kConv);
    a.g[1] = rows_gemv(L.w[1], w.z, kHD);
    a.ngemv = 2;
    a.split = kConv / 16;
    a.K = kHidden;
    a.mode = RT_ROWS_NORM;
    a.h = *h;
    a.res = res;
    a.w = L.in_ln_w;
    a.eps = 1e-6f;
    a.y_norm = w.normed;
    a.h_out = res ? other_h(*h) : nullptr;
    int rc;
    if ((rc = rows_step(a))) return rc;
    if (res) *h = a.h_out;
    {
        Step s(QP_GDN);
        DevState* st = L.st;
        RtLinearAttnArgs la{};
        la.qkv = w.qkv;
        la.normed = w.normed;
        la.conv_in = st->conv[st->cur].as<float>();
        la.conv_out = st->conv[st->cur ^ 1].as<float>();
        la.conv_w = L.conv_w;
        la.wa = L.wa;
        la.wb = L.wb;
        la.nea = L.nea;
        la.dt = L.dt;
        la.state = st->rec.as<float>();
        la.attn = w.attn;
        la.z = w.z;
        la.zsilu = w.zsilu;
        RT_LAUNCH(rt_launch_linear_attn(la, g.stream));
        st->cur ^= 1;
        if ((rc = s.done())) return rc;
    }
    // the gated RMSNorm runs in the o GEMV's prologue
    RtRowsArgs o{};
    o.g[0] = rows_gemv(L.w[2], w.o, kHidden);
    o.ngemv = 1;
    o.split = kHidden / 16;
    o.K = kHD;
    o.mode = RT_ROWS_GATED;
    o.attn = w.attn;
    o.zsilu = w.zsilu;
    o.w = L.norm_w;
    o.eps = 1e-6f;
    if ((rc = rows_step(o))) return rc;
    return mlp_steps(L, &L.w[3], h, w.o);
}

int layer_steps(const FwdLayer& L, float** h, const float* res) {
    return L.linear ? linear_steps(L, h, res) : mlp_steps(L, &L.w[0], h, res);
}

int add_pending(float* h, const float* res) {
    if (!res) return BFP8_OK;
    Step s(QP_RESID);
    RT_LAUNCH(rt_launch_add_residual(h, res, kHidden, g.stream));
    return s.done();
}

int h_in(float* dev, const float* h) {
    HIP_OK(hipMemcpyAsync(dev, h, (size_t)kHidden * 4, hipMemcpyHostToDevice, g.stream));
    return BFP8_OK;
}

int h_out(float* h, const float* dev) {
    HIP_OK(hipMemcpyAsync(h, dev, (size_t)kHidden * 4, hipMemcpyDeviceToHost, g.stream));
    HIP_OK(hipStreamSynchronize(g.stream));
    return BFP8_OK;
}

// A token's hidden state hd and lm_head result back to the host.  When hd is
// h2 the two are adjacent and come back in one copy through pinned memory;
// otherwise in two, and the next token starts in the other buffer: the layer
// sequence fixes how often the state moves between h and h2, so it then ends
// in h2.
int result_out(float* h, const float* hd, int* out) {
    Workspace& w = F.ws;
    const size_t hb = (size_t)kHidden * 4;
    if (hd == w.h2) {
        if (int rc = g.rt_pin.reserve(hb + 16)) return rc;
        HIP_OK(hipMemcpyAsync(g.rt_pin.p, w.h2, hb + 16, hipMemcpyDeviceToHost, g.stream));
        HIP_OK(hipStreamSynchronize(g.stream));
        memcpy(h, g.rt_pin.p, hb);
        memcpy(out, static_cast<const char*>(g.rt_pin.p) + hb, 16);
        return BFP8_OK;
    }
    w.start_h2 = !w.start_h2;
    HIP_OK(hipMemcpyAsync(out, w.lm, 16, hipMemcpyDeviceToHost, g.stream));
    return h_out(h, hd);
}

// Copies back the device states that resident calls left newer than the
// caller's buffers.
int sync_states_out() {
    for (auto& kv : F.states) {
        DevState* st = kv.second.get();
        if (!st->dirty) continue;
        if (int rc = state_out(st)) return rc;
        st->dirty = false;
    }
    HIP_OK(hipStreamSynchronize(g.stream));
    return BFP8_OK;
}

// A layer's states before a forward call: refreshed from the caller's
// buffers unless resident.
int states_in(const std::vector<FwdLayer*>& layers) {
    for (FwdLayer* L : layers) {
        if (!L->linear) continue;
        if (F.resident) {
            L->st->resident_used = true;
            L->st->dirty = true;
        } else if (int rc = state_in(L->st)) {
            return rc;
        }
    }
    return BFP8_OK;
}

int states_out(const std::vector<FwdLayer*>& layers) {
    if (F.resident) return BFP8_OK;
    for (FwdLayer* L : layers)
        if (L->linear)
            if (int rc = state_out(L->st)) return rc;
    return BFP8_OK;
}

int layer_call(const FwdLayer& L, float* h, int slot) {
    const double t0 = g_prof_on ? now_ms() : 0.0;
    int rc;
    const std::vector<FwdLayer*> one{const_cast<FwdLayer*>(&L)};
    float* hd = F.ws.h;
    if ((rc = h_in(hd, h)) || (rc = states_in(one))) return rc;
    if ((rc = layer_steps(L, &hd, nullptr)) || (rc = add_pending(hd, F.ws.down))) return rc;
    if ((rc = states_out(one))) return rc;
    if ((rc = h_out(h, hd))) return rc;
    if (g_prof_on) g_prof_ms[slot] += now_ms() - t0;
    return BFP8_OK;
}

void drop_forward() {
    F.layers.clear();
    for (auto& kv : F.params) kv.second.release();
    F.params.clear();
    for (auto& kv : F.planes) {
        kv.second.mant.release();
        kv.second.exps.release();
    }
    F.planes.clear();
    for (auto& kv : F.states) {
        kv.second->conv[0].release();
        kv.second->conv[1].release();
        kv.second->rec.release();
    }
    F.states.clear();
}

}  // namespace

// Called by bfp8_cache_clear (lock held).
void forward_cache_clear() { drop_forward(); }

int forward_preload_param(const void* p, size_t bytes) {
    const void* d;
    return fwd_param(p, bytes, &d);
}

}  // namespace qhost

using namespace qhost;

extern "C" {

// ---- reference runtime symbols, host pointers ---------------------------------------------
void rmsnorm(float* y, const float* x, const float* w, int n, float eps) {
    if (n <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("rmsnorm", ensure_init_locked());
    HostCall c;
    const size_t oy = c.add(y, (size_t)n * 4, true), ox = c.add(x, (size_t)n * 4, false),
                 ow = c.add(w, (size_t)n * 4, false);
    RT_CHECK("rmsnorm", c.upload());
    RtNormArgs a{};
    a.h = c.dev<float>(ox);
    a.w = c.dev<float>(ow);
    a.y = c.dev<float>(oy);
    a.n = n;
    a.eps = eps;
    if (rt_launch_rmsnorm(a, g.stream) != hipSuccess) {
        set_error("rmsnorm launch failed");
        fatal("rmsnorm");
    }
    RT_CHECK("rmsnorm", c.download());
}

void swiglu(float* y, const float* gate, const float* up, int n) {
    if (n <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("swiglu", ensure_init_locked());
    HostCall c;
    const size_t oy = c.add(y, (size_t)n * 4, true), og = c.add(gate, (size_t)n * 4, false),
                 ou = c.add(up, (size_t)n * 4, false);
    RT_CHECK("swiglu", c.upload());
    RtSwigluArgs a{};
    a.y = c.dev<float>(oy);
    a.gate = c.dev<float>(og);
    a.up = c.dev<float>(ou);
    a.n = n;
    if (rt_launch_swiglu(a, g.stream) != hipSuccess) {
        set_error("swiglu launch failed");
        fatal("swiglu");
    }
    RT_CHECK("swiglu", c.download());
}

void add_residual(float* x, const float* res, int n) {
    if (n <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("add_residual", ensure_init_locked());
    HostCall c;
    const size_t ox = c.add(x, (size_t)n * 4, true), orr = c.add(res, (size_t)n * 4, false);
    RT_CHECK("add_residual", c.upload());
    if (rt_launch_add_residual(c.dev<float>(ox), c.dev<float>(orr), n, g.stream) != hipSuccess) {
        set_error("add_residual launch failed");
        fatal("add_residual");
    }
    RT_CHECK("add_residual", c.download());
}

void causal_conv1d_update_silu(float* y, const float* x, float* conv_state, const float* weight, int channels) {
    if (channels <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("causal_conv1d_update_silu", ensure_init_locked());
    HostCall c;
    const size_t C = (size_t)channels;
    const size_t oy = c.add(y, C * 4, true), ox = c.add(x, C * 4, false), os = c.add(conv_state, 3 * C * 4, true),
                 ow = c.add(weight, 4 * C * 4, false);
    RT_CHECK("causal_conv1d_update_silu", c.upload());
    RtConvArgs a{};
    a.y = c.dev<float>(oy);
    a.x = c.dev<float>(ox);
    a.state = c.dev<float>(os);
    a.w = c.dev<float>(ow);
    a.channels = channels;
    if (rt_launch_conv1d(a, g.stream) != hipSuccess) {
        set_error("conv1d launch failed");
        fatal("causal_conv1d_update_silu");
    }
    RT_CHECK("causal_conv1d_update_silu", c.download());
}

void qk_l2norm(float* q, float* k, int num_heads, int head_dim) {
    if (num_heads <= 0 || head_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("qk_l2norm", ensure_init_locked());
    HostCall c;
    const size_t n = (size_t)num_heads * head_dim * 4;
    const size_t oq = c.add(q, n, true), ok = c.add(k, n, true);
    RT_CHECK("qk_l2norm", c.upload());
    if (rt_launch_qk_l2norm(c.dev<float>(oq), c.dev<float>(ok), num_heads, head_dim, g.stream) != hipSuccess) {
        set_error("qk_l2norm launch failed");
        fatal("qk_l2norm");
    }
    RT_CHECK("qk_l2norm", c.download());
}

void gdn_gates(float* alpha, float* beta, const float* x, const float* wa, const float* wb, const float* neg_exp_alog,
               const float* dt, int H, int K) {
    if (H <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("gdn_gates", ensure_init_locked());
    HostCall c;
    const size_t kk = (size_t)(K > 0 ? K : 0);
    const size_t oa = c.add(alpha, (size_t)H * 4, true), ob = c.add(beta, (size_t)H * 4, true),
                 ox = c.add(x, kk * 4, false), owa = c.add(wa, (size_t)H * kk * 4, false),
                 owb = c.add(wb, (size_t)H * kk * 4, false), on = c.add(neg_exp_alog, (size_t)H * 4, false),
                 od = c.add(dt, (size_t)H * 4, false);
    RT_CHECK("gdn_gates", c.upload());
    RtGatesArgs a{};
    a.alpha = c.dev<float>(oa);
    a.beta = c.dev<float>(ob);
    a.x = c.dev<float>(ox);
    a.wa = c.dev<float>(owa);
    a.wb = c.dev<float>(owb);
    a.nea = c.dev<float>(on);
    a.dt = c.dev<float>(od);
    a.H = H;
    a.K = (int)kk;
    if (rt_launch_gates(a, g.stream) != hipSuccess) {
        set_error("gdn_gates launch failed");
        fatal("gdn_gates");
    }
    RT_CHECK("gdn_gates", c.download());
}

void gdn_recurrent_step(float* attn_out, float* state, const float* q, const float* k, const float* v,
                        const float* alpha, const float* beta, int num_heads, int head_dim) {
    if (num_heads <= 0 || head_dim <= 0) return;
    if ((head_dim & 3) || head_dim > RT_MAX_HEAD_DIM) {
        set_error("gdn_recurrent_step: head_dim %d is not a multiple of 4 up to %d", head_dim, RT_MAX_HEAD_DIM);
        fatal("gdn_recurrent_step");
    }
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("gdn_recurrent_step", ensure_init_locked());
    HostCall c;
    const size_t H = (size_t)num_heads, D = (size_t)head_dim;
    const size_t oo = c.add(attn_out, H * D * 4, true), os = c.add(state, H * D * D * 4, true),
                 oq = c.add(q, H * D * 4, false), ok = c.add(k, H * D * 4, false), ov = c.add(v, H * D * 4, false),
                 oa = c.add(alpha, H * 4, false), ob = c.add(beta, H * 4, false);
    RT_CHECK("gdn_recurrent_step", c.upload());
    RtGdnArgs a{};
    a.out = c.dev<float>(oo);
    a.state = c.dev<float>(os);
    a.q = c.dev<float>(oq);
    a.k = c.dev<float>(ok);
    a.v = c.dev<float>(ov);
    a.alpha = c.dev<float>(oa);
    a.beta = c.dev<float>(ob);
    a.H = num_heads;
    a.D = head_dim;
    if (rt_launch_gdn_step(a, g.stream) != hipSuccess) {
        set_error("gdn_recurrent_step launch failed");
        fatal("gdn_recurrent_step");
    }
    RT_CHECK("gdn_recurrent_step", c.download());
}

void rmsnorm_gated(float* y, const float* x, const float* z, const float* norm_w, int num_heads, int head_dim,
                   float eps) {
    if (num_heads <= 0 || head_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    RT_CHECK("rmsnorm_gated", ensure_init_locked());
    HostCall c;
    const size_t n = (size_t)num_heads * head_dim * 4;
    const size_t oy = c.add(y, n, true), ox = c.add(x, n, false), oz = c.add(z, n, false),
                 ow = c.add(norm_w, (size_t)head_dim * 4, false);
    RT_CHECK("rmsnorm_gated", c.upload());
    RtGatedArgs a{};
    a.y = c.dev<float>(oy);
    a.x = c.dev<float>(ox);
    a.z = c.dev<float>(oz);
    a.w = c.dev<float>(ow);
    a.H = num_heads;
    a.D = head_dim;
    a.eps = eps;
    if (rt_launch_gated(a, g.stream) != hipSuccess) {
        set_error("rmsnorm_gated launch failed");
        fatal("rmsnorm_gated");
    }
    RT_CHECK("rmsnorm_gated", c.download());
}

// ---- the forward loop ------------------------------------------------------------------------
void forward_linear_layer(const LinearLayerPlan* p, float* h) {
    if (!p || !h) return;
    std::lock_guard<std::mutex> lk(g.mu);
    FwdLayer* L = nullptr;
    RT_CHECK("forward_linear_layer", ensure_init_locked());
    RT_CHECK("forward_linear_layer", ensure_workspace());
    RT_CHECK("forward_linear_layer", fwd_linear_layer(p, &L));
    RT_CHECK("forward_linear_layer", layer_call(*L, h, QP_LINEAR));
}

void forward_mlp(const MlpPlan* p, float* h) {
    if (!p || !h) return;
    std::lock_guard<std::mutex> lk(g.mu);
    FwdLayer* L = nullptr;
    RT_CHECK("forward_mlp", ensure_init_locked());
    RT_CHECK("forward_mlp", ensure_workspace());
    RT_CHECK("forward_mlp", fwd_mlp_layer(p, &L));
    RT_CHECK("forward_mlp", layer_call(*L, h, QP_MLP));
}

int forward_token_c(int token_id, float* h, const LinearLayerPlan* linear_plans, const MlpPlan* mlp_plans,
                    const int* layer_is_full, const float* final_norm_w, const uint16_t* embed_table,
                    FullAttnCallback full_attn_cb, void* py_context) {
    if (!h || !linear_plans || !mlp_plans || !layer_is_full || !final_norm_w || !embed_table) {
        set_error("forward_token_c: null argument");
        fatal("forward_token_c");
    }
    std::unique_lock<std::mutex> lk(g.mu);
    const double t_total = g_prof_on ? now_ms() : 0.0;
    RT_CHECK("forward_token_c", ensure_init_locked());
    RT_CHECK("forward_token_c", ensure_workspace());
    // layers, the table and the final norm (built on first use)
    std::vector<FwdLayer*> layers(kLayers);
    int li = 0;
    for (int l = 0; l < kLayers; ++l) {
        if (layer_is_full[l])
            RT_CHECK("forward_token_c", fwd_mlp_layer(&mlp_plans[l], &layers[l]));
        else
            RT_CHECK("forward_token_c", fwd_linear_layer(&linear_plans[li++], &layers[l]));
    }
    const float* fnorm = nullptr;
    const uint16_t* table = nullptr;
    const size_t tbytes = (size_t)kVocab * kHidden * 2;
    RT_CHECK("forward_token_c", fwd_vec(final_norm_w, kHidden, &fnorm));
    int tiled = 0;  // the cached table's layout
    if (bf16_table_lookup(embed_table, kVocab, kHidden, &table, &tiled)) {
        // cached on an earlier token: no /proc/self/maps scan
    } else if (range_readonly_cached(embed_table, tbytes)) {
        RT_CHECK("forward_token_c", bf16_table_for(embed_table, kVocab, kHidden, &table, &tiled));
    } else {
        RT_CHECK("forward_token_c", fwd_vec(embed_table, (size_t)kVocab * kHidden, &table));
    }
    Workspace& w = F.ws;
    float* hd = w.start_h2 ? w.h2 : w.h;  // the hidden state on the device
    RT_CHECK("forward_token_c", states_in(layers));
    {
        Step s(QP_EMBED);
        int row = token_id % kVocab;
        if (row < 0) row += kVocab;
        if (rt_launch_embed(hd, table, tiled ? bfp8_ntiles(kVocab) : 0, row, kHidden, g.stream) != hipSuccess) {
            set_error("embedding launch failed");
            fatal("forward_token_c");
        }
        RT_CHECK("forward_token_c", s.done());
    }
    const float* pending = nullptr;  // down projection not yet added to h
    for (int l = 0; l < kLayers; ++l) {
        FwdLayer& L = *layers[l];
        const double t_layer = g_prof_on ? now_ms() : 0.0;
        if (layer_is_full[l]) {
            if (full_attn_cb) {
                RT_CHECK("forward_token_c", add_pending(hd, pending));
                pending = nullptr;
                RT_CHECK("forward_token_c", h_out(h, hd));
                const double t_cb = g_prof_on ? now_ms() : 0.0;
                lk.unlock();
                full_attn_cb(l, h, py_context);
                lk.lock();
                if (g_prof_on) g_prof_ms[QP_PYCALLBACK] += now_ms() - t_cb;
                RT_CHECK("forward_token_c", h_in(hd, h));
            }
            RT_CHECK("forward_token_c", layer_steps(L, &hd, pending));
            if (g_prof_on) g_prof_ms[QP_MLP] += now_ms() - t_layer;
        } else {
            RT_CHECK("forward_token_c", layer_steps(L, &hd, pending));
            if (g_prof_on) g_prof_ms[QP_LINEAR] += now_ms() - t_layer;
        }
        pending = w.down;
    }
    RT_CHECK("forward_token_c", norm_step(hd, pending, fnorm, w.normed));
    {
        Step s(QP_LMHEAD);
        RT_CHECK("forward_token_c", bf16_lm_head_dev(w.lm, reinterpret_cast<float*>(w.lm + 1), w.lm + 2, w.lm + 3,
                                                     nullptr, w.normed, table, tiled, kVocab, kHidden, 1, 0,
                                                     g.stream));
        RT_CHECK("forward_token_c", s.done());
    }
    int out[4] = {0, 0, 0, 0};
    RT_CHECK("forward_token_c", states_out(layers));
    RT_CHECK("forward_token_c", result_out(h, hd, out));
    if (g_prof_on) g_prof_ms[QP_TOTAL] += now_ms() - t_total;
    return out[3];
}

int qwen_forward_state_resident(int on) {
    std::lock_guard<std::mutex> lk(g.mu);
    const int prev = F.resident;
    if (prev && !on && g.ready && sync_states_out() != BFP8_OK) fatal("qwen_forward_state_resident");
    F.resident = on ? 1 : 0;
    return prev;
}

void qwen_forward_reset_state(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!g.ready) return;
    for (auto& kv : F.states) {
        DevState* st = kv.second.get();
        // hipMemsetAsync is fine here: this call is never captured in a graph
        if (hipMemsetAsync(st->conv[st->cur].p, 0, st->conv[st->cur].n, g.stream) != hipSuccess ||
            hipMemsetAsync(st->rec.p, 0, st->rec.n, g.stream) != hipSuccess) {
            set_error("state reset failed");
            fatal("qwen_forward_reset_state");
        }
        st->dirty = st->resident_used;
    }
    if (hipStreamSynchronize(g.stream) != hipSuccess) fatal("qwen_forward_reset_state");
}

void qwen_forward_sync_state(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.ready && sync_states_out() != BFP8_OK) fatal("qwen_forward_sync_state");
}

}  // extern "C"
