// sweep.hip -- a plan of many BFP8 GEMVs (and at most one fused lm_head with
// its top-k) in ONE persistent launch on gfx950.
//
// Compiled with -fgpu-flush-denormals-to-zero -ffp-contract=off, like
// bfp8_ftz.hip: the per-block epilogue is the reference's Advanced SIMD one,
//   fs_q = fs_q + ((float(S_q) * 2^(e-134)) * xscale_b)   (block order),
//   y    = (fs_0 + fs_2) + (fs_1 + fs_3)                  (04/qwen_kernels_opt.c:226-277),
// and the activation quantizer is quant_x_blocks' (04/qwen_kernels_opt.c:177-205).
//
// Work: units of one 64-row tile of one GEMV.  A workgroup has five
// wavefronts.  Four stream: wavefront q computes residue lane q of the unit's
// 64 rows (lane = row), one non-temporal 16-byte load per lane and block (1 KiB
// contiguous per wavefront, 4 KiB per workgroup), two 4-block chunks always in
// flight, across unit boundaries too; a unit ends with its four partial sums
// in LDS and one barrier.  The fifth is the control wavefront: it finds out
// which unit the workgroup takes next, publishes the unit's planes in LDS,
// loads and quantizes its activation into LDS (16 lanes per 64-element
// block), one unit ahead of the stream, and finishes each unit after its
// barrier (the GEMV's y, or the lm_head tile's ranked top-k list).  So a
// streaming wavefront issues nothing but its weight loads: its vector memory
// operations complete in issue order, and a slow ticket, activation or store
// issued between two weight chunks would hold up the second one.
//
//   * Which unit a workgroup takes next is dynamic: after its static units
//     (the lm_head's tiles, dealt round robin over every workgroup but the
//     merging one -- or, without an lm_head, queue unit w) the control
//     wavefront takes tickets from a device counter, so that the workgroups
//     the memory system serves faster take more units and all end together.
//     The queue holds the GEMVs' tiles GEMV by GEMV, the GEMVs with the most
//     blocks first, and is split into nqueues interleaved sub-queues (units
//     s, s + nqueues, ...), each with its own counter (4 KiB apart), taken by
//     the workgroups w with (w / 8) mod nqueues = s.  One counter for all
//     workgroups served about one ticket per 0.1 us.  Workgroups are
//     dispatched to the 8 XCDs in turn, so each sub-queue is shared by
//     workgroups of every XCD and of several dispatch slots of a CU: the
//     memory system serves XCDs and slots at different rates, and sub-queues
//     tied to one XCD ended up to 15 us apart.  A plan's launches take two
//     counter sets in turn: a launch starts with its set at zero and zeroes
//     the other (the previous launch's, which ended before it began) for the
//     next, so no workgroup waits at its end for a count of finished ones.
//   * The lm_head's tiles publish their top-k lists as epoch-tagged keys
//     (topk_merge.h: one agent-scope atomic 64-bit store per key) and the last
//     workgroup of the grid only merges them, from the start of the launch:
//     it re-reads (bounded) any key that does not yet carry the launch's
//     epoch, so it reads each list as soon as it is published.
#include <float.h>

#include <algorithm>
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "gemv_dev.h"
#include "quant_block.h"
#include "topk_merge.h"
#include "wave_topk.h"

namespace {

constexpr int kStreamWaves = 4;
constexpr int kThreads = (kStreamWaves + 1) * 64;  // + the control wavefront
constexpr int kChunk = 4;                           // blocks per chunk (one exponent word)
constexpr int kMaxNb = 64;                          // K <= 4096
constexpr int kXPasses = kMaxNb / 4;                // 1 KiB activation loads per control wavefront
// The control wavefront's activation staging (kMaxNb * 256 bytes) is dynamic
// LDS: with it in the static size the compiler takes LDS as what limits
// occupancy and raises the kernel's VGPR allocation to ~100 (4 wavefronts
// per SIMD), and a CU then holds two of these workgroups, not three.
constexpr int kXinBytes = kMaxNb * 256;
constexpr int kTabWords = sizeof(Bfp8SweepGemv) / 4;
constexpr int kTabLoads = BFP8_SWEEP_MAX_GEMV * kTabWords / 256;           // 1 KiB table loads
constexpr int kDescSpin = 1 << 22;                  // polls of a published unit before a wavefront gives up
static_assert(sizeof(Bfp8SweepGemv) == 48, "table entry");
static_assert(kTabLoads * 256 == BFP8_SWEEP_MAX_GEMV * kTabWords, "the table is whole 1 KiB loads");
static_assert(BFP8_SWEEP_MIN_NB % (2 * kChunk) == 0, "units have an even number of chunks");

struct Chunk {
    u32x4 w[kChunk];
    uint32_t e;
};

struct Unit {  // wave-uniform
    uint64_t mant, exps;  // the tile's planes
    uint64_t x;           // the activation
    uint64_t y;           // outputs (0: the lm_head)
    int nb, tile, rows;
    int valid, head;
};

// A unit as the control wavefront publishes it for the streaming ones: the
// workgroup's unit number seq - 1 (the streaming wavefronts wait for seq).
struct UnitDesc {
    uint32_t w[6];  // mant, exps (two words each), nb, valid
    uint32_t seq;
    uint32_t pad_;
};

struct SweepLds {
    uint32_t split[2][kMaxNb * 32];  // quantized activations (bfp8_layout.h split records), by unit parity
    float scale[2][kMaxNb];
    uint32_t tab[BFP8_SWEEP_MAX_GEMV * kTabWords];  // Bfp8SweepGemv table (control wavefront)
    UnitDesc desc[2];                // published units, by unit parity
    uint32_t xready;                 // j + 1: unit j's activation is in xin
    float red[2][256];               // the streaming wavefronts' partial sums, by unit parity
    uint64_t keys[64];               // the lm_head tile's rank keys (control wavefront)
    MergeLds<kStreamWaves> merge;    // the merging workgroup
};

// ---- memory operations ------------------------------------------------------------------------
// Buffer loads over [base, base + bytes): 0 bytes make every access out of
// range, so nothing is read and the result is 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(uint64_t base, uint32_t bytes) {
    return make_rsrc(reinterpret_cast<const void*>(base), bytes);
}

// 1 KiB from global memory straight into LDS: lane l's 16 bytes at byte
// offset voff of the buffer land at lds + 16 l.  No registers hold the data;
// the wavefront's vector memory count covers the write to LDS.
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t* lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, 0, 0, 0);
}

// vmcnt(0): every load of the wavefront is in, the LDS ones too; LDS is
// read only after it.
__device__ __forceinline__ void wait_vm_all() {
    __builtin_amdgcn_s_waitcnt(0x0F70);
    asm volatile("" ::: "memory");
}

// Chunk k of unit u (an invalid unit: an empty range).  Every chunk is the
// same five loads, issued unconditionally and kept in place (the compiler
// would otherwise sink the exponent load past the next chunk's loads, or
// hoist the previous chunk's arithmetic above them), so that the compiler's
// wait before a chunk's first use counts exactly the loads issued after it.
__device__ __forceinline__ void issue_chunk(Chunk& c, const Unit& u, int k, uint32_t vw, uint32_t ve) {
    const uint32_t wb = u.valid ? (uint32_t)u.nb * 4096u : 0u;
    const uint32_t eb = u.valid ? (uint32_t)(u.nb >> 2) * 256u : 0u;
    const __amdgpu_buffer_rsrc_t wr = rsrc(u.mant, wb), er = rsrc(u.exps, eb);
    const int s0 = k * (kChunk * 4096);
    c.e = load_e(er, (int)ve, k * 256);
#pragma unroll
    for (int b = 0; b < kChunk; ++b) c.w[b] = load_w(wr, (int)vw, s0 + b * 4096);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// ---- arithmetic --------------------------------------------------------------------------------
// fs is computed here: the compiler would otherwise sink a chunk's
// arithmetic past a following wait (an awaited unit), keeping its LDS
// operands live in ~70 more VGPRs.
__device__ __forceinline__ void computed(float& fs) { asm volatile("" : "+v"(fs)); }

__device__ __forceinline__ float epilogue(float fs, int S, uint32_t e, float xs) {
    const float t1 = (float)S * exp_scale_ftz(e);
    const float t2 = t1 * xs;
    return fs + t2;
}

// Chunk k of a unit: blocks 4k .. 4k + 3 in order (every unit has whole
// chunks), its activation in split / scale.  One block at a time, its LDS
// reads included (the compiler would otherwise interleave blocks or read
// ahead, up to ~150 VGPRs: fewer workgroups fit a CU, sweep_residency below).
__device__ __forceinline__ float reduce_chunk(float fs, const Chunk& c, int k, int q, const uint32_t* split,
                                              const float* scale) {
    const float4 sc = *reinterpret_cast<const float4*>(&scale[4 * k]);
    const float xs[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
        const int b = 4 * k + u;
        const uint4 h = *reinterpret_cast<const uint4*>(&split[b * 32 + q * 8]);
        const uint4 l = *reinterpret_cast<const uint4*>(&split[b * 32 + q * 8 + 4]);
        const u32x4 w = c.w[u];
        int S = __builtin_amdgcn_sdot4((int)w.x, (int)h.x, 0, false);
        S = __builtin_amdgcn_sdot4((int)w.y, (int)h.y, S, false);
        S = __builtin_amdgcn_sdot4((int)w.z, (int)h.z, S, false);
        S = __builtin_amdgcn_sdot4((int)w.w, (int)h.w, S, false);
        S = (int)((uint32_t)S << 8);
        S = __builtin_amdgcn_sdot4((int)w.x, (int)l.x, S, false);
        S = __builtin_amdgcn_sdot4((int)w.y, (int)l.y, S, false);
        S = __builtin_amdgcn_sdot4((int)w.z, (int)l.z, S, false);
        S = __builtin_amdgcn_sdot4((int)w.w, (int)l.w, S, false);
        fs = epilogue(fs, S, (c.e >> (8 * u)) & 0xffu, xs[u]);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
    return fs;
}

// ---- the workgroup's units ---------------------------------------------------------------------
struct Ctx {  // wave-uniform, fixed for the launch
    int wg, nwg, lane;
    int ns;            // static units of this workgroup
    int hnwg;          // workgroups that stream lm_head tiles (all but the merging one)
    int ngemv, nunits, ticket0;
    int sub, nqueues;  // this workgroup's sub-queue ((w / 8) mod nqueues), their number
    uint32_t* ctr;     // the sub-queue's counter
    uint64_t head_mant, head_exps, head_x;
    int head_nb, head_ntiles, head_rows, topk;
    uint64_t* partials;
    uint32_t epoch;
};

__device__ __forceinline__ Unit no_unit() {
    Unit U;
    U.mant = U.exps = U.x = U.y = 0;
    U.nb = U.tile = U.rows = 0;
    U.valid = U.head = 0;
    return U;
}

// Static unit j of this workgroup that is an lm_head tile.
__device__ __forceinline__ Unit head_unit(const Ctx& C, int j) {
    Unit U;
    U.tile = C.wg + j * C.hnwg;
    U.nb = C.head_nb;
    U.mant = C.head_mant + (uint64_t)U.tile * (uint64_t)U.nb * 4096u;
    U.exps = C.head_exps + (uint64_t)U.tile * (uint64_t)(U.nb >> 2) * 256u;
    U.x = C.head_x;
    U.y = 0;
    U.rows = C.head_rows;
    U.head = 1;
    U.valid = 1;
    return U;
}

__device__ __forceinline__ uint32_t tab_word(const SweepLds& L, int i) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)L.tab[i]);
}

// Queue unit u (0 <= u < nunits): its GEMV is the last whose first unit is <= u
// (the table is ordered by first unit, up to 128 entries).
__device__ __forceinline__ Unit queue_unit(const Ctx& C, const SweepLds& L, int u) {
    const int l = C.lane;
    constexpr int kFirst = offsetof(Bfp8SweepGemv, first) / 4;
    const bool p0 = l < C.ngemv && (int)L.tab[l * kTabWords + kFirst] <= u;
    const bool p1 = l + 64 < C.ngemv && (int)L.tab[(l + 64) * kTabWords + kFirst] <= u;
    const uint64_t m0 = __builtin_amdgcn_ballot_w64(p0), m1 = __builtin_amdgcn_ballot_w64(p1);
    const int g = m1 ? 127 - __builtin_clzll(m1) : (m0 ? 63 - __builtin_clzll(m0) : 0);
    const int o = g * kTabWords;
    Unit U;
    const uint64_t mant = (uint64_t)tab_word(L, o) | ((uint64_t)tab_word(L, o + 1) << 32);
    const uint64_t exps = (uint64_t)tab_word(L, o + 2) | ((uint64_t)tab_word(L, o + 3) << 32);
    U.x = (uint64_t)tab_word(L, o + 4) | ((uint64_t)tab_word(L, o + 5) << 32);
    U.y = (uint64_t)tab_word(L, o + 6) | ((uint64_t)tab_word(L, o + 7) << 32);
    U.nb = (int)tab_word(L, o + 8);
    U.rows = (int)tab_word(L, o + 9);
    const int first = (int)tab_word(L, o + 10), ntiles = (int)tab_word(L, o + 11);
    U.tile = min(max(u - first, 0), max(ntiles - 1, 0));
    U.mant = mant + (uint64_t)U.tile * (uint64_t)U.nb * 4096u;
    U.exps = exps + (uint64_t)U.tile * (uint64_t)(U.nb >> 2) * 256u;
    U.head = 0;
    U.valid = 1;
    return U;
}

// The workgroup's unit number j, in two steps so that other work can
// overlap the ticket: take() issues the ticket (lane 0, only past the static
// units), resolve() waits for it and forms the unit.
__device__ __forceinline__ uint32_t take(const Ctx& C, int j) {
    uint32_t t = 0;
    if (j >= C.ns && C.lane == 0) t = __hip_atomic_fetch_add(C.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return t;
}

__device__ __forceinline__ Unit resolve(const Ctx& C, const SweepLds& L, int j, uint32_t t) {
    if (j < C.ns) return C.head_ntiles > 0 ? head_unit(C, j) : queue_unit(C, L, C.wg);
    t = (uint32_t)__builtin_amdgcn_readlane((int)t, 0);
    const uint32_t u = (uint32_t)(C.ticket0 + C.sub) + (uint32_t)C.nqueues * t;
    return u < (uint32_t)C.nunits ? queue_unit(C, L, (int)u) : no_unit();
}

// The control wavefront publishes unit j: the fields, then, after a
// workgroup-scope release, the sequence word the streaming wavefronts wait
// for.
__device__ __forceinline__ void publish(SweepLds& L, int j, const Unit& U, int lane) {
    UnitDesc& d = L.desc[j & 1];
    if (lane == 0) {
        d.w[0] = (uint32_t)U.mant;
        d.w[1] = (uint32_t)(U.mant >> 32);
        d.w[2] = (uint32_t)U.exps;
        d.w[3] = (uint32_t)(U.exps >> 32);
        d.w[4] = (uint32_t)U.nb;
        d.w[5] = (uint32_t)U.valid;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_store(&d.seq, (uint32_t)(j + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A streaming wavefront waits for unit j (normally published long before it
// is needed) and reads it.  An unpublished unit after the bounded wait reads
// as no unit.
__device__ __forceinline__ Unit await_unit(const SweepLds& L, int j) {
    const UnitDesc& d = L.desc[j & 1];
    bool ok = false;
    for (int i = 0; i < kDescSpin; ++i) {
        const uint32_t s = __hip_atomic_load(&d.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (__builtin_amdgcn_readfirstlane((int)s) == j + 1) {
            ok = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    uint32_t w[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) w[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)d.w[i]);
    Unit U = no_unit();
    U.mant = (uint64_t)w[0] | ((uint64_t)w[1] << 32);
    U.exps = (uint64_t)w[2] | ((uint64_t)w[3] << 32);
    U.nb = (int)w[4];
    U.valid = ok ? (int)(w[5] & 1u) : 0;
    return U;
}

// The control wavefront loads a unit's activation into LDS (xin, dynamic),
// and the streaming wavefronts quantize it into split / scale: in pass p,
// row k of a wavefront (16 lanes) quantizes block 4 p + k from its lanes'
// four elements each.  Every pass's 1 KiB goes out at once, straight to LDS
// (one round trip for any K, no registers); passes beyond the unit's blocks
// are out of the buffer's range (no memory access) and not read.  An invalid
// unit issues empty loads.
__device__ __forceinline__ void issue_x(const Unit& U, uint32_t* xin, int lane) {
    const __amdgpu_buffer_rsrc_t xr = rsrc(U.x, U.valid ? (uint32_t)U.nb * 256u : 0u);
#pragma unroll
    for (int p = 0; p < kXPasses; ++p) load_to_lds(xr, &xin[p * 256], (uint32_t)(p * 64 + lane) * 16u);
}

// The control wavefront tells the streaming ones that unit j's activation
// is in xin (after wait_vm_all); they wait for it (bounded, like await_unit).
__device__ __forceinline__ void x_ready(SweepLds& L, int j, int lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_store(&L.xready, (uint32_t)(j + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void await_x(const SweepLds& L, int j) {
    for (int i = 0; i < kDescSpin; ++i) {
        const uint32_t s = __hip_atomic_load(&L.xready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (__builtin_amdgcn_readfirstlane((int)s) == j + 1) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Streaming wavefront q quantizes passes q, q + 4, ... of unit U's
// activation (in xin) into split / scale; the four share the work, which
// one wavefront took 0.3 us per pass for.
__device__ __forceinline__ void quantize_x(const Unit& U, uint32_t* split, float* scale, const uint32_t* xin, int q,
                                           int lane) {
    const int ii = lane & 15, row = lane >> 4;
    const int npass = U.valid ? U.nb >> 2 : 0;
    for (int p = q; p < npass; p += kStreamWaves) {
        const float4 v = *reinterpret_cast<const float4*>(&xin[p * 256 + lane * 4]);
        const float x4[4] = {v.x, v.y, v.z, v.w};
        bfp8_quant4_store_lds(x4, ii, &scale[4 * p + row], &split[(4 * p + row) * 32], true);
    }
}

// The control wavefront finishes unit U from the streaming wavefronts'
// partial sums red (lane = row): y = (fs0 + fs2) + (fs1 + fs3).  A GEMV tile
// stores its rows' y; an lm_head tile ranks its 64 keys (a key's rank is the
// number of keys above it: keys are unique) and publishes its best topk as
// its partial list, entry rank.
__device__ __forceinline__ void finish_unit(const Ctx& C, const Unit& U, const float* red, SweepLds& L) {
    const int lane = C.lane;
    const float y = (red[lane] + red[128 + lane]) + (red[64 + lane] + red[192 + lane]);
    const int row = U.tile * BFP8_TILE_ROWS + lane;
    if (!U.head) {
        if (row < U.rows) reinterpret_cast<float*>(U.y)[row] = y;
        return;
    }
    const uint64_t mine = tile_rank_key(y, row, row < U.rows);
    L.keys[lane] = mine;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const u64x2* k2 = reinterpret_cast<const u64x2*>(L.keys);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const u64x2 v = k2[i];
        cnt += (v.x > mine ? 1 : 0) + (v.y > mine ? 1 : 0);
    }
    if (cnt < C.topk) {
        const EpochKeys kf{C.epoch};
        kf.store(C.partials + (size_t)U.tile * C.topk + cnt, kf.make(tile_partial_key(mine), (int)~(uint32_t)mine));
    }
    // the keys are read before they are written again (the next lm_head tile)
    __builtin_amdgcn_wave_barrier();
}

// B_start: a workgroup barrier that waits for this wavefront's LDS operations
// only.  __syncthreads() would first wait for the control wavefront's loads
// to LDS (a release covers them: vmcnt(0)), and the streaming wavefronts
// would issue their first weight loads only when the table and the
// activation are in, ~2 us into the launch; so the LDS words initialized
// before it are what it publishes, and those loads are still in flight when
// the weight loads go out.
__device__ __forceinline__ void barrier_start() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---- the two roles -----------------------------------------------------------------------------
// The control wavefront, unit by unit: between barriers B_j (the start of
// unit j) and B_j+1 it takes unit j + 1 (the ticket overlaps finishing unit
// j - 1, whose partial sums were in LDS at B_j), publishes it and loads its
// activation into xin, which the streaming wavefronts quantize into the
// slot of unit j - 1 (whose last chunk was reduced before B_j) before B_j+1.
__device__ void control_role(const Ctx& C, const Bfp8SweepGemv* gemvs, SweepLds& L, uint32_t* xin) {
    const int lane = C.lane;
    // LDS holds what the previous workgroup on this CU left there: no
    // sequence word may read as published before its unit is (the streaming
    // wavefronts first look at one after B_start)
    if (lane == 0) {
        __hip_atomic_store(&L.desc[0].seq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_store(&L.desc[1].seq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_store(&L.xready, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // the GEMV table goes to LDS, and a first unit that is an lm_head tile
    // needs no table: its activation's loads go out with it, all before any
    // weight load of the workgroup (B_start), so that they do not queue
    // behind the weight streams
    const __amdgpu_buffer_rsrc_t tr = rsrc((uint64_t)gemvs, (uint32_t)(C.ngemv * (int)sizeof(Bfp8SweepGemv)));
#pragma unroll
    for (int j = 0; j < kTabLoads; ++j) load_to_lds(tr, &L.tab[j * 256], (uint32_t)(lane + 64 * j) * 16u);
    const bool head0 = C.ns > 0 && C.head_ntiles > 0;
    Unit U = head0 ? head_unit(C, 0) : no_unit();
    if (head0) issue_x(U, xin, lane);
    barrier_start();  // B_start
    wait_vm_all();
    if (!head0) {
        // published before its activation is read: the streaming wavefronts
        // start its weights meanwhile
        U = resolve(C, L, 0, take(C, 0));
        publish(L, 0, U, lane);
        issue_x(U, xin, lane);
        wait_vm_all();
    }
    x_ready(L, 0, lane);
    __syncthreads();  // B_0
    if (!U.valid) return;
    Unit P = no_unit();  // the unit to finish (its partial sums are in LDS)
    int j = 0;
    for (;; ++j) {
        const uint32_t t = take(C, j + 1);
        if (P.valid) finish_unit(C, P, L.red[(j - 1) & 1], L);
        const Unit N = resolve(C, L, j + 1, t);
        publish(L, j + 1, N, lane);
        issue_x(N, xin, lane);
        wait_vm_all();
        x_ready(L, j + 1, lane);
        __syncthreads();  // B_j+1 (after the last unit: its closing barrier)
        P = U;
        if (!N.valid) break;
        U = N;
    }
    finish_unit(C, P, L.red[j & 1], L);
}

// A streaming wavefront.  Chunks of a unit alternate between c[0] (even) and
// c[1] (odd); units have an even number of chunks, so every unit starts in
// c[0], and a unit's first two chunks are issued before the previous unit's
// barrier.  A step issues the next chunk (the next unit's chunks 0 and 1
// after a unit's last ones, an empty range when there is none), then waits
// for and reduces the current one.
__device__ void stream_role(const Ctx& C, int q, SweepLds& L, const uint32_t* xin) {
    const int lane = C.lane;
    const uint32_t vw = (uint32_t)(q * 1024 + lane * 16), ve = (uint32_t)(lane * 4);
    Chunk c[2];
    Unit U;
    // the first unit's chunks 0 and 1 go out before its activation is in
    // LDS (after the control wavefront's first loads: B_start); an lm_head
    // tile is known without the control wavefront
    barrier_start();  // B_start
    const bool head0 = C.ns > 0 && C.head_ntiles > 0;
    U = head0 ? head_unit(C, 0) : await_unit(L, 0);
    issue_chunk(c[0], U, 0, vw, ve);
    issue_chunk(c[1], U, 1, vw, ve);
    await_x(L, 0);
    quantize_x(U, L.split[0], L.scale[0], xin, q, lane);
    __syncthreads();  // B_0
    for (int j = 0; U.valid; ++j) {
        const uint32_t* sp = L.split[j & 1];
        const float* sc = L.scale[j & 1];
        const int nch = U.nb / kChunk;
        float fs = reduce_chunk(0.0f, c[0], 0, q, sp, sc);
        for (int k = 1; k + 1 < nch; k += 2) {
            issue_chunk(c[0], U, k + 1, vw, ve);
            fs = reduce_chunk(fs, c[1], k, q, sp, sc);
            issue_chunk(c[1], U, k + 2, vw, ve);
            fs = reduce_chunk(fs, c[0], k + 1, q, sp, sc);
        }
        computed(fs);
        const Unit N = await_unit(L, j + 1);
        issue_chunk(c[0], N, 0, vw, ve);
        fs = reduce_chunk(fs, c[1], nch - 1, q, sp, sc);
        issue_chunk(c[1], N, 1, vw, ve);
        L.red[j & 1][q * 64 + lane] = fs;
        await_x(L, j + 1);
        quantize_x(N, L.split[(j + 1) & 1], L.scale[(j + 1) & 1], xin, q, lane);
        __syncthreads();  // B_j+1 (the next unit's activation is in LDS)
        U = N;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the last (empty) chunks are in
}

}  // namespace

extern "C" __global__ __launch_bounds__(kThreads) void bfp8_sweep_kernel(Bfp8SweepArgs a) {
    __shared__ __align__(16) SweepLds L;
    extern __shared__ __align__(16) uint32_t xin[];  // kXinBytes
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    Ctx C;
    C.lane = threadIdx.x & 63;
    C.wg = (int)blockIdx.x;
    C.nwg = (int)gridDim.x;
    C.ngemv = a.ngemv;
    C.nunits = a.nunits;
    C.ticket0 = a.ticket0;
    C.nqueues = a.nqueues;
    C.sub = (C.wg / 8) % a.nqueues;
    C.ctr = a.counters + C.sub * BFP8_SWEEP_CTR_STRIDE;
    C.head_mant = (uint64_t)a.head_mant;
    C.head_exps = (uint64_t)a.head_exps;
    C.head_x = (uint64_t)a.head_x;
    C.head_nb = a.head_nb;
    C.head_ntiles = a.head_ntiles;
    C.head_rows = a.head_pair_rows;
    C.topk = a.topk;
    C.partials = a.partials;
    C.epoch = a.epoch;
    const bool head = a.head_ntiles > 0;
    C.hnwg = head ? C.nwg - 1 : C.nwg;
    if (head)
        C.ns = C.wg < C.hnwg && C.wg < a.head_ntiles ? (a.head_ntiles - C.wg + C.hnwg - 1) / C.hnwg : 0;
    else
        C.ns = C.wg < a.nunits ? 1 : 0;

    // the other counter set, for the next launch: the last workgroup's fifth
    // wavefront (idle in the merging workgroup), one lane per counter
    if (C.wg == C.nwg - 1 && wave == kStreamWaves && C.lane < a.nqueues)
        __hip_atomic_store(a.counters_next + C.lane * BFP8_SWEEP_CTR_STRIDE, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    if (head && C.wg == C.nwg - 1) {
        // the merging workgroup: four wavefronts merge the lm_head's lists as
        // they are published (the fifth ends here; a barrier waits only for
        // the wavefronts that have not ended)
        if (wave < kStreamWaves) {
            const TopkArgs ta{a.partials, a.out_ids, a.out_scores, a.out_count, a.out_argmax, a.topk, a.head_ntiles};
            topk_merge<kStreamWaves, 4, 4, false>(ta, EpochKeys{a.epoch}, L.merge);
        }
    } else if (wave == kStreamWaves) {
        control_role(C, a.gemvs, L, xin);
        return;
    } else {
        stream_role(C, wave, L, xin);
    }
}

// ---- launcher -----------------------------------------------------------------------------
// CUs and resident workgroups per CU of the kernel (queried once).  A
// workgroup's five wavefronts put two on one SIMD, so a CU holds at most
// (wavefronts per SIMD) / 2 of them, whatever the occupancy query says: at
// 89 VGPRs (5 wavefronts per SIMD) only two of three workgroups per CU ran
// at once, the third started when one of them ended.
static void sweep_residency(int* cus, int* occ) {
    static const int2 r = [] {
        int dev = 0, n = 256, o = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
            n = p.multiProcessorCount;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, reinterpret_cast<const void*>(bfp8_sweep_kernel),
                                                         kThreads, kXinBytes) != hipSuccess ||
            o <= 0)
            o = 1;
        hipFuncAttributes fa;
        if (hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(bfp8_sweep_kernel)) == hipSuccess &&
            fa.numRegs > 0) {
            const int per_simd = std::min(8, 512 / ((fa.numRegs + 7) & ~7));
            o = std::max(1, std::min(o, per_simd / 2));
        }
        return int2{n, o};
    }();
    *cus = r.x;
    *occ = r.y;
}

int bfp8_sweep_grid(int per_cu) {
    int cus = 0, occ = 0;
    sweep_residency(&cus, &occ);
    return cus * (occ < per_cu ? occ : per_cu);
}

hipError_t bfp8_launch_sweep(const Bfp8SweepArgs& a, int nwg, hipStream_t s) {
    if (nwg <= 0) return hipSuccess;
    int cus = 0, occ = 0;
    sweep_residency(&cus, &occ);
    if (nwg > cus * occ || a.ngemv > BFP8_SWEEP_MAX_GEMV || a.head_ntiles > BFP8_TOPK_MAX_TILES || a.nqueues < 1 ||
        a.nqueues > BFP8_SWEEP_QUEUES || (a.nqueues > 1 && 8 * a.nqueues > nwg) || (a.head_ntiles > 0 && nwg < 2))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(bfp8_sweep_kernel, dim3(nwg), dim3(kThreads), kXinBytes, s, a);
    return hipGetLastError();
}
