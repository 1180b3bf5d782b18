// wave_topk.h -- wavefront-level top-k building blocks shared by the GEMV
// and lm_head kernels: 64-bit (score, row) keys, xor-lane exchange, bitonic
// sort and merge networks over one wave64.  Device code only; every function
// is inline and works on integers, so it behaves the same in flush-to-zero and
// IEEE translation units.
#pragma once

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// ---- top-k keys ------------------------------------------------------------
// Order (score desc, id asc) as one unsigned 64-bit key, larger = better.
// Candidates are the scores the reference would ever offer: > -FLT_MAX, not
// NaN (04/qwen_sampling.c:243-248 with thr = -FLT_MAX, compared in IEEE
// arithmetic).  -0 equals +0 there, so it is keyed as +0; a subnormal score
// keeps its value.  The tests are on the bits: a float compare inside a
// flush-to-zero unit would read a subnormal score as zero.  0 is "no
// candidate".
__device__ __forceinline__ uint64_t topk_key(float y, int row) {
    uint32_t b = __float_as_uint(y);
    const uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u || b == 0xff800000u || b == 0xff7fffffu) return 0;  // NaN, -inf, -FLT_MAX
    if (a == 0u) b = 0u;
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)row;
}
__device__ __forceinline__ float key_score(uint64_t k) {
    uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)~(uint32_t)k; }

// The same order for ranking a tile's rows: every row gets a distinct key,
// rows without a candidate (invalid score, or past the rows in use) one below
// every candidate (high word 0).  tile_partial_key maps those back to 0.
__device__ __forceinline__ uint64_t tile_rank_key(float y, int row, bool in_use) {
    const uint64_t k = in_use ? topk_key(y, row) : 0ull;
    return k ? k : (uint64_t)(uint32_t)~(uint32_t)row;
}
__device__ __forceinline__ uint64_t tile_partial_key(uint64_t k) { return (k >> 32) ? k : 0ull; }

// A 64-row tile's top-`topk` list (descending, "no candidate" 0s last) by
// rank instead of a sort, on all four wavefronts of the workgroup: keys[]
// holds the tile's 64 distinct rank keys (LDS, visible to the workgroup);
// lane (r, qq) = (lane >> 2, lane & 3) of wavefront w counts the keys among
// keys[16qq .. 16qq+15] above its row's key 16w + r, the quad adds the four
// counts (DPP), and quarter 0 stores the key at its rank.  Distinct keys make
// the ranks a permutation of 0..63, so slots 0..topk-1 are all written.
__device__ __forceinline__ void tile_topk_rank(const uint64_t* keys, uint64_t* partials, int tile, int topk, int w,
                                               int lane) {
    const int r = lane >> 2, qq = lane & 3;
    const uint64_t mine = keys[16 * w + r];
    const uint64_t* quarter = keys + 16 * qq;
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) cnt += quarter[i] > mine ? 1 : 0;
    cnt += __builtin_amdgcn_update_dpp(0, cnt, 0xB1, 0xF, 0xF, false);  // + quad lane ^ 1
    cnt += __builtin_amdgcn_update_dpp(0, cnt, 0x4E, 0xF, 0xF, false);  // + quad lane ^ 2
    if (qq == 0 && cnt < topk) partials[(size_t)tile * topk + cnt] = tile_partial_key(mine);
}

// ---- wavefront exchange ----------------------------------------------------
// Lane i receives lane i^j.  j = 1, 2: DPP quad permutes; j = 4, 8: two DPP
// moves each (quad_perm [3,2,1,0] gives i^3, row_half_mirror i^7, row_mirror
// i^15 within a row of 16: i^3^7 = i^4, i^15^7 = i^8), no LDS round trip;
// j = 16: ds_swizzle bit-mask mode (and 0x1f, xor 16, within 32 lanes);
// j = 32, 63: ds_bpermute.  Always called with j a constant after unrolling.
template <int kCtrl>
__device__ __forceinline__ int dpp_move(int v) {
    return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t xor_lane32(uint32_t v, int j) {
    switch (j) {
        case 1: return (uint32_t)dpp_move<0xB1>((int)v);
        case 2: return (uint32_t)dpp_move<0x4E>((int)v);
        case 4: return (uint32_t)dpp_move<0x141>(dpp_move<0x1B>((int)v));
        case 8: return (uint32_t)dpp_move<0x141>(dpp_move<0x140>((int)v));
        case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (16 << 10));
        default: return (uint32_t)__shfl_xor((int)v, j, 64);
    }
}
__device__ __forceinline__ uint64_t xor_lane(uint64_t v, int j) {
    const uint32_t lo = xor_lane32((uint32_t)v, j);
    const uint32_t hi = xor_lane32((uint32_t)(v >> 32), j);
    return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort of N independent columns (one key per lane each), column n
// descending by lane when desc[n], else ascending; the N compare-exchange
// chains interleave.  A compare-exchange keeps the partner's key when
// (partner > own) equals "this lane keeps the larger" -- one 64-bit compare
// and one select.
template <int N>
__device__ __forceinline__ void wave_sort(uint64_t (&key)[N], const bool (&desc)[N], int lane) {
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const bool up = ((lane & j) == 0) == ((lane & k) == 0);
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const uint64_t o = xor_lane(key[n], j);
                key[n] = ((o > key[n]) == (up == desc[n])) ? o : key[n];
            }
        }
    }
}

// a and b sorted in opposite directions -> the 64 largest keys of both,
// sorted descending (kDesc) or ascending: max(a[i], b[i]) holds them as a
// bitonic sequence, six half-cleaner stages sort it.
template <bool kDesc>
__device__ __forceinline__ uint64_t wave_merge(uint64_t a, uint64_t b, int lane) {
    uint64_t c = a > b ? a : b;
#pragma unroll
    for (int j = 32; j > 0; j >>= 1) {
        const uint64_t o = xor_lane(c, j);
        c = ((o > c) == (((lane & j) == 0) == kDesc)) ? o : c;
    }
    return c;
}

// Pairwise tree merge of N (power of two) lists held as even = descending,
// odd = ascending; the result is descending.
template <int N>
__device__ __forceinline__ uint64_t wave_merge_tree(uint64_t (&v)[N], int lane) {
#pragma unroll
    for (int s = 1; s < N; s <<= 1) {
#pragma unroll
        for (int i = 0; i < N; i += 2 * s) {
            if ((i / (2 * s)) % 2 == 0)
                v[i] = wave_merge<true>(v[i], v[i + s], lane);
            else
                v[i] = wave_merge<false>(v[i], v[i + s], lane);
        }
    }
    return v[0];
}

}  // namespace
