// bfp8_layout.h -- the GPU-side BFP8 weight and activation layouts.
//
// The reference stores each BFP8 tensor as two planes (05/bfp8_packer.py:53-86,
// sliced by the engine at 04/qwen_real_engine.py:834-846):
//   mantissas  int8  [M][K]     (row stride K; block b of row m = bytes 64b..64b+63)
//   exponents  uint8 [M][K/64]  (scale of a block = 2^(e-134))
//
// The reference's NEON GEMV keeps four int32 accumulator lanes per row: lane j
// sums the products of elements k = j (mod 4) of a block (the "residue"
// lanes, 04/qwen_kernels_opt.c:226-257), and its float epilogue is defined per
// residue lane.  The GPU layout is built around that:
//
// Mantissa plane ("tile-block-residue"):
//   rows are grouped in tiles of 64 (one wavefront lane per row; the last
//   tile is zero-padded).  For tile t, block b, residue q (0..3), lane r:
//     16 bytes at  ((t*NB + b)*4 + q)*1024 + r*16
//   holding the 16 mantissas of row 64t+r, block b, residue q.  Byte 4d+p of
//   the 16 is element k = 16d + 4p + q of the block, so each dword holds four
//   elements of one residue, ready for one v_dot4_i32_i8.  One wavefront
//   load of 64 lanes x 16 B reads 1 KiB of contiguous memory.
//
// Exponent plane:
//   for tile t, block group g = b/4, lane r: one dword at
//     ((t*NB4 + g)*64 + r)*4,   NB4 = ceil(NB/4),
//   byte p = exponent of block 4g+p of row 64t+r (raw e, unchanged).
//
// Activation split ("xsplit"):
//   xq (int16, |xq| <= 16384) is written exactly as 256*xh + xl with
//   xl = (int8)(xq & 0xff) and xh = (xq - xl) >> 8 (so |xh| <= 64).  For
//   block b and residue q, 8 dwords at word offset (b*4 + q)*8:
//     dwords 0..3: xh of elements 16d + 4p + q (d = dword, p = byte)
//     dwords 4..7: xl of the same elements
//   so S_q = (dot4 chain over xh) * 256 + (dot4 chain over xl), exactly.
#pragma once
#include <stddef.h>
#include <stdint.h>

#define BFP8_BLOCK 64
#define BFP8_TILE_ROWS 64
#define BFP8_XSPLIT_WORDS_PER_BLOCK 32

#if defined(__HIPCC__)
#define BFP8_HD __host__ __device__
#else
#define BFP8_HD
#endif

BFP8_HD static inline int bfp8_nblocks(int K) { return K > 0 ? K / BFP8_BLOCK : 0; }
BFP8_HD static inline int bfp8_ntiles(int M) { return M > 0 ? (M + BFP8_TILE_ROWS - 1) / BFP8_TILE_ROWS : 0; }
BFP8_HD static inline int bfp8_nb4(int nb) { return (nb + 3) / 4; }

BFP8_HD static inline size_t bfp8_gpu_mant_bytes(int M, int K) {
    return (size_t)bfp8_ntiles(M) * (size_t)bfp8_nblocks(K) * 4096u;
}
BFP8_HD static inline size_t bfp8_gpu_exps_bytes(int M, int K) {
    return (size_t)bfp8_ntiles(M) * (size_t)bfp8_nb4(bfp8_nblocks(K)) * 256u;
}
BFP8_HD static inline size_t bfp8_xsplit_bytes(int K) {
    return (size_t)bfp8_nblocks(K) * BFP8_XSPLIT_WORDS_PER_BLOCK * 4u;
}
