// Tile geometry of the MFMA kernels, shared by host and device code.
//
//   fp32                      128 x 128 tiles everywhere; direct global->LDS
//                             loads (mec_gemm_dma.h) for 16-byte vectors,
//                             else staged through registers (mec_gemm_f32.h);
//                             64 x 64 direct-to-LDS tiles at a small n
//                             (f32_small_n), so that the grid covers the CUs,
//                             and per launch where a 128 x 128 grid is small
//                             for its K or fills its rounds of CUs poorly
//                             (f32_small_fwd, f32_small_bwd)
//   bf16 / fp16, 16-byte      forward sums and gradient-matrix tiles 256 x 256
//   vectors                   (x rows x y rows, 8 waves), direct global->LDS
//                             loads (mec_gemm_dma.h); contractions 256 x 256
//                             (output rows x feature columns, 8 waves) in a
//                             kernel of their own, a last column of at most
//                             128 features in 512 x 128 tiles where faster;
//                             256 x 384 where those take fewer rounds of work
//   bf16 / fp16, other        forward sums and gradient-matrix tiles 128 x 128
//   layouts                   staged through registers (mec_gemm_16.h); the
//                             contractions read internal buffers, which are
//                             always 16-byte vectors, so they keep 256 x 256
//   fp32 data with bf16       the bf16 tiles on internal bf16 / split copies
//   products (bf16, bf16x3)   of the inputs (always 16-byte vectors)
//
// The backward's block decomposition uses blocks of a multiple of
// block_quantum(dtype) rows, so that every tile kind divides a block.
#pragma once
#include <stdint.h>

namespace mec {

struct TileDims {
  int bm, bn;
};

constexpr int kDtypeF32 = 0;
constexpr int kDtypeBF16 = 1;
constexpr int kDtypeF16 = 2;
constexpr int kDtypeX3 = 3;   // fp32 data, products as three bf16 MFMA terms
constexpr int kDtypeF32B = 4;  // fp32 data, bf16 products

// fp32 direct-to-LDS problems whose 128 x 128 grid has fewer than two tiles
// per CU of a 256-CU device (n <= 2816) run 64 x 64 tiles instead (`small`)
inline bool f32_small_n(int64_t n) {
  const int64_t t = (n + 127) / 128;
  return t * t < 512;
}
// Share of the CU slots of a launch of `tiles` workgroups, one per CU per
// round, that its rounds keep busy: tiles / (cus * rounds).
inline double round_fill(int64_t tiles, int cus) {
  const int64_t rounds = (tiles + cus - 1) / cus;
  return (double)tiles / ((double)rounds * cus);
}
// fp32 forward tiles: 64 x 64 for f32_small_n, and for D >= 512 where the
// 128 x 128 grid fills its rounds below 90% (measured on one MI355X: the
// forward 7-23% faster at N = 3072 and 5120, D = 512-1024; at D = 128-256 and
// elsewhere the 128 x 128 tiles were as fast or up to 26% faster).
inline bool f32_small_fwd(int64_t n, int64_t d, int cus) {
  if (f32_small_n(n)) return true;
  const int64_t t = (n + 127) / 128;
  return d >= 512 && round_fill(t * t, cus) < 0.9;
}
// fp32 backward tiles for blocks of bs rows: 64 x 64 for f32_small_n, and
// where a step's 128 x 128 gradient-matrix tiles (ceil(n/128) ceil(bs/128))
// are few for their K (tiles x D <= 2^17) or fill their rounds below 90%.
// Measured on one MI355X: at D = 128-256 (1024-row blocks) the 64 x 64
// backward was 1.2-2.6x faster up to N = 8192 and even at 2^17; with a poor
// last round (N = 3072 and 5120 at D = 512-1024) 9-20% faster; elsewhere the
// 128 x 128 tiles were as fast or up to 10% faster.
inline bool f32_small_bwd(int64_t n, int64_t d, int64_t bs, int cus) {
  if (f32_small_n(n)) return true;
  const int64_t g = ((n + 127) / 128) * ((bs + 127) / 128);
  return g * d <= ((int64_t)1 << 17) || round_fill(g, cus) < 0.9;
}
// forward sums and gradient-matrix tiles (x rows x y rows)
inline TileDims fwd_tile_dims(int dtype, bool vec, bool small = false) {
  if (dtype == kDtypeX3 || dtype == kDtypeF32B) return {256, 256};
  if (dtype == kDtypeF32 && vec && small) return {64, 64};
  if (dtype == kDtypeF32 || !vec) return {128, 128};
  return {256, 256};
}
// contraction tiles (output rows x feature columns)
inline TileDims con_tile_dims(int dtype, bool small = false) {
  if (dtype == kDtypeF32) return small ? TileDims{64, 64} : TileDims{128, 128};
  return {256, 256};
}
// contractions run in their own kernel (k_grad_contract) rather than inside k_grad_step
inline bool separate_contractions(int dtype) { return dtype != kDtypeF32; }
// k_grad_contract: a last feature column of at most 128 of the 256 features
// of a tile is contracted by 512 x 128 tiles (one per pair of row tiles, so
// the block's row tiles must pair up) instead of half-empty 256 x 256 tiles
inline bool narrow_contract_shape(int d, int ctm) {
  const int rem = d % 256;
  return rem != 0 && rem <= 128 && ctm % 2 == 0;
}
inline int block_quantum(int dtype) { return dtype == kDtypeF32 ? 128 : 256; }

}  // namespace mec
