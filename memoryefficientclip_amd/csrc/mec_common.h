// Common device helpers for the MI355X (gfx950) contrastive-loss kernels.
//
// Conventions used by every kernel in this library:
//   * x, y are row-major [n, d] feature matrices with a row stride (ldx, ldy)
//     in elements and unit column stride.  x is the "row" side of the
//     similarity matrix S = X^ Y^T (image for CLIP, text for LiT).
//   * rx[i] = 1 / max(||x_i||, 1e-12) when the L2 normalisation is fused,
//     else 1.  Same for ry.  S_ij = rx_i * ry_j * (x_i . y_j).
//   * E_ij = exp((S_ij - 1) / T) = exp2(S_ij * c - c) with c = log2(e) / T
//     (the fixed-max trick: for unit rows S <= 1 so E <= 1).
//   * The diagonal i == j is kept out of every tile reduction; it is added
//     back exactly from diag[i] = x_i . y_i by the finalize/postpass kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include <type_traits>

namespace mec {

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time (the
// index can then be a template argument, e.g. an instruction's immediate offset)
template <int I, int N, class F>
__device__ __forceinline__ void static_for_from(F& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_from<I + 1, N>(f);
  }
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_from<0, N>(f);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Workspace layout: 8 float vectors of length n, then ceil(n / FIN_ROWS)
// doubles of per-workgroup loss partials (see include/mec.h).
enum WsSlot {
  WS_RX = 0, WS_RY = 1, WS_DIAG = 2, WS_ROW_OFF = 3, WS_COL_OFF = 4,
  WS_INV_ROW = 5, WS_INV_COL = 6, WS_KAPPA = 7, WS_NSLOTS = 8
};
constexpr int FIN_ROWS = 256;  // rows per workgroup of the loss finalize (one per thread)
// deterministic forward: at most DET_P row blocks x DET_Q column blocks of
// tiles, whose (DET_Q + DET_P) x n partial sums follow the loss partials in
// the workspace (DET_Q row partials per row, then DET_P column partials per
// column)
constexpr int DET_P = 32, DET_Q = 16;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// two values in one dword, a in the low half
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)a, (__bf16)b});
}

// IEEE fp16 (_Float16 storage), round to nearest even (v_cvt_f16_f32 /
// v_cvt_pk_f16_f32)
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Store at device scope: a relaxed atomic store, which gfx950 issues as a
// global store with sc1 (written through this XCD's L2).  For a launch's last
// stores, read by the next launch.  Measured against plain stores on the
// kept-matrix path (1024 x 1024 similarities, 1024 x 512 outputs): the forward
// 1.2 us and the fused backward 1.3 us shorter; the finalize's in-place
// stores, which sit mid-launch, 0.7 us longer, so they stay plain.
__device__ __forceinline__ void store_device(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
// v_mfma_f32_32x32x16_{bf16,f16}: 8 16-bit values of A and of B per lane
// (their bits in an i16x8), fp32 accumulate
template <bool F16>
__device__ __forceinline__ f32x16 mfma16_32x32x16(i16x8 a, i16x8 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Row index (within a 32x32 MFMA output block) held by accumulator register r
// of lane `lane`: rows come in groups of 4, lanes 32..63 hold the odd groups.
__device__ __forceinline__ int acc_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// Workgroup ids are dispatched round-robin over the 8 XCDs (id % 8).  Remap a
// launch-local id in [0, nbid) (nbid a multiple of 8) so that each XCD gets a
// contiguous range of logical ids; identity when nbid is not a multiple of 8.
__device__ __forceinline__ int xcd_remap(int bid, int nbid) {
  return (nbid & 7) == 0 ? (bid & 7) * (nbid >> 3) + (bid >> 3) : bid;
}

// Order logical ids pid in [0, tiles_m * tiles_n) in groups of `group_m` tile
// rows, so that neighbouring workgroups share operand rows in one XCD's L2.
__device__ __forceinline__ void group_tile(int pid, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  int per_group = group_m * tiles_n;
  int gid = pid / per_group;
  int first_m = gid * group_m;
  int gsize = tiles_m - first_m;
  if (gsize > group_m) gsize = group_m;
  int in_group = pid - gid * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// Both steps for a launch of exactly tiles_m * tiles_n workgroups.
__device__ __forceinline__ void tile_swizzle(int bid, int nbid, int tiles_m, int tiles_n,
                                             int group_m, int& tm, int& tn) {
  group_tile(xcd_remap(bid, nbid), tiles_m, tiles_n, group_m, tm, tn);
}

// Wave-wide sum over the 32 lanes of each half-wave (lanes l and l^32 are not mixed).
__device__ __forceinline__ float half_wave_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 1, 64);
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v += __shfl_xor(v, 32, 64);
  return half_wave_sum(v);
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Transpose-reduce of 32 per-lane values across the 32 lanes of a half-wave:
// on return lane l holds sum over the half-wave's lanes of vals[l % 32].
// Costs 31 shuffles instead of 32 * 5.
__device__ __forceinline__ float transpose_reduce32(float (&v)[32], int lane) {
  const int q = lane & 31;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    bool hi = q & 16;
    float send = hi ? v[k] : v[k + 16];
    float keep = hi ? v[k + 16] : v[k];
    v[k] = keep + __shfl_xor(send, 16, 64);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    bool hi = q & 8;
    float send = hi ? v[k] : v[k + 8];
    float keep = hi ? v[k + 8] : v[k];
    v[k] = keep + __shfl_xor(send, 8, 64);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    bool hi = q & 4;
    float send = hi ? v[k] : v[k + 4];
    float keep = hi ? v[k + 4] : v[k];
    v[k] = keep + __shfl_xor(send, 4, 64);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    bool hi = q & 2;
    float send = hi ? v[k] : v[k + 2];
    float keep = hi ? v[k + 2] : v[k];
    v[k] = keep + __shfl_xor(send, 2, 64);
  }
  {
    bool hi = q & 1;
    float send = hi ? v[0] : v[1];
    float keep = hi ? v[1] : v[0];
    v[0] = keep + __shfl_xor(send, 1, 64);
  }
  return v[0];
}

}  // namespace mec
