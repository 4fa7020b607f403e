// MFMA tile kernels of the contrastive-loss hot path (fp32, bf16 and fp16 inputs;
// the element type and layout select the MFMA core and tile shape, the
// epilogues are shared):
//   k_sumexp        forward: tiled S = X Y^T, E = exp2(S c - c), off-diagonal
//                       row (and column) partial sums, one atomic per row/column
//                       per tile.  Replaces clip_sum_exp_kernel (clip_loss.py:9-64)
//                       and lit_sum_exp_kernel (lit_loss.py:9-62).
//   k_grad_step     backward, one launch per pipeline step t = 0..nb over
//                       the block diagonals of the N x N gradient matrix:
//                       recompute S for diagonal t and write the blocks
//                       G'_ij = E_ij (1/R_i + 1/C_j) (LiT: E_ij / R_i), i != j,
//                       to one of two bounded scratch buffers
//                       (clip_loss.py:96-124, lit_loss.py:94-120), while
//                       contracting diagonal t-1 from the other buffer:
//                       dX_I += G'_IJ Y^_J and dY_J += G'_IJ^T X^_I as plain MFMA
//                       contractions without contending atomics
//                       (clip_loss.py:127-156, lit_loss.py:123-148); fp32
//                       runs both kinds of tile in this launch.
//   k_grad_g_chain  the 16-bit gradient-matrix tiles of inputs already
//                       normalized, chained in persistent workgroups.
//   k_grad_contract the 16-bit types' contractions of one pipeline step, in
//                       a launch of their own with larger tiles (256 x 256,
//                       or 256 x 384 where that takes fewer rounds, and
//                       narrow ones for a last column of at most 128
//                       features).
//   k_sumexp_det, k_det_reduce
//                   the forward sums without atomics across workgroups, in
//                       one pass (deterministic mode, and always for the
//                       16-bit tiles that chain).
#pragma once
#include <type_traits>

#include "mec_gemm_f32.h"
#include "mec_gemm_16.h"
#include "mec_gemm_dma.h"
#include "mec_tiles.h"

namespace mec {

// ------------------------------------------------------------ tile configs
// Every config: BM x BN output tile per workgroup of WM x WN waves (NT
// threads), each wave a TM x TN sub-tile of FM x FN 32x32 MFMA blocks whose
// accumulator register r of lane l holds element (acc_row(r, l), l % 32).
#ifndef MEC_16BIT_BK
#define MEC_16BIT_BK 64
#endif

// fp32, 128 x 128, operands staged through registers
struct TileF32 {
  using Elem = float;
  using Op = g32::Operand;
  static constexpr bool TA = false, GB = false;
  static constexpr int TB = 0;
  static constexpr int BM = 128, BN = 128, TM = 64, TN = 64, FM = 2, FN = 2, WM = 2, WN = 2, NT = 256;
  static constexpr int LDS_BYTES = g32::LDS_FLOATS * 4;
  static constexpr bool CHAIN = false;
  template <bool VECA, bool VECB>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[FM][FN]) {
    g32::mainloop<VECA, VECB>(a, b, K, (float*)lds, acc);
  }
  static __device__ __forceinline__ float pack(float v) { return v; }
  static __device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
    *(f32x4*)p = f32x4{a, b, c, d};
  }
};

// fp32 -> 16-bit packing of the gradient-matrix tiles (two values per 32-bit word)
template <bool F16>
struct Pack16 {
  static __device__ __forceinline__ uint32_t pack2(float a, float b) { return F16 ? pack2_f16(a, b) : pack2_bf16(a, b); }
};

// bf16 / fp16, 128 x 128, operands staged through registers (any alignment / D)
template <bool F16>
struct Tile16V : Pack16<F16> {
  using Elem = uint16_t;
  using Op = g16::Operand;
  static constexpr bool TA = false, GB = false;
  static constexpr int TB = 0;
  static constexpr int BM = 128, BN = 128, TM = 64, TN = 64, FM = 2, FN = 2, WM = 2, WN = 2, NT = 256;
  static constexpr int LDS_BYTES = g16::Cfg<MEC_16BIT_BK>::LDS_ELEMS * 2;
  static constexpr bool CHAIN = false;
  template <bool VECA, bool VECB>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[FM][FN]) {
    g16::mainloop<MEC_16BIT_BK, VECA, VECB, F16>(a, b, K, (uint16_t*)lds, acc);
  }
};

struct PackF32 {
  static __device__ __forceinline__ float pack(float v) { return v; }
  static __device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
    *(f32x4*)p = f32x4{a, b, c, d};
  }
};
template <int KIND> struct PackOf { using type = Pack16<KIND == gdma::K_F16>; };
template <> struct PackOf<gdma::K_F32> { using type = PackF32; };

// BM_ x BN_, direct global->LDS loads (16-byte aligned rows, ld and kmax
// multiples of the elements per 16-byte vector), element kind KIND (bf16,
// fp16 or fp32); TA_: A stored k-row-major (a transposed gradient-matrix
// block); GB_: A a 16-bit gradient-matrix block in the blocked layout
// (gdma::gb_offset; TA_ then selects the x side's reading); TB_: B stored
// k-row-major (fp32 raw input rows; 1: 16-byte lanes, 2: 4-byte lanes); S_:
// stages of the LDS ring (gdma::Geo::S)
template <int BM_, int BN_, bool TA_, int WM_, int WN_, int KIND, int SA_ = 2, bool GB_ = false, bool ROLL_ = false,
          int TB_ = 0, int S_ = 2, int KS_ = 1>
struct TileD : PackOf<KIND>::type {
  using Elem = typename std::conditional<KIND == gdma::K_F32, float, uint16_t>::type;
  using Op = gdma::Operand;
  using G = gdma::Geo<BM_, BN_, TA_, WM_, WN_, KIND, SA_, GB_, TB_, S_, KS_>;
  static constexpr bool TA = TA_, GB = GB_, ROLL = ROLL_;
  static constexpr int TB = TB_;
  static constexpr int BM = G::BM, BN = G::BN, TM = G::TM, TN = G::TN, FM = G::FM, FN = G::FN;
  static constexpr int WM = G::WM, WN = G::WN, NT = G::NT;
  static constexpr int LDS_BYTES = G::LDS_BYTES;
  static constexpr bool CHAIN = true;
  template <bool VECA, bool VECB, bool ZERO = true>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[FM][FN]) {
    if constexpr (ROLL) {
      gdma::mainloop_roll<G, ZERO>(a, b, K, (char*)lds, acc);
    } else {
      gdma::mainloop<G, ZERO>(a, b, K, (char*)lds, acc);
    }
  }
  // run() with a hook on the operand values (gdma::NormHook; fp32 tiles)
  template <class FH>
  static __device__ __forceinline__ void run_fh(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[FM][FN],
                                                const FH& fh) {
    static_assert(!ROLL, "the two-fragment-set schedule");
    gdma::LoadPlan<G> lp;
    gdma::prologue<G>(a, b, (char*)lds, lp);
    if constexpr (G::KS == 2) {
      gdma::mainloop_ks2<G, FH>(lp, K, (char*)lds, acc, fh);
      gdma::drain_loads();
      gdma::ks_reduce<G>((char*)lds, acc);
    } else {
      int p0 = 0;
      gdma::mainloop_core<G, true, false, gdma::NoHook, 0, FH>(lp, lp.ra, lp.rb, false, K, (char*)lds, p0, acc,
                                                               gdma::NoHook(), false, fh);
      gdma::drain_loads();
    }
  }
  // Tiles in a chain (a persistent workgroup): start() issues the first
  // tile's chunk 0; chain() runs one tile and, with has_next, leaves chunk 0
  // of the tile (an, bn) in flight for the next call.
  using Plan = gdma::LoadPlan<G>;
  static __device__ __forceinline__ void start(const Op& a, const Op& b, void* lds, Plan& lp) {
    gdma::prologue<G>(a, b, (char*)lds, lp);
  }
  template <class Hook, int VMF = 0>
  static __device__ __forceinline__ void chain(Plan& lp, const Op& an, const Op& bn, bool has_next, int K, void* lds,
                                               int& p0, f32x16 (&acc)[FM][FN], const Hook& hook,
                                               bool vmf_first = false) {
    gdma::mainloop_core<G, true, true, Hook, VMF>(lp, Plan::rsrc_a(an), Plan::rsrc_b(bn), has_next, K, (char*)lds,
                                                  p0, acc, hook, vmf_first);
  }
  static constexpr int STAGE_BYTES = G::STAGE;  // one ring stage
};

// Input element types: float, bf16 bits (uint16_t), fp16 (_Float16).  The
// 16-bit types share every tile and kernel; F16 selects the MFMA and packing.
template <typename T> struct Is16 { static constexpr bool value = false, f16 = false; };
template <> struct Is16<uint16_t> { static constexpr bool value = true, f16 = false; };
template <> struct Is16<_Float16> { static constexpr bool value = true, f16 = true; };
template <typename T> constexpr int kind16() { return Is16<T>::f16 ? gdma::K_F16 : gdma::K_BF16; }

// forward sums and gradient-matrix tiles; contractions (see mec_tiles.h)
template <typename T, bool VEC, bool IS16 = Is16<T>::value> struct FwdTileSel;
template <typename T> struct FwdTileSel<T, false, false> { using type = TileF32; };
template <typename T> struct FwdTileSel<T, true, false> { using type = TileD<128, 128, false, 2, 2, gdma::K_F32>; };
template <typename T> struct FwdTileSel<T, true, true> { using type = TileD<256, 256, false, 4, 2, kind16<T>()>; };
template <typename T> struct FwdTileSel<T, false, true> { using type = Tile16V<Is16<T>::f16>; };
template <typename T, bool VEC> using FwdTile = typename FwdTileSel<T, VEC>::type;
// fp32 at a small N (few 128 x 128 tiles for the CUs): 64 x 64 direct-to-LDS
// tiles of 2 x 2 waves (32 x 32 each) for the forward, the gradient-matrix
// tiles and the contractions, on a ring of SMALL_STAGES stages (16 KB each):
// one wave per SIMD and 16 MFMAs per chunk leave two stages too short a lead
// for the operand loads (measured: the contraction 24.7, 24.7 and 23.3 us per
// launch at N = 1024, D = 512 with 2, 3 and 4 stages)
constexpr int SMALL_STAGES = 4;
template <typename T, bool VEC, bool SMALL> struct GemmTileSel { using type = FwdTile<T, VEC>; };
template <> struct GemmTileSel<float, true, true> {
  using type = TileD<64, 64, false, 2, 2, gdma::K_F32, 2, false, false, 0, SMALL_STAGES>;
};
template <typename T, bool VEC, bool SMALL> using GemmTile = typename GemmTileSel<T, VEC, SMALL>::type;
// Contractions.  fp32 stores each gradient-matrix block once, row-major and
// scaled by both norms (H = diag(rx) G' diag(ry)), and runs the contractions
// inside k_grad_step on the direct-to-LDS core: the x side reads H K-major,
// the y side reads it transposed (k = its row index), and both read the raw
// input rows of the other side as a transposed feature operand (VEC: 16-byte
// lanes, else 4-byte lanes), so no transposed copies exist.  The 16-bit types
// store only G'^T, which the y side reads K-major and the x side reads
// transposed through LDS, in a kernel of their own (k_grad_contract) with
// 256 x 256 tiles of 8 waves, against transposed normalised input copies.
template <typename T, bool VEC = true, bool IS16 = Is16<T>::value> struct ConTileSel;
// (the gradient-matrix operand streams from HBM: three A stages, 160 KB of LDS)
// nx, ny: the narrow tiles of a last feature column of at most 128 features
// (D % 256 in [1, 128]): 512 rows x 128 features, the same 128 x 64 per-wave
// sub-tile shape (operand reads per MFMA) as the wide tiles, two stages (160 KB)
// wx, wy: 256 rows x 384 features where those take fewer rounds of work
// (D = 1152: three feature tiles instead of four and a half-empty fifth), 2 x
// 4 waves of 128 x 96: 192 accumulator registers, one fragment set on the
// rolling operand schedule (gdma::mainloop_roll), the gradient-matrix operand
// in four half-chunk stages and the other in two (160 KB)
template <typename T, bool VEC> struct ConTileSel<T, VEC, false> {
  using x = TileD<128, 128, false, 2, 2, gdma::K_F32, 2, false, false, VEC ? 1 : 2>;
  using y = TileD<128, 128, true, 2, 2, gdma::K_F32, 2, false, false, VEC ? 1 : 2>;
  using nx = x;  // (no narrow tiles)
  using ny = x;
  using wx = x;
  using wy = x;
};
template <typename T, bool VEC> struct ConTileSel<T, VEC, true> {
  using x = TileD<256, 256, true, 4, 2, kind16<T>(), 3, true>;
  using y = TileD<256, 256, false, 4, 2, kind16<T>(), 3, true>;
  using nx = TileD<512, 128, true, 4, 2, kind16<T>(), 2, true>;
  using ny = TileD<512, 128, false, 4, 2, kind16<T>(), 2, true>;
  using wx = TileD<256, 384, true, 2, 4, kind16<T>(), 4, true, true>;
  using wy = TileD<256, 384, false, 2, 4, kind16<T>(), 4, true, true>;
};
template <typename T, bool VEC = true> using ConTileX = typename ConTileSel<T, VEC>::x;
template <typename T, bool VEC = true> using ConTileY = typename ConTileSel<T, VEC>::y;
template <typename T> using ConTileNX = typename ConTileSel<T, true>::nx;
template <typename T> using ConTileNY = typename ConTileSel<T, true>::ny;
template <typename T, bool VEC, bool SMALL> struct ConTileSmall {
  using x = ConTileX<T, VEC>;
  using y = ConTileY<T, VEC>;
};
template <bool VEC> struct ConTileSmall<float, VEC, true> {
  using x = TileD<64, 64, false, 2, 2, gdma::K_F32, 2, false, false, VEC ? 1 : 2, SMALL_STAGES>;
  using y = TileD<64, 64, true, 2, 2, gdma::K_F32, 2, false, false, VEC ? 1 : 2, SMALL_STAGES>;
};
// the 16-bit types keep one layout of the gradient-matrix blocks (G'^T)
template <typename T> struct GtOnly { static constexpr bool value = Is16<T>::value; };
// Scale of the stored gradient-matrix entries.  0 < G'_ij <= 2 (E_ij <= 1,
// E_ij / R_i <= 1, E_ij / C_j <= 1) and typical entries are ~1/N, which are
// fp16 subnormals from N ~ 2^14 on: fp16 stores 2^14 G' (at most 2^15, below
// the fp16 maximum 65504) and the contractions scale back by 2^-14 (exact).
template <typename T> struct GScale { static constexpr float value = 1.f; };
template <> struct GScale<_Float16> { static constexpr float value = 16384.f; };

// workgroups per CU the launch bounds promise (the 16-bit direct-load tiles
// use 96 KB of LDS or more: one per CU)
template <typename T, bool VEC> struct Occ {
  static constexpr int fwd = Is16<T>::value ? (VEC ? 1 : 2) : 2, bwd = Is16<T>::value ? (VEC ? 1 : 2) : 2;
};

// Operand of a tile core from a typed pointer (the 16-bit cores address bits)
template <class TL, typename T>
__device__ __forceinline__ typename TL::Op tile_op(const T* p, int64_t ld, int rows, int kmax) {
  return typename TL::Op{reinterpret_cast<const typename TL::Elem*>(p), ld, rows, kmax};
}

template <int A, int B> struct CMax { static constexpr int value = A > B ? A : B; };

// ---------------------------------------------------------------- forward
// E = exp2(S c - c) of this wave's TM x TN accumulators (S scaled by rx_i ry_j
// when NORM); rowv[bm * 16 + r] and colv[bn] collect this lane's partial row
// and column sums.  MASK zeroes the diagonal and entries outside [0, N).
// Eb (not null): every entry of the tile, masked ones as 0, is also stored at
// Eb[row * ldE + column] (tile-relative; each 32-lane half writes 128 bytes
// of one row); STORE_S stores the exponent's row-scaled similarity S_ij rx_i
// there instead (unmasked), from which E is exp2(s c ry_j - c) as here.
template <class TL, bool NORM, bool MASK, bool STORE_S = false>
__device__ __forceinline__ void sumexp_epilogue(const f32x16 (&acc)[TL::FM][TL::FN], float c, int m0, int n0, int N,
                                                const float* s_rx, const float* s_ry, float (&rowv)[TL::FM * 16],
                                                float (&colv)[TL::FN], float* __restrict__ Eb = nullptr,
                                                int ldE = 0) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w / TL::WN, wn = w % TL::WN;
  float sv[STORE_S ? TL::FN : 1][STORE_S ? TL::FM * 16 : 1];  // STORE_S: the similarities to store
#pragma unroll
  for (int k = 0; k < TL::FM * 16; ++k) rowv[k] = 0.f;
#pragma unroll
  for (int bn = 0; bn < TL::FN; ++bn) {
    const int nl = wn * TL::TN + bn * 32 + (lane & 31);
    const int j = n0 + nl;
    const float cy = NORM ? c * s_ry[nl] : c;
    float cs = 0.f;
#pragma unroll
    for (int bm = 0; bm < TL::FM; ++bm) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * TL::TM + bm * 32 + acc_row(r, lane);
        const int i = m0 + ml;
        const float sc = NORM ? acc[bm][bn][r] * s_rx[ml] : acc[bm][bn][r];
        float e = fast_exp2(fmaf(sc, cy, -c));
        if (MASK) e = (i < N && j < N && i != j) ? e : 0.f;
        if constexpr (STORE_S)
          sv[bn][bm * 16 + r] = sc;
        else if (Eb)
          Eb[(int64_t)ml * ldE + nl] = e;
        rowv[bm * 16 + r] += e;
        cs += e;
      }
    }
    colv[bn] = cs;
  }
  // STORE_S: the stores after every LDS read of the scales (a store through a
  // generic pointer may alias LDS, so each store interleaved with the reads
  // made the next read wait for it), at device scope (the next launch reads
  // them)
  if constexpr (STORE_S) {
#pragma unroll
    for (int bn = 0; bn < TL::FN; ++bn)
#pragma unroll
      for (int bm = 0; bm < TL::FM; ++bm)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          store_device(&Eb[(int64_t)(wm * TL::TM + bm * 32 + acc_row(r, lane)) * ldE + wn * TL::TN + bn * 32 +
                           (lane & 31)],
                       sv[bn][bm * 16 + r]);
  }
}

// Workgroup barrier for the epilogues' own LDS arrays: their LDS operations
// complete (lgkmcnt), then s_barrier.  __syncthreads() would also wait for the
// next tile's global->LDS loads in flight into the ring.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
  asm volatile("s_barrier" ::: "memory");
}

// Row and column sums of E over one tile: thread t gets the sums of row m0 + t
// (rs) and column n0 + t (cs), which sums_flush adds into ws.  rxv / ryv:
// 1/|x| of row m0 + t and 1/|y| of column n0 + t (NORM).
template <class TL, bool LIT, bool NORM, bool STORE_S = false>
__device__ __forceinline__ void sumexp_tile(const f32x16 (&acc)[TL::FM][TL::FN], float c, int m0, int n0, int N,
                                            float rxv, float ryv, float* s_rx, float* s_ry, float* s_row,
                                            float* s_col, float& rs_out, float& cs_out, float* __restrict__ Eb = nullptr,
                                            int ldE = 0, bool active = true) {
  static_assert(TL::NT >= TL::BM && TL::NT >= TL::BN, "one row and one column per thread");
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w / TL::WN, wn = w % TL::WN;
  if (t < TL::BM) {
    s_rx[t] = rxv;
    s_row[t] = 0.f;
  }
  if (t < TL::BN) {
    s_ry[t] = ryv;
    s_col[t] = 0.f;
  }
  lds_barrier();
  // (active: waves that hold accumulators; the others, k-group 1 of a split-k
  // tile, only take part in the barriers)
  if (active) {
    float rowv[TL::FM * 16];
    float colv[TL::FN];
    // interior tiles (no diagonal entry, no row or column beyond N) need no mask
    const bool diag = m0 < n0 + TL::BN && n0 < m0 + TL::BM;
    if (!diag && m0 + TL::BM <= N && n0 + TL::BN <= N)
      sumexp_epilogue<TL, NORM, false, STORE_S>(acc, c, m0, n0, N, s_rx, s_ry, rowv, colv, Eb, ldE);
    else
      sumexp_epilogue<TL, NORM, true, STORE_S>(acc, c, m0, n0, N, s_rx, s_ry, rowv, colv, Eb, ldE);
    if constexpr (TL::FM == 1) {
      // one 32-row block: its 16 row sums padded to the 32 of the reduction
      float v[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) v[k] = k < 16 ? rowv[k] : 0.f;
      const float rs = transpose_reduce32(v, lane);
      const int q = lane & 31;
      if (q < 16)
        __hip_atomic_fetch_add(&s_row[wm * TL::TM + acc_row(q, lane)], rs, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
#pragma unroll
      for (int h = 0; h < TL::FM / 2; ++h) {
        const float rs = transpose_reduce32(*reinterpret_cast<float(*)[32]>(&rowv[32 * h]), lane);
        const int q = lane & 31;
        const int ml = wm * TL::TM + h * 64 + (q >> 4) * 32 + acc_row(q & 15, lane);
        __hip_atomic_fetch_add(&s_row[ml], rs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    if (!LIT) {
#pragma unroll
      for (int bn = 0; bn < TL::FN; ++bn) {
        colv[bn] += __shfl_xor(colv[bn], 32, 64);
        if (lane < 32)
          __hip_atomic_fetch_add(&s_col[wn * TL::TN + bn * 32 + lane], colv[bn], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  }
  lds_barrier();
  rs_out = t < TL::BM ? s_row[t] : 0.f;
  cs_out = (!LIT && t < TL::BN) ? s_col[t] : 0.f;
}
template <class TL, bool LIT>
__device__ __forceinline__ void sums_flush(float* __restrict__ ws, int m0, int n0, int N, float rs, float cs) {
  const int64_t n64 = N;
  const int t = threadIdx.x;
  if (t < TL::BM && m0 + t < N)
    __hip_atomic_fetch_add(&ws[WS_ROW_OFF * n64 + m0 + t], rs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (!LIT && t < TL::BN && n0 + t < N)
    __hip_atomic_fetch_add(&ws[WS_COL_OFF * n64 + n0 + t], cs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Forward tiles that chain (FwdChain): the 16-bit direct-to-LDS tiles
// without the norm scaling, which always take the deterministic forward's
// block walk (k_sumexp_det) with chained tiles.  Measured: the 16-bit forward
// (one workgroup per CU, nothing else to overlap its epilogue) is 7% faster
// chained, and the block walk with its fixed-order sums another 2-7% faster
// than chained tiles with atomic sums; fp32 (two workgroups per CU, one's
// epilogue already overlaps the other's k-loop) was 4% slower chained; the
// normalizing 16-bit epilogue spills registers in the chained loop, or is
// slower when kept from spilling.
template <typename T, bool VEC, bool NORM> struct FwdChain {
  static constexpr bool value = FwdTile<T, VEC>::CHAIN && Is16<T>::value && !NORM;
};

// Forward sums with relaxed atomics into ws (as the reference,
// clip_loss.py:63-64): one tile per workgroup of the tiles_m x tiles_n grid
// (XCD-grouped order).  The chain-eligible 16-bit tiles (FwdChain) run
// k_sumexp_det instead.
template <typename T, bool LIT, bool NORM, bool VEC, bool SMALL = false>
__global__ __launch_bounds__((GemmTile<T, VEC, SMALL>::NT), (Occ<T, VEC>::fwd)) void k_sumexp(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ldy, int N, int D, int kmax, float c,
    float* __restrict__ ws, int tiles_m, int tiles_n) {
  using TL = GemmTile<T, VEC, SMALL>;
  static_assert(TL::FM % 2 == 0 || TL::FM == 1, "the row reduction takes 64-row halves of the wave sub-tile");
  __shared__ __attribute__((aligned(1024))) char lds[TL::LDS_BYTES];
  __shared__ float s_rx[TL::BM], s_ry[TL::BN], s_row[TL::BM], s_col[TL::BN];
  const int64_t n64 = N;
  const int t = threadIdx.x;
  int tm, tn;
  tile_swizzle(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, 8, tm, tn);
  const int m0 = tm * TL::BM, n0 = tn * TL::BN;
  f32x16 acc[TL::FM][TL::FN];
  TL::template run<VEC, VEC>(tile_op<TL>(X + (int64_t)m0 * ldx, ldx, min(N - m0, TL::BM), kmax),
                             tile_op<TL>(Y + (int64_t)n0 * ldy, ldy, min(N - n0, TL::BN), kmax), D, lds, acc);
  // the norms after the k-loop: loaded before it, they cost the fp32 forward
  // 4% (17.30 -> 18.02 ms at the headline shape)
  const float rxv = (NORM && t < TL::BM && m0 + t < N) ? ws[WS_RX * n64 + m0 + t] : 1.f;
  const float ryv = (NORM && t < TL::BN && n0 + t < N) ? ws[WS_RY * n64 + n0 + t] : 1.f;
  float rs, cs;
  sumexp_tile<TL, LIT, NORM>(acc, c, m0, n0, N, rxv, ryv, s_rx, s_ry, s_row, s_col, rs, cs);
  sums_flush<TL, LIT>(ws, m0, n0, N, rs, cs);
}

// ------------------------------------------------- deterministic forward
// The sums without atomics across workgroups, in one pass over the tiles.
// The tile grid is cut into P x Q blocks (P <= DET_P row blocks, Q <= DET_Q
// column blocks, both clamped to the tile counts); workgroup (p, q) walks its
// block, row tiles outer and column tiles inner, in order.  Within a tile:
//   rows: each lane's row sums over its columns (registers, fixed order),
//     transpose_reduce32 across the half-wave, one LDS slot per (wave column,
//     row) with one writer; thread t adds the slots in wave order to its
//     running sum of row m0 + t over the block's column tiles, and writes it
//     to rowpart[q * N + row] after the last one;
//   columns (CLIP): each lane's column sums over its rows, plus the other
//     lane half, one LDS slot per (wave row, column); thread t adds the slots
//     in wave order and adds that to colpart[p * N + column] (written at the
//     block's first row tile; only this workgroup touches these entries).
// k_det_reduce then sums the Q row partials and the P column partials of each
// index in order.  Every sum is a fixed function of the inputs and of the
// tile shape, E is computed once, and the partials take (DET_P + DET_Q) * N
// floats of the workspace.
template <typename T, bool LIT, bool NORM, bool VEC>
__global__ __launch_bounds__((FwdTile<T, VEC>::NT), (Occ<T, VEC>::fwd)) void k_sumexp_det(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ldy, int N, int D, int kmax, float c,
    const float* __restrict__ rx, const float* __restrict__ ry, float* __restrict__ rowpart,
    float* __restrict__ colpart, int tiles_m, int tiles_n, int P, int Q) {
  using TL = FwdTile<T, VEC>;
  static_assert(TL::FM == 2, "row reduction assumes 64-row wave sub-tiles");
  static_assert(TL::WN == 2, "two row-sum slots per row");
  static_assert(TL::NT >= TL::BM && TL::NT >= TL::BN, "one row and one column per thread");
  __shared__ __attribute__((aligned(1024))) char lds[TL::LDS_BYTES];
  __shared__ float s_rx[TL::BM], s_ry[TL::BN], s_row[TL::WN][TL::BM], s_col[TL::WM][TL::BN];
  __shared__ __attribute__((aligned(16))) float s_cold[TL::BN];
  const int nbm = tiles_m / P, rbm = tiles_m % P, nbn = tiles_n / Q, rbn = tiles_n % Q;
  // Workgroup -> block.  Even blocks (no remainder tiles): XCD x = blockIdx % 8
  // takes row blocks [x P/8, (x+1) P/8) against every column block, its first
  // dispatched workgroups the low half of the column blocks, so that the
  // concurrent workgroups of one XCD share 4 x-panel and 8 y-panel streams.
  // Otherwise neighbouring ids (one XCD) share a row block, and the first
  // tiles_m % P row blocks and tiles_n % Q column blocks, which take one tile
  // more, are the first dispatched, so the longer workgroups start early.
  // Measured (forward, same box): even blocks 2% faster at 65536 x 768 and
  // 262144 x 1152 with the first mapping; with remainder tiles 2% faster at
  // 65792 and 66000 rows with the second.  The partition, and so every sum,
  // is the same either way.
  int p, q;
  if (rbm == 0 && rbn == 0 && P % 8 == 0 && (int)gridDim.x == P * Q) {
    const int x = blockIdx.x & 7, j = blockIdx.x >> 3, pr = P / 8;
    p = x * pr + j % pr;
    q = j / pr;
  } else {
    const int pid = xcd_remap(blockIdx.x, gridDim.x);
    p = pid / Q;
    q = pid - p * Q;
  }
  const int tm0 = p * nbm + min(p, rbm), tm1 = tm0 + nbm + (p < rbm ? 1 : 0);
  const int tn0 = q * nbn + min(q, rbn), tn1 = tn0 + nbn + (q < rbn ? 1 : 0);
  const int64_t n64 = N;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w / TL::WN, wn = w % TL::WN;
  // the row (within the tile) whose slot this lane owns after transpose_reduce32
  const int qr = lane & 31;
  const int my_row = wm * TL::TM + (qr >> 4) * 32 + acc_row(qr & 15, lane);
  auto op_a = [&](int tm) {
    const int m0 = tm * TL::BM;
    return tile_op<TL>(X + (int64_t)m0 * ldx, ldx, min(N - m0, TL::BM), kmax);
  };
  auto op_b = [&](int tn) {
    const int n0 = tn * TL::BN;
    return tile_op<TL>(Y + (int64_t)n0 * ldy, ldy, min(N - n0, TL::BN), kmax);
  };
  // tile (tm, tn) of the block: its sums into the slots, then thread t's row
  // sum into rs and its column partial into colpart (cold: the partial so far
  // was prefetched into s_cold)
  auto tile_sums = [&](const f32x16 (&acc)[TL::FM][TL::FN], int tm, int tn, float& rs, bool cold = false) {
    const int m0 = tm * TL::BM, n0 = tn * TL::BN;
    float rowv[TL::FM * 16];
    float colv[TL::FN];
    const bool diag = m0 < n0 + TL::BN && n0 < m0 + TL::BM;
    if (!diag && m0 + TL::BM <= N && n0 + TL::BN <= N)
      sumexp_epilogue<TL, NORM, false>(acc, c, m0, n0, N, s_rx, s_ry, rowv, colv);
    else
      sumexp_epilogue<TL, NORM, true>(acc, c, m0, n0, N, s_rx, s_ry, rowv, colv);
    s_row[wn][my_row] = transpose_reduce32(rowv, lane);
    if (!LIT) {
#pragma unroll
      for (int bn = 0; bn < TL::FN; ++bn) {
        const float v = colv[bn] + __shfl_xor(colv[bn], 32, 64);
        if (lane < 32) s_col[wm][wn * TL::TN + bn * 32 + lane] = v;
      }
    }
    lds_barrier();
    if (t < TL::BM) rs += s_row[0][t] + s_row[1][t];
    if (!LIT && t < TL::BN && n0 + t < N) {
      float v = s_col[0][t];
#pragma unroll
      for (int k = 1; k < TL::WM; ++k) v += s_col[k][t];
      float* cp = colpart + (int64_t)p * n64 + n0 + t;
      *cp = tm == tm0 ? v : (cold ? s_cold[t] : *cp) + v;
    }
  };
  if constexpr (FwdChain<T, VEC, NORM>::value) {
    // chained tiles (no norm scaling: s_rx, s_ry unused): the last chunk of
    // each tile's k-loop loads chunk 0 of the next, which lands during the
    // epilogue.  The k-loop's barriers order one tile's slot reads before the
    // next tile's slot writes.
    const int ntn = tn1 - tn0, K = (tm1 - tm0) * ntn;
    if (K <= 0) return;
    // The column partials a tile adds to (written at an earlier row tile) reach
    // s_cold by direct loads issued after the tile's first barrier; the next
    // chunk's barrier awaits every load, so they have landed by the epilogue.
    // With a single k-chunk there is no such barrier: the partials are read
    // from global memory in the epilogue instead.
    const bool pf = !LIT && D > TL::G::BK;
    typename TL::Plan lp;
    TL::start(op_a(tm0), op_b(tn0), lds, lp);
    int p0 = 0;
    float rs = 0.f;  // thread t: row tm * BM + t over this block's column tiles
    for (int k = 0; k < K; ++k) {
      const int tm = tm0 + k / ntn, tn = tn0 + k % ntn;
      const bool has_next = k + 1 < K;
      const int tmn = has_next ? tm0 + (k + 1) / ntn : tm, tnn = has_next ? tn0 + (k + 1) % ntn : tn;
      auto hook = [&] {
        if (pf && tm > tm0 && w < TL::BN / 64) {
          const int n0 = tn * TL::BN;
          const __amdgpu_buffer_rsrc_t r =
              __builtin_amdgcn_make_buffer_rsrc((void*)(colpart + (int64_t)p * n64 + n0), 0, (N - n0) * 4, 0x00020000);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)&s_cold[w * 64], 4,
                                                   (uint32_t)(w * 64 + lane) * 4, 0, 0, 0);
        }
      };
      f32x16 acc[TL::FM][TL::FN];
      TL::chain(lp, op_a(tmn), op_b(tnn), has_next, D, lds, p0, acc, hook);
      tile_sums(acc, tm, tn, rs, pf);
      if (tn == tn1 - 1) {
        if (t < TL::BM && tm * TL::BM + t < N) rowpart[(int64_t)q * n64 + tm * TL::BM + t] = rs;
        rs = 0.f;
      }
    }
    gdma::drain_loads();
  } else {
    for (int tm = tm0; tm < tm1; ++tm) {
      const int m0 = tm * TL::BM;
      const auto A = op_a(tm);
      float rs = 0.f;  // thread t: row m0 + t over this block's column tiles
      for (int tn = tn0; tn < tn1; ++tn) {
        const int n0 = tn * TL::BN;
        __syncthreads();  // the previous tile's epilogue is done with the LDS stages and slots
        if (t < TL::BM) s_rx[t] = (NORM && m0 + t < N) ? rx[m0 + t] : 1.f;
        if (t < TL::BN) s_ry[t] = (NORM && n0 + t < N) ? ry[n0 + t] : 1.f;
        f32x16 acc[TL::FM][TL::FN];
        TL::template run<VEC, VEC>(A, op_b(tn), D, lds, acc);  // its first barrier publishes s_rx, s_ry
        tile_sums(acc, tm, tn, rs);
      }
      if (t < TL::BM && m0 + t < N && tn1 > tn0) rowpart[(int64_t)q * n64 + m0 + t] = rs;
    }
  }
}

// out_row[i] = sum over q < Q of rowpart[q * N + i] and (CLIP) out_col[i] =
// sum over p < P of colpart[p * N + i], each in that order
template <bool LIT>
__global__ __launch_bounds__(256) void k_det_reduce(const float* __restrict__ rowpart, int Q,
                                                    const float* __restrict__ colpart, int P, int N,
                                                    float* __restrict__ out_row, float* __restrict__ out_col) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  const int64_t n64 = N;
  float v = 0.f;
  for (int k = 0; k < Q; ++k) v += rowpart[k * n64 + i];
  out_row[i] = v;
  if (!LIT) {
    float u = 0.f;
    for (int k = 0; k < P; ++k) u += colpart[k * n64 + i];
    out_col[i] = u;
  }
}

// ---------------------------------------------------------------- backward
// Block decomposition of the N x N gradient matrix: nb blocks of bs rows
// (bs a multiple of block_quantum; the last block may be short).  Diagonal s
// pairs block I with block J = (I + s) mod nb, so one diagonal touches every
// block row and every block column exactly once.
struct BlockGrid {
  int bs;    // block size (rows)
  int nb;    // number of blocks (= number of diagonals)
  int gtm;   // gradient-matrix tiles per block, row direction (bs / BM)
  int gtn;   // gradient-matrix tiles per block, column direction (bs / BN)
  int ctm;   // contraction tiles per block, row direction (bs / BM of the contraction)
  int ctd;   // contraction tiles over the features (ceil(D / BN of the contraction, 256 or 384); with cnw,
             // floor(D / 256))
  int cnw;   // 16-bit, D % 256 in [1, 128], ctm even: the features past ctd * 256 are contracted by narrow
             // tiles of 512 rows (ConTileNX / ConTileNY), one per pair of row tiles
};

// Scratch of the backward (all in the input dtype T, row-major):
//   G[2]   two buffers of nb blocks of bs x bs: block I of buffer s&1 holds
//          G'(I, (I+s) mod nb) of diagonal s (fp32 only);
//   GT[2]  the same blocks transposed (fp32: CLIP only, row-major; 16-bit:
//          always, the only copy, in the blocked layout gdma::gb_offset);
//   XT, YT the normalised inputs transposed, [D][ldt] with ldt = N rounded
//          up to 128 and zero columns [N, ldt): element (d, i) = rx_i x_i[d].
// Every contraction operand is then K-major (k contiguous).  The bf16x3 mode
// keeps GT, XT and YT as bf16 hi planes (gt, xt, yt) and lo planes (gt_lo,
// xt_lo, yt_lo), all null otherwise.
struct GradBufs {
  void* g[2];
  void* gt[2];
  const void* xt;
  const void* yt;
  int64_t ldt;
  void* gt_lo[2];
  const void* xt_lo;
  const void* yt_lo;
};

// One pipeline step of the backward (launch t = 0 .. nb):
//   workgroups [0, cx_pad)               x side of the contraction of diagonal t-1
//   [cx_pad, cx_pad + cy_pad)            y side (CLIP)
//   [cx_pad + cy_pad, ... + g_pad)       G' tiles of diagonal t
// The long contraction tiles (K = bs) come first so the short G' tiles
// (K = d) fill the tail of the launch.  Each sub-range starts at a multiple
// of 8, so `id % 8` is still the XCD a workgroup runs on.
struct StepPlan {
  int diag_g;        // diagonal whose G' this launch writes (-1: none)
  int diag_c;        // diagonal this launch contracts (-1: none)
  int accumulate;    // contraction adds to the accumulators (else overwrites)
  int g_n, g_pad;    // G' tiles (nb * gtm * gtn or 0), padded to a multiple of 8
  int cx_n, cx_pad;  // x-side contraction tiles (nb * ctm * ctd; cnw: nb * ctm / 2 * (2 ctd + 1); or 0), padded
  int cy_n, cy_pad;  // y-side contraction tiles, padded
};

// fp32 gradient-matrix tile: H_ij = rx_i G'_ij ry_j (G'_ij without the norm
// scaling, NORM = false) of this wave's TM x TN accumulators, row-major at Gb
// with row pitch bs (scalar stores, coalesced across lanes).  Stored once:
// the x side's contraction reads its rows, the y side's reads it transposed,
// and both multiply it with the raw inputs (the norms are in H).  MASK zeroes
// the diagonal and entries outside [0, N).
template <class TL, bool LIT, bool NORM, bool MASK>
__device__ __forceinline__ void grad_g_store(const f32x16 (&acc)[TL::FM][TL::FN], float c, int i0, int j0, int N,
                                             float* __restrict__ Gb, int bs, const float* s_rx, const float* s_ry,
                                             const float* s_ir, const float* s_ic) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w / TL::WN, wn = w % TL::WN;
#pragma unroll
  for (int bm = 0; bm < TL::FM; ++bm) {
#pragma unroll
    for (int bn = 0; bn < TL::FN; ++bn) {
      const int nl = wn * TL::TN + bn * 32 + (lane & 31);
      const int j = j0 + nl;
      const float ryj = NORM ? s_ry[nl] : 1.f;
      const float cy = c * ryj;
      const float icj = s_ic[nl];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * TL::TM + bm * 32 + acc_row(r, lane);
        const int i = i0 + ml;
        const float rxi = NORM ? s_rx[ml] : 1.f;
        const float e = fast_exp2(fmaf(acc[bm][bn][r] * rxi, cy, -c));
        float g = LIT ? e * s_ir[ml] : e * (s_ir[ml] + icj);
        if (NORM) g *= rxi * ryj;
        if (MASK) g = (i < N && j < N && i != j) ? g : 0.f;
        Gb[(int64_t)ml * bs + nl] = g;
      }
    }
  }
}

// 16-bit gradient-matrix tiles (k_grad_g_chain and k_grad_step): G'^T
// straight from the accumulators into the
// tile's blocks at GTb (blocked layout, gdma::gb_offset), no staging.  GSC:
// the storage scale, when s_ir / s_ic do not already carry it.  For a 32 x 32 accumulator block, register
// group g4 of lane l holds rows i = 8 g4 + 4 (l / 32) .. + 3 of column
// j = l % 32; swapping groups 2p + 1 of the low lane half with groups 2p of
// the high half (v_permlane32_swap) leaves lane l with the 8 rows
// 16 p + 8 (l / 32) .. + 7, i.e. slot (l % 32, l / 32) of i-block p: every
// 16-byte store of the wave writes one whole 1 KB block, 16 per lane and tile.
template <class TL>
constexpr int gt_chain_stores() {
  return TL::FM * TL::FN * 2;
}
// X3 (bf16x3): a second plane bf16(G' - bf16(G')) at GTl, the same way.
template <class TL, bool LIT, bool NORM, bool MASK, int GSC, bool X3 = false>
__device__ __forceinline__ void grad_gt_store_direct(const f32x16 (&acc)[TL::FM][TL::FN], float c, int i0, int j0,
                                                     int N, uint16_t* __restrict__ GTb, int bs, const float* s_rx,
                                                     const float* s_ry, const float* s_ir, const float* s_ic,
                                                     uint16_t* __restrict__ GTl = nullptr) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr int NP = X3 ? 2 : 1;  // planes
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w / TL::WN, wn = w % TL::WN;
  const int64_t rowb = (int64_t)(bs >> 4) * 512;  // elements per row of blocks
  // Non-temporal stores through buffer descriptors at the tile's planes (the
  // write-once G'^T should not displace the operand panels from the caches).
  // __builtin_nontemporal_store lost its hint in this function for the
  // one-plane case (no nt bit in the stores); the buffer store's cache-policy
  // operand (2: nt) keeps it.  A tile's offsets stay below 8 * bs * 64 bytes.
  const __amdgpu_buffer_rsrc_t rs_hi = __builtin_amdgcn_make_buffer_rsrc((void*)GTb, 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_lo =
      __builtin_amdgcn_make_buffer_rsrc((void*)(X3 ? GTl : GTb), 0, 0x7fffffff, 0x00020000);
#pragma unroll
  for (int bn = 0; bn < TL::FN; ++bn) {
    const int nl = wn * TL::TN + bn * 32 + (lane & 31);
    const int j = j0 + nl;
    const float cy = NORM ? c * s_ry[nl] : c;
    const float icj = s_ic[nl];
    const int64_t jrow = ((wn * TL::TN + bn * 32) >> 5) * rowb;
#pragma unroll
    for (int bm = 0; bm < TL::FM; ++bm) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        uint32_t pk[NP][2][2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float gv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * (2 * p + q) + e;
            const int ml = wm * TL::TM + bm * 32 + acc_row(r, lane);
            const int i = i0 + ml;
            const float sc = NORM ? acc[bm][bn][r] * s_rx[ml] : acc[bm][bn][r];
            const float ex = fast_exp2(fmaf(sc, cy, -c));
            float g = LIT ? ex * s_ir[ml] : ex * (s_ir[ml] + icj);
            if (GSC != 1) g *= (float)GSC;  // storage scale (exact: a power of two)
            if (MASK) g = (i < N && j < N && i != j) ? g : 0.f;
            gv[e] = g;
          }
          pk[0][q][0] = TL::pack2(gv[0], gv[1]);
          pk[0][q][1] = TL::pack2(gv[2], gv[3]);
          if constexpr (X3) {
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[e] -= bf16_to_f32(f32_to_bf16(gv[e]));
            pk[NP - 1][q][0] = TL::pack2(gv[0], gv[1]);
            pk[NP - 1][q][1] = TL::pack2(gv[2], gv[3]);
          }
        }
        const int ib = (wm * TL::TM + bm * 32) / 16 + p;
        const int64_t off = jrow + ib * 512 + gdma::gb_slot(lane & 31, lane >> 5, p) * 8;
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) {
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const auto sw = __builtin_amdgcn_permlane32_swap(pk[pl][0][d], pk[pl][1][d], false, false);
            pk[pl][0][d] = sw[0];
            pk[pl][1][d] = sw[1];
          }
          const u32x4 u = u32x4{pk[pl][0][0], pk[pl][0][1], pk[pl][1][0], pk[pl][1][1]};
          __builtin_amdgcn_raw_buffer_store_b128(u, pl ? rs_lo : rs_hi, (uint32_t)(off * 2), 0, 2);
        }
      }
    }
  }
}

// Recompute the similarity tile (i0, j0) and store G'_ij = E_ij (1/R_i + 1/C_j)
// (LiT: E_ij / R_i) for i != j, 0 on the diagonal and outside [0, N): fp32
// scaled by the norms (H, grad_g_store) into the block at Gb (row pitch bs);
// the 16-bit types transposed at GTb in the blocked layout (X3: its bf16 hi
// plane at GTb and lo plane at GTl).
// Follows clip_loss.py:96-124 / lit_loss.py:94-120.
template <class TL, typename T, bool LIT, bool NORM, bool VEC, bool X3>
__device__ __forceinline__ void grad_g_tile(const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y,
                                            int64_t ldy, int N, int D, int kmax, float c, const float* __restrict__ ws,
                                            T* __restrict__ Gb, T* __restrict__ GTb, T* __restrict__ GTl, int bs,
                                            int i0, int j0, char* lds, float* s_rx, float* s_ry, float* s_ir,
                                            float* s_ic) {
  const int64_t n64 = N;
  const int t = threadIdx.x;
  const auto A = tile_op<TL>(X + (int64_t)i0 * ldx, ldx, min(N - i0, TL::BM), kmax);
  const auto B = tile_op<TL>(Y + (int64_t)j0 * ldy, ldy, min(N - j0, TL::BN), kmax);
  f32x16 acc[TL::FM][TL::FN];
  TL::template run<VEC, VEC>(A, B, D, lds, acc);
  // 1/R_i and 1/C_j carry the storage scale of G' (a power of two: exact)
  constexpr float GS = GScale<T>::value;
  for (int u = t; u < TL::BM; u += TL::NT) {
    const bool ok = i0 + u < N;
    s_rx[u] = (NORM && ok) ? ws[WS_RX * n64 + i0 + u] : 1.f;
    s_ir[u] = ok ? GS * ws[WS_INV_ROW * n64 + i0 + u] : 0.f;
  }
  for (int u = t; u < TL::BN; u += TL::NT) {
    const bool ok = j0 + u < N;
    s_ry[u] = (NORM && ok) ? ws[WS_RY * n64 + j0 + u] : 1.f;
    s_ic[u] = (!LIT && ok) ? GS * ws[WS_INV_COL * n64 + j0 + u] : 0.f;
  }
  __syncthreads();
  const bool diag = i0 < j0 + TL::BN && j0 < i0 + TL::BM;
  if constexpr (X3) {
    static_assert(std::is_same<T, uint16_t>::value, "bf16x3 runs on bf16 split operands");
    if (!diag && i0 + TL::BM <= N && j0 + TL::BN <= N)
      grad_gt_store_direct<TL, LIT, NORM, false, 1, true>(acc, c, i0, j0, N, GTb, bs, s_rx, s_ry, s_ir, s_ic, GTl);
    else
      grad_gt_store_direct<TL, LIT, NORM, true, 1, true>(acc, c, i0, j0, N, GTb, bs, s_rx, s_ry, s_ir, s_ic, GTl);
  } else if constexpr (GtOnly<T>::value) {
    // (s_ir, s_ic carry the storage scale)
    if (!diag && i0 + TL::BM <= N && j0 + TL::BN <= N)
      grad_gt_store_direct<TL, LIT, NORM, false, 1>(acc, c, i0, j0, N, (uint16_t*)GTb, bs, s_rx, s_ry, s_ir, s_ic);
    else
      grad_gt_store_direct<TL, LIT, NORM, true, 1>(acc, c, i0, j0, N, (uint16_t*)GTb, bs, s_rx, s_ry, s_ir, s_ic);
  } else {
    if (!diag && i0 + TL::BM <= N && j0 + TL::BN <= N)
      grad_g_store<TL, LIT, NORM, false>(acc, c, i0, j0, N, (float*)Gb, bs, s_rx, s_ry, s_ir, s_ic);
    else
      grad_g_store<TL, LIT, NORM, true>(acc, c, i0, j0, N, (float*)Gb, bs, s_rx, s_ry, s_ir, s_ic);
  }
}

// One BM x BN output tile of a contraction: rows r0.. of block P, feature
// columns d0..:
//   x side: acc_x[i, d] (+)= sum_{j in Q} G'(P,Q)[i, j]  * YT[d, j]   (Q = P + s)
//           (16-bit: G'(P,Q)[i, j] read from the transposed block G'T(P,Q)[j, i])
//   y side: acc_y[j, d] (+)= sum_{i in Q} G'T(Q,P)[j, i] * XT[d, i]   (Q = P - s)
// fp32 (TC::TB): the blocks hold H = diag(rx) G' diag(ry) and OT is the raw
// input of the other side, read by rows (element (k, d) at OT[k * ldt + d]):
//   x side: acc_x[i, d] (+)= sum_j H(P,Q)[i, j] y[q0 + j, d] = rx_i (G' Y^)[i, d]
//   y side: acc_y[j, d] (+)= sum_i H(Q,P)[i, j] x[q0 + i, d] = ry_j (G'^T X^)[j, d]
// (the post-pass takes the row's norm factor out again).
// Each output tile has one owner per launch: accumulation across launches
// adds each element once per launch, in launch order (the reference instead
// lets every (row-tile, column-tile) program add into dX/dY with contending
// atomics, clip_loss.py:148-156).
// X3 (bf16x3): Gblk/OT are the hi planes and Glo/OTlo the lo planes; the
// tile is hi.hi + hi.lo + lo.hi, three passes over K into one accumulator.
template <class TC, typename T, bool X3 = false>
__device__ __forceinline__ void grad_contract_tile(int N, int D, const T* __restrict__ Gblk,
                                                   const T* __restrict__ Glo, const T* __restrict__ OT,
                                                   const T* __restrict__ OTlo, int64_t ldt, const BlockGrid& bg,
                                                   int P, int Q, int tm, int td, bool accumulate,
                                                   float* __restrict__ out, char* lds) {
  const int r0 = P * bg.bs + tm * TC::BM;
  if (r0 >= N) return;
  const int d0 = td * TC::BN;
  const int q0 = Q * bg.bs;
  const int qn = min(bg.bs, N - q0);
  // entries of G' and XT/YT at k in [qn, round8(qn)) are stored zeros
  const int kq = (qn + 7) & ~7;
  // A: rows tm*BM.. of the block (K-major), or columns tm*BM.. of a transposed
  // block (blocked layout: i-block tm*BM/16 of the first j-block row)
  const int64_t a_off = TC::TA ? (int64_t)(tm * TC::BM) * (TC::GB ? 32 : 1) : (int64_t)(tm * TC::BM) * bg.bs;
  const auto A = tile_op<TC>(Gblk + a_off, bg.bs, TC::BM, kq);
  // the feature operand: transposed copy (rows d, k = q0 + j) or, fp32, the
  // raw rows q0 + k (only the block's qn valid rows)
  const int64_t b_off = TC::TB ? (int64_t)q0 * ldt + d0 : (int64_t)d0 * ldt + q0;
  const auto B = tile_op<TC>(OT + b_off, ldt, min(D - d0, TC::BN), TC::TB ? qn : kq);
  f32x16 acc[TC::FM][TC::FN];
  TC::template run<true, true>(A, B, kq, lds, acc);
  if constexpr (X3) {
    __syncthreads();  // every wave is past its last read of the ring
    TC::template run<true, true, false>(A, tile_op<TC>(OTlo + b_off, ldt, min(D - d0, TC::BN), kq), kq, lds, acc);
    __syncthreads();
    TC::template run<true, true, false>(tile_op<TC>(Glo + a_off, bg.bs, TC::BM, kq), B, kq, lds, acc);
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w / TC::WN, wn = w % TC::WN;
#pragma unroll
  for (int bm = 0; bm < TC::FM; ++bm) {
#pragma unroll
    for (int bn = 0; bn < TC::FN; ++bn) {
      const int d = d0 + wn * TC::TN + bn * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = r0 + wm * TC::TM + bm * 32 + acc_row(r, lane);
        if (row < N && d < D) {
          float* p = out + (int64_t)row * D + d;
          // a fire-and-forget add in L2 instead of a load-add-store round trip;
          // the tile has one owner per launch, so the summation order (launch
          // order) and the result are deterministic
          const float v = acc[bm][bn][r] * (1.f / GScale<T>::value);
          if (accumulate)
            __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            *p = v;
        }
      }
    }
  }
}

// Contraction workgroup `sub` (in [0, cx_pad + cy_pad)) of one pipeline step.
// TNX / TNY: the narrow tiles (bg.cnw).
// X, Y: the raw inputs (fp32: the feature operands of the contractions).
template <class TCX, class TCY, class TNX, class TNY, typename T, bool X3 = false>
__device__ __forceinline__ void grad_contract_dispatch(int sub, int N, int D, const GradBufs& gb, const BlockGrid& bg,
                                                       const StepPlan& sp, float* __restrict__ acc_x,
                                                       float* __restrict__ acc_y, char* lds, const T* X = nullptr,
                                                       int64_t ldx = 0, const T* Y = nullptr, int64_t ldy = 0) {
  const int64_t blk = (int64_t)bg.bs * bg.bs;  // elements per G' block
  const bool is_x = sub < sp.cx_pad;
  if (!is_x) sub -= sp.cx_pad;
  const int pid = xcd_remap(sub, is_x ? sp.cx_pad : sp.cy_pad);
  if (pid >= (is_x ? sp.cx_n : sp.cy_n)) return;
  int tmg, td, rows = bg.ctm;  // rows: row tiles per block of this tile's height
  bool narrow = false;
  if constexpr (GtOnly<T>::value) {
    // 16-bit: feature tiles fastest, so the tiles sharing one gradient-matrix
    // panel run side by side on one XCD and the panel is fetched from HBM
    // about once (its contractions are bound by that traffic)
    if (bg.cnw) {
      // per pair of row tiles: the wide tiles of both, then the narrow tile
      // of their 512 rows (feature tile 2 ctd of 128 features)
      const int per = 2 * bg.ctd + 1;
      const int grp = pid / per, u = pid - grp * per;
      if (u == 2 * bg.ctd) {
        narrow = true;
        tmg = grp;
        td = 2 * bg.ctd;
        rows = bg.ctm / 2;
      } else {
        tmg = 2 * grp + u / bg.ctd;
        td = u - (u / bg.ctd) * bg.ctd;
      }
    } else {
      tmg = pid / bg.ctd;
      td = pid - tmg * bg.ctd;
    }
  } else {
    group_tile(pid, bg.nb * bg.ctm, bg.ctd, 8, tmg, td);
  }
  const int P = tmg / rows, tm = tmg - P * rows;  // P: block owning the output rows
  const int buf = sp.diag_c & 1;
  if (is_x) {
    const int Q = (P + sp.diag_c) % bg.nb;
    const T* gx = (const T*)(GtOnly<T>::value ? gb.gt[buf] : gb.g[buf]) + P * blk;
    const T* gxl = X3 ? (const T*)gb.gt_lo[buf] + P * blk : nullptr;
    if (narrow)
      grad_contract_tile<TNX, T, X3>(N, D, gx, gxl, (const T*)gb.yt, (const T*)gb.yt_lo, gb.ldt, bg, P, Q, tm, td,
                                     sp.accumulate != 0, acc_x, lds);
    else if constexpr (TCX::TB)
      grad_contract_tile<TCX, T, X3>(N, D, gx, gxl, Y, nullptr, ldy, bg, P, Q, tm, td, sp.accumulate != 0, acc_x,
                                     lds);
    else
      grad_contract_tile<TCX, T, X3>(N, D, gx, gxl, (const T*)gb.yt, (const T*)gb.yt_lo, gb.ldt, bg, P, Q, tm, td,
                                     sp.accumulate != 0, acc_x, lds);
  } else {
    const int Q = (P - sp.diag_c + bg.nb) % bg.nb;
    const T* gy = (const T*)(GtOnly<T>::value ? gb.gt[buf] : gb.g[buf]) + Q * blk;
    const T* gyl = X3 ? (const T*)gb.gt_lo[buf] + Q * blk : nullptr;
    if (narrow)
      grad_contract_tile<TNY, T, X3>(N, D, gy, gyl, (const T*)gb.xt, (const T*)gb.xt_lo, gb.ldt, bg, P, Q, tm, td,
                                     sp.accumulate != 0, acc_y, lds);
    else if constexpr (TCY::TB)
      grad_contract_tile<TCY, T, X3>(N, D, gy, gyl, X, nullptr, ldx, bg, P, Q, tm, td, sp.accumulate != 0, acc_y,
                                     lds);
    else
      grad_contract_tile<TCY, T, X3>(N, D, gy, gyl, (const T*)gb.xt, (const T*)gb.xt_lo, gb.ldt, bg, P, Q, tm, td,
                                     sp.accumulate != 0, acc_y, lds);
  }
}

// 16-bit (and bf16x3) contractions of one pipeline step (the x side of
// diagonal diag_c, then the y side).
// W: the 256 x 384 tiles (ConTileSel::wx / wy; no narrow tiles)
template <typename T, bool X3 = false, bool W = false>
__global__ __launch_bounds__(ConTileX<T>::NT, 1) void k_grad_contract(int N, int D, GradBufs gb, BlockGrid bg,
                                                                     StepPlan sp, float* __restrict__ acc_x,
                                                                     float* __restrict__ acc_y) {
  using Sel = ConTileSel<T, true>;
  using TCX = typename std::conditional<W, typename Sel::wx, typename Sel::x>::type;
  using TCY = typename std::conditional<W, typename Sel::wy, typename Sel::y>::type;
  using TNX = typename std::conditional<W, TCX, typename Sel::nx>::type;
  using TNY = typename std::conditional<W, TCY, typename Sel::ny>::type;
  static_assert(TCX::BM == TCY::BM && TCX::BN == TCY::BN && TCX::NT == TCY::NT && TCX::NT == ConTileX<T>::NT,
                "one contraction tile shape and workgroup size");
  static_assert(W || (TNX::NT == TCX::NT && TNY::NT == TCX::NT && TNX::BM == 2 * TCX::BM && 2 * TNX::BN == TCX::BN),
                "narrow tiles: two row tiles high, half a feature tile wide");
  __shared__ __attribute__((aligned(1024)))
  char lds[CMax<CMax<TCX::LDS_BYTES, TCY::LDS_BYTES>::value, CMax<TNX::LDS_BYTES, TNY::LDS_BYTES>::value>::value];
  grad_contract_dispatch<TCX, TCY, TNX, TNY, T, X3>(blockIdx.x, N, D, gb, bg, sp, acc_x, acc_y, lds);
}

// One pipeline step: G' tiles of diagonal diag_g and, for fp32, the
// contractions of diagonal diag_c (the 16-bit types run those in
// k_grad_contract; fp32 with the raw inputs as feature operands, VEC
// selecting 16-byte or 4-byte load lanes for them).  X3: bf16 split operands
// (K = 3 dp), G'^T written as hi and lo planes.
template <typename T, bool LIT, bool NORM, bool VEC, bool X3 = false, bool SMALL = false>
__global__ __launch_bounds__((GemmTile<T, VEC, SMALL>::NT), (Occ<T, VEC>::bwd)) void k_grad_step(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ldy, int N, int D, int kmax, float c,
    const float* __restrict__ ws, GradBufs gb, BlockGrid bg, StepPlan sp, float* __restrict__ acc_x,
    float* __restrict__ acc_y) {
  using TF = GemmTile<T, VEC, SMALL>;
  constexpr bool FUSED = !GtOnly<T>::value;  // contractions in this kernel
  using TCX = typename std::conditional<FUSED, typename ConTileSmall<T, VEC, SMALL>::x, TF>::type;
  using TCY = typename std::conditional<FUSED, typename ConTileSmall<T, VEC, SMALL>::y, TF>::type;
  static_assert(TCX::NT == TF::NT && TCY::NT == TF::NT, "one workgroup size per launch");
  __shared__ __attribute__((aligned(1024))) char lds[CMax<TF::LDS_BYTES, CMax<TCX::LDS_BYTES, TCY::LDS_BYTES>::value>::value];
  __shared__ float s_rx[TF::BM], s_ry[TF::BN], s_ir[TF::BM], s_ic[TF::BN];
  const int64_t blk = (int64_t)bg.bs * bg.bs;  // elements per G' block
  int sub = blockIdx.x;
  if (sub < sp.cx_pad + sp.cy_pad) {
    if constexpr (FUSED)
      grad_contract_dispatch<TCX, TCY, TCX, TCY, T>(sub, N, D, gb, bg, sp, acc_x, acc_y, lds, X, ldx, Y, ldy);
    return;
  }
  sub -= sp.cx_pad + sp.cy_pad;
  const int pid = xcd_remap(sub, sp.g_pad);
  if (pid >= sp.g_n) return;
  int tmg, tn;
  group_tile(pid, bg.nb * bg.gtm, bg.gtn, 8, tmg, tn);
  const int I = tmg / bg.gtm, tm = tmg - I * bg.gtm;
  const int J = (I + sp.diag_g) % bg.nb;
  const int i0 = I * bg.bs + tm * TF::BM, j0 = J * bg.bs + tn * TF::BN;
  if (i0 >= N || j0 >= N) return;  // never read by the contraction
  const int buf = sp.diag_g & 1;
  T* Gb = GtOnly<T>::value ? nullptr : (T*)gb.g[buf] + I * blk + (int64_t)(tm * TF::BM) * bg.bs + tn * TF::BN;
  // G'^T: row-major (fp32) or the tile's first block in the blocked layout (16-bit)
  const int64_t gt_off = I * blk + (GtOnly<T>::value ? gdma::gb_offset(tn * TF::BN, tm * TF::BM, bg.bs)
                                                     : (int64_t)(tn * TF::BN) * bg.bs + tm * TF::BM);
  T* GTb = GtOnly<T>::value ? (T*)gb.gt[buf] + gt_off : nullptr;
  T* GTl = X3 ? (T*)gb.gt_lo[buf] + gt_off : nullptr;
  grad_g_tile<TF, T, LIT, NORM, VEC, X3>(X, ldx, Y, ldy, N, D, kmax, c, ws, Gb, GTb, GTl, bg.bs, i0, j0, lds, s_rx,
                                         s_ry, s_ir, s_ic);
}

// 16-bit gradient-matrix tiles of diagonal sp.diag_g on the direct-to-LDS
// 256 x 256 tiles, chained as in the forward's block walk: persistent
// workgroups walk the tiles t = blockIdx.x + i * gridDim.x (XCD-grouped
// order; contiguous row-major runs of tiles or 2D blocks per workgroup were
// slower here, unlike in the forward), and the last
// chunk of each tile's k-loop loads chunk 0 of the next, which lands while
// the tile's G'^T is stored straight from the accumulators
// (grad_gt_store_direct).  The next tile's first barrier waits only for those
// loads, not for the stores.  The per-row and per-column vectors of a tile
// (rx, ry, 1/R, 1/C) reach LDS by direct loads into one of two buffers,
// issued right after the previous tile's first barrier (when every wave is
// done with that buffer).
template <typename T, bool LIT, bool NORM, bool X3 = false>
__global__ __launch_bounds__((FwdTile<T, true>::NT), 1) void k_grad_g_chain(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ldy, int N, int D, int kmax, float c,
    const float* __restrict__ ws, GradBufs gb, BlockGrid bg, StepPlan sp) {
  using TL = FwdTile<T, true>;
  static_assert(TL::CHAIN && GtOnly<T>::value, "chained 16-bit direct-to-LDS tiles");
  static_assert(TL::BM == 256 && TL::BN == 256 && TL::NT == 512, "one 64-float quarter per vector load, 8 waves");
  enum { V_RX = 0, V_RY = 1, V_IR = 2, V_IC = 3 };
  __shared__ __attribute__((aligned(1024))) char lds[TL::LDS_BYTES];
  __shared__ __attribute__((aligned(16))) float s_vec[2][4][TL::BM];
  constexpr int NST = gt_chain_stores<TL>() * (X3 ? 2 : 1);  // G'^T stores per lane and tile (X3: two planes)
  const int64_t n64 = N;
  const int64_t blk = (int64_t)bg.bs * bg.bs;
  const int buf = sp.diag_g & 1;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // tile -> (i0, j0, its place in the G'^T block); false for padding ids and tiles wholly past N
  auto coords = [&](int tile, int& i0, int& j0, uint16_t*& gt) {
    const int pid = xcd_remap(tile, sp.g_pad);
    if (pid >= sp.g_n) return false;
    int tmg, tn;
    group_tile(pid, bg.nb * bg.gtm, bg.gtn, 8, tmg, tn);
    const int I = tmg / bg.gtm, tm = tmg - I * bg.gtm;
    const int J = (I + sp.diag_g) % bg.nb;
    i0 = I * bg.bs + tm * TL::BM;
    j0 = J * bg.bs + tn * TL::BN;
    gt = (uint16_t*)gb.gt[buf] + I * blk + gdma::gb_offset(tn * TL::BN, tm * TL::BM, bg.bs);
    return i0 < N && j0 < N;
  };
  auto next_valid = [&](int tile, int& i0, int& j0, uint16_t*& gt) {
    for (; tile < sp.g_pad; tile += (int)gridDim.x)
      if (coords(tile, i0, j0, gt)) return tile;
    return sp.g_pad;
  };
  auto op_a = [&](int i0) { return tile_op<TL>(X + (int64_t)i0 * ldx, ldx, min(N - i0, TL::BM), kmax); };
  auto op_b = [&](int j0) { return tile_op<TL>(Y + (int64_t)j0 * ldy, ldy, min(N - j0, TL::BN), kmax); };
  // The vectors of tile (i0, j0) into s_vec[b]: load k (of 16) fills quarter
  // k % 4 of vector k / 4; wave w issues loads w and w + 8.  Entries past N
  // read as 0 (the buffer descriptor ends at N); 1/R and 1/C carry the
  // storage scale of G' in the epilogue.
  auto vec_loads = [&](int i0, int j0, int b) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int k = w + 8 * u, v = k >> 2, qr = k & 3;
      const bool need = v == V_IR || (v == V_IC && !LIT) || ((v == V_RX || v == V_RY) && NORM);
      if (!need) continue;
      const int slot = v == V_RX ? WS_RX : v == V_RY ? WS_RY : v == V_IR ? WS_INV_ROW : WS_INV_COL;
      const int o = (v == V_RX || v == V_IR) ? i0 : j0;
      const __amdgpu_buffer_rsrc_t r =
          __builtin_amdgcn_make_buffer_rsrc((void*)(ws + slot * n64 + o), 0, (N - o) * 4, 0x00020000);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)&s_vec[b][v][qr * 64], 4, (uint32_t)(qr * 64 + lane) * 4, 0,
          0, 0);
    }
  };
  int i0, j0;
  uint16_t* gt;
  int tile = next_valid(blockIdx.x, i0, j0, gt);
  if (tile >= sp.g_pad) return;
  vec_loads(i0, j0, 0);
  typename TL::Plan lp;
  TL::start(op_a(i0), op_b(j0), lds, lp);
  int p0 = 0, vb = 0;
  bool first = true;
  f32x16 acc[TL::FM][TL::FN];
  for (;;) {
    int i1 = i0, j1 = j0;
    uint16_t* gt1 = gt;
    const int next = next_valid(tile + (int)gridDim.x, i1, j1, gt1);
    const bool has_next = next < sp.g_pad;
    // the next tile's vectors go out after this tile's first barrier; the
    // first tile's chunk 0 has no stores behind it: its barrier waits for all
    auto hook = [&] {
      if (has_next) vec_loads(i1, j1, vb ^ 1);
    };
    TL::template chain<decltype(hook), NST>(lp, op_a(i1), op_b(j1), has_next, D, lds, p0, acc, hook, !first);
    first = false;
    const float* sv = &s_vec[vb][0][0];
    const bool diag = i0 < j0 + TL::BN && j0 < i0 + TL::BM;
    // (X3: the lo plane at the same offset in gt_lo)
    uint16_t* gtl = X3 ? (uint16_t*)gb.gt_lo[buf] + (gt - (uint16_t*)gb.gt[buf]) : nullptr;
    if (!diag && i0 + TL::BM <= N && j0 + TL::BN <= N)
      grad_gt_store_direct<TL, LIT, NORM, false, (int)GScale<T>::value, X3>(
          acc, c, i0, j0, N, gt, bg.bs, sv + V_RX * TL::BM, sv + V_RY * TL::BM, sv + V_IR * TL::BM,
          sv + V_IC * TL::BM, gtl);
    else
      grad_gt_store_direct<TL, LIT, NORM, true, (int)GScale<T>::value, X3>(
          acc, c, i0, j0, N, gt, bg.bs, sv + V_RX * TL::BM, sv + V_RY * TL::BM, sv + V_IR * TL::BM,
          sv + V_IC * TL::BM, gtl);
    if (!has_next) break;
    tile = next;
    i0 = i1;
    j0 = j1;
    gt = gt1;
    vb ^= 1;
  }
  gdma::drain_loads();
}

}  // namespace mec
