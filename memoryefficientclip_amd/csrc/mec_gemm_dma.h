// MFMA tile core for gfx950 with direct global->LDS loads, for bf16, fp16
// and fp32 operands (Geo::KIND).
//
// Geometry: a BM x BN output tile per workgroup of WM x WN waves, each wave a
// (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks, fp32 accumulate:
// v_mfma_f32_32x32x16_{bf16,f16} (one per block and k-step) or
// v_mfma_f32_32x32x2_f32 (four per block and k-step).  The 16-bit tiles
// (forward, gradient matrix, contractions) are 256 x 256 with 4 x 2 waves,
// one workgroup per CU (96 KB of ring; contractions 256 x 384 with 2 x 4
// waves where that takes fewer rounds, on the rolling operand schedule at the
// end of this file); fp32 tiles are 128 x 128 with 2 x 2 waves (48 KB), two
// (forward) or three (backward) workgroups per CU.
//
// Operands are K-major (element (row, k) at base[row * ld + k]).  K is staged
// in chunks of ROWB bytes per row through a ring of LDS stages ([row][ROWB]):
//   fp32: 64-byte rows (BK = 16), 3 stages; the loads of chunk kt+2 are
//         spread over the MFMAs of chunk kt.
//   16-bit: 128-byte rows (BK = 64, whole cache lines: half the L2 requests
//         of 64-byte rows), 2 stages of 64 KB; the loads of chunk kt+1 are
//         spread over the first two of chunk kt's four k-steps, and each
//         k-step's operand reads over the MFMAs of the step before.
// One barrier per chunk.  Each chunk arrives by buffer_load_dwordx4 ... lds:
// every lane of a wave moves 16 bytes and the wave writes one contiguous 1 KB
// block (1024 / ROWB rows) of the stage; which 16-byte k-vector of a row a
// lane fetches is XOR-swizzled (vector v of row r sits in slot v ^ swz(r))
// so that the MFMA operand reads (ds_read_b128, lanes 0..15 on rows 0..15 at
// one k-vector) hit 16 distinct 16-byte bank groups.
//
// Masking costs nothing in the loop: each operand's buffer descriptor covers
// exactly its valid rows and k range, so rows beyond `rows` read as zero, and
// lanes whose k-vector lies at or beyond kmax in the tail chunk get an
// out-of-range offset (also zero).  Requirements (checked by the host):
// 16-byte aligned base, ld and kmax multiples of the elements per 16-byte
// vector, and (rows - 1) * ld + kmax elements within 2^31 - 1 bytes (byte
// offsets are 32-bit, and the offset 2^31 must read as zero).
//
// Within a chunk the 16-byte vector fed to k-step s (0 .. NS-1) by lane half
// h = lane / 32 is vector h * NS + s for both operands (fp32: its four values
// feed four MFMAs in order), so the contraction over the chunk is exact.
//
// Transposed A (TA = true): A is stored k-row-major (element (m, k) at
// base[k * ld + m], m contiguous), e.g. a transposed gradient-matrix block.
// Its stage region is [BK k-rows][BM m] (BM = 256: 2 k-rows per 1 KB load
// block; BM = 512: one; the 16-byte slot of m-vector v in k-row r at
// v ^ 4 (r & 3)), and each MFMA
// fragment (8 consecutive k at one m) is assembled from two
// ds_read_b64_tr_b16: within each group of 16 lanes, source lane j points at
// 4 consecutive m of k-row k0 + j / 4, and result lane i receives k-rows
// k0 .. k0 + 3 of column m0 + i.  With the swizzle, the 32 lanes of a pass
// (4 k-rows x 32 m x 2 bytes) cover all 64 banks once.
//
// Transposed fp32 operands (TA for A, TB for B; the backward's contractions:
// the gradient-matrix block read across its rows, and the raw input rows as
// the feature operand): the stage region is [BK k-rows][E] floats (E = BM or
// BN, 256 or 512 bytes per k-row); the 16-byte slot of m-vector v in k-row r
// sits at v ^ 8 ((r >> 4) & 1), so that the two lane halves of an MFMA
// fragment read (k-rows 16 apart, 32 consecutive m each) land on different
// banks.  A fragment (4 consecutive k at one m per lane, k = 16 h + 4 s + t
// as for K-major operands) takes four ds_read_b32.  TB = 1 fills the stage
// with 16-byte lanes (16-byte aligned rows, ld and the valid columns
// multiples of 4); TB = 2 with 4-byte lanes (any layout), four loads per
// 1 KB block.  The feature operand's buffer descriptor is rebased at every
// chunk (64-bit base arithmetic), so its panel may span any number of rows;
// per-lane offsets stay within a chunk (31 rows of pitch ld: ld < 2^24).
#pragma once
#include "mec_common.h"

namespace mec {
namespace gdma {

constexpr uint32_t OOB = 0x80000000u;  // buffer offset that reads as zero

// element kinds: bf16 and fp16 (v_mfma_f32_32x32x16_*, one MFMA per k-step
// and block) and fp32 (v_mfma_f32_32x32x2_f32, four per k-step and block)
enum Kind { K_BF16 = 0, K_F16 = 1, K_F32 = 2 };

// Blocked gradient-matrix layout (GB): a bs x bs 16-bit block of G'^T
// (rows j, columns i) stored as 1 KB blocks of 32 rows x 16 columns, block
// (jb, ib) at element ((jb * bs / 16) + ib) * 512; within it, the 8 values
// i = 16 ib + 8 ih .. + 7 of row j = 32 jb + jj form the 16-byte slot
// gb_slot(jj, ih, ib & 1).  A wave's accumulators (after a lane-half swap)
// fill one whole block per 16-byte store, and the contractions copy whole
// blocks into LDS.  The XOR keeps their transposed fragment reads (4 rows j x
// 32 columns i per pass) on distinct banks.
__host__ __device__ constexpr int gb_slot(int jj, int ih, int ibp) { return (jj ^ (8 * ih + 4 * ibp)) + 32 * ih; }
__host__ __device__ constexpr int64_t gb_offset(int j, int i, int bs) {
  return ((int64_t)(j >> 5) * (bs >> 4) + (i >> 4)) * 512 + gb_slot(j & 31, (i >> 3) & 1, (i >> 4) & 1) * 8 + (i & 7);
}

template <int BM_, int BN_, bool TA_ = false, int WM_ = 2, int WN_ = 2, int KIND_ = K_BF16, int SA_ = 2,
          bool GB_ = false, int TB_ = 0, int S_ = 2, int KS_ = 1>
struct Geo {
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int KIND = KIND_;
  static constexpr bool F16 = KIND == K_F16;           // fp16 MFMAs (16-bit kinds)
  static constexpr int ESZ = KIND == K_F32 ? 4 : 2;    // bytes per element
  static constexpr int EPV = 16 / ESZ;                 // elements per 16-byte vector
  // ring: chunks of 128 bytes per operand row (whole cache lines) in 2 stages
  static constexpr int ROWB = 128;                     // bytes per staged row of a chunk
  // LDS stages of the ring (A and B together, SA = 2): chunk kt + S - 1 is
  // loaded while chunk kt is consumed.  2, or more for tiles whose k-loop is
  // too short per chunk to cover an L2 or HBM round trip (64 x 64 fp32).
  static constexpr int S = S_;
  static_assert(S >= 2 && S <= 4 && (S == 2 || SA_ == 2), "2-4 stages of A and B together");
  static constexpr int RPB = 1024 / ROWB;              // rows per 1 KB load block
  static constexpr int SLOTS = ROWB / 16;              // 16-byte vectors per row
  static constexpr int NS = ROWB / 32;                 // k-steps per chunk (one vector per lane half each)
  static constexpr int BK = ROWB / ESZ;                // k per chunk
  // bank-conflict swizzle: vector v of row r sits in slot v ^ swz(r), so that
  // 16 consecutive rows at one vector hit 16 distinct 16-byte bank groups
  // (rows r and r + 2 share banks at this pitch)
  static __device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
  static constexpr int MPB = KIND == K_F32 ? 4 : 1;    // MFMAs per block and k-step
  static constexpr bool TA = TA_;                      // A stored k-row-major
  static_assert(!TA || (ESZ == 2 ? (BM == 256 || BM == 512) : (BM == 64 || BM == 128)),
                "transposed A: 16-bit with 512- or 1024-byte k-rows, fp32 with 256- or 512-byte k-rows");
  static constexpr int TKPB = TA ? 1024 / (BM * ESZ) : 1;  // transposed A: k-rows per 1 KB load block
  // B stored k-row-major (fp32): 0 no, 1 with 16-byte lanes, 2 with 4-byte lanes
  static constexpr int TB = TB_;
  static_assert(TB == 0 || (KIND == K_F32 && (BN == 64 || BN == 128)), "transposed B: fp32, 256- or 512-byte k-rows");
  static constexpr int TKPB_B = TB ? 1024 / (BN * ESZ) : 1;  // transposed B: k-rows per 1 KB block
  static constexpr int BW = TB == 2 ? 4 : 1;                  // loads per 1 KB block of B
  // fp32 transposed operands: slot XOR of k-row r (the two lane halves of a
  // fragment read k-rows 16 apart)
  static __host__ __device__ constexpr int swt32(int r) { return 8 * ((r >> 4) & 1); }
  // A in the blocked gradient-matrix layout (gb_offset; bs = ld): TA, the x
  // side's operand (m = i, k = j: a chunk is 2 x BM/16 blocks), else the y
  // side's (m = j, k = i: BM/32 x 4 blocks).  Stage block b holds block
  // (jb, ib) of the chunk: b = jb * BM/16 + ib (TA), b = jb * 4 + ib (else).
  // k-step s, lane half h take the k-vector kvec(s, h): one i-block per
  // k-step (blocked) or vector h * NS + s (row-major operands).
  static constexpr bool GB = GB_;
  static_assert(!GB || (ESZ == 2 && BK == 64), "blocked A: 16-bit, 64 k per chunk");
  static __device__ __forceinline__ int kvec(int s, int h) { return GB ? 2 * s + h : h * NS + s; }
  static __device__ __forceinline__ void gb_block(int b, int& jb, int& ib) {
    if (TA) {
      jb = b / (BM / 16);
      ib = b - jb * (BM / 16);
    } else if (SA == 4) {
      // half-chunk slots: blocks [0, A_BLOCKS / 2) are k-steps 0-1 (i-blocks
      // 0, 1), the rest k-steps 2-3; within a half, block b' = 2 jb + (ib & 1)
      const int hh = b / (BM / 16), bh = b - hh * (BM / 16);
      jb = bh >> 1;
      ib = 2 * hh + (bh & 1);
    } else {
      jb = b >> 2;
      ib = b & 3;
    }
  }
  // KS = 2 splits k: waves w and w + WM WN compute the same sub-tile from
  // alternate halves of every chunk's k-steps (mainloop_ks2), so that two
  // waves share each SIMD; the loads are split over all KS WM WN waves
  static constexpr int KS = KS_;
  static_assert(KS == 1 || KS == 2, "k split by 1 or 2");
  static constexpr int WM = WM_, WN = WN_, NW = WM * WN * KS, NT = 64 * NW;
  // this wave's sub-tile (wave_m, wave_n) and k-group
  static __device__ __forceinline__ unsigned wave_mnu() {
    return KS == 1 ? (threadIdx.x >> 6) : (threadIdx.x >> 6) % (WM * WN);
  }
  static __device__ __forceinline__ int wave_mn() { return (int)wave_mnu(); }
  static __device__ __forceinline__ int wave_m() { return (int)(wave_mnu() / WN); }
  static __device__ __forceinline__ int wave_n() { return (int)(wave_mnu() % WN); }
  static __device__ __forceinline__ int wave_k() { return KS == 1 ? 0 : (int)((threadIdx.x >> 6) / (WM * WN)); }
  static constexpr int TM = BM / WM, TN = BN / WN;     // wave sub-tile
  static constexpr int FM = TM / 32, FN = TN / 32;     // 32x32 MFMA blocks per wave
  static constexpr int ROWS = BM + BN;
  static constexpr int STAGE = ROWS * ROWB;
  // A stages: 2 (the ring's stages hold A and B of one chunk each), or 3 (A
  // gets a ring of its own, one chunk deeper than B's, for an A streamed from
  // HBM; not chained): then A stages s = 0..2 come first, B's two after them.
  // 4: A in four half-chunk slots (blocked A on the rolling schedule: the
  // k-steps 0-1 and 2-3 of a chunk are whole 1 KB blocks), B in two stages
  // after them; a_stage(s) is half-slot s.  Same LDS as two stages.
  static constexpr int SA = SA_;
  static_assert(SA == 2 || SA == 3 || SA == 4, "two or three A stages, or four A half-stages");
  static constexpr int A_STAGE = BM * ROWB, B_STAGE = BN * ROWB;
  static constexpr int LDS_BYTES = SA == 2 ? S * STAGE : (SA == 3 ? 3 : 2) * A_STAGE + 2 * B_STAGE;
  static __device__ __forceinline__ char* a_stage(char* lds, int s) {
    return SA == 2 ? lds + s * STAGE : lds + s * (SA == 4 ? A_STAGE / 2 : A_STAGE);
  }
  static __device__ __forceinline__ char* b_stage(char* lds, int s) {
    return SA == 2 ? lds + s * STAGE + A_STAGE : lds + (SA == 3 ? 3 : 2) * A_STAGE + s * B_STAGE;
  }
  static constexpr int A_BLK = BM / RPB, B_BLK = BN / RPB;  // 1 KB blocks of A / B per stage
  static constexpr int IPW = A_BLK / NW + B_BLK / NW * BW;  // load instructions per wave per chunk
  static constexpr int NMF = FM * FN * MPB;            // MFMAs per k-step
  static_assert(A_BLK % NW == 0 && B_BLK % NW == 0 && BM % RPB == 0, "load split");
  static_assert((NW * RPB) % 16 == 0, "the loads of one wave share the row swizzle");
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave sub-tile of 32x32 blocks");
};

struct Operand {
  const void* base;  // element (row, k) at base[row * ld + k] (transposed A: base[k * ld + row];
                     // blocked A: the tile's first block, ld = the block's bs)
  int64_t ld;
  int rows;          // valid rows from base (rows beyond read as 0; transposed A: all BM rows readable)
  int kmax;          // valid k range [0, kmax), a multiple of the elements per 16-byte vector
};


template <int ESZ>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const Operand& op) {
  const int64_t elems = op.rows > 0 ? (int64_t)(op.rows - 1) * op.ld + op.kmax : 0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)op.base, 0, (int)(elems * ESZ), 0x00020000);
}
// transposed B: the descriptor of the chunk of BK k-rows starting at k-row
// k0 of the panel at base (pitch ld elements): its valid rows (below kmax),
// the last one up to ncols columns
template <int ESZ, int BK>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_chunk(const char* base, int64_t ld, int kmax, int ncols,
                                                                  int k0) {
  const int rows = kmax - k0;
  const int r = rows < BK ? rows : BK;
  const int64_t bytes = r > 0 ? ((int64_t)(r - 1) * ld + ncols) * ESZ : 0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)k0 * ld * ESZ), 0, (int)bytes, 0x00020000);
}
// transposed A: k-rows [0, kmax) of BM elements
template <int BM, int ESZ>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_t(const Operand& op) {
  const int64_t elems = op.kmax > 0 ? (int64_t)(op.kmax - 1) * op.ld + BM : 0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)op.base, 0, (int)(elems * ESZ), 0x00020000);
}

// This wave's IPW loads of every chunk: per-lane byte offset at k = 0, the
// lane's k-vector start, and the 1 KB LDS block each load fills.  Load i of
// wave w fills block b = i * NW + w, so blocks [0, BM / 16) (operand A) are
// the loads i < A_LOADS of every wave: which operand a load reads is known at
// compile time.
template <class G>
struct LoadPlan {
  static constexpr int A_BLOCKS = G::A_BLK;  // 1 KB blocks of A per stage (transposed A too)
  static constexpr int A_LOADS = A_BLOCKS / G::NW;
  // lanes per k-row of a 1 KB block of transposed A / B (16-byte lanes)
  static constexpr int LPK_A = 64 / G::TKPB, LPK_B = 64 / G::TKPB_B;
  static constexpr int KRB_B = G::BN * G::ESZ;  // transposed B: bytes per k-row
  __amdgpu_buffer_rsrc_t ra, rb;
  uint32_t voff[G::IPW];
  int kv;          // k of this lane's 16-byte vector within a chunk (K-major operands)
  int kr;          // this lane's half of the wave (lane / 32; blocked A)
  int kt;          // transposed A: k-row of this lane within a 1 KB block
  int kb;          // transposed B: this lane's k-row within the chunk for load A_LOADS (wide lanes)
  int w;           // wave index (uniform)
  int kmax_a, kmax_b;
  int64_t lda;     // transposed A: bytes per k-row
  // transposed B: the panel (element (n, k) at b_base[k * ldb + n]) and its valid columns
  const char* b_base;
  int64_t ldb;
  int ncols_b;
  static __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_a(const Operand& A) {
    if constexpr (G::GB) {
      // the tile's blocks: TA, i-blocks [0, BM/16) of the j-block rows up to
      // kmax; else its BM/32 j-block rows (every i-block)
      const int64_t rows32 = ((int64_t)A.kmax + 31) / 32;
      const int64_t elems = G::TA ? (rows32 > 0 ? (rows32 - 1) * 32 * A.ld + G::BM * 32 : 0) : (int64_t)G::BM * A.ld;
      return __builtin_amdgcn_make_buffer_rsrc((void*)A.base, 0, (int)(elems * 2), 0x00020000);
    } else {
      return G::TA ? make_rsrc_t<G::BM, G::ESZ>(A) : make_rsrc<G::ESZ>(A);
    }
  }
  static __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_b(const Operand& B) { return make_rsrc<G::ESZ>(B); }
  // transposed B, load q = I - A_LOADS: its k-row within the chunk, minus kb
  // (a compile-time function of q; for wide lanes kb carries the lane's part)
  static constexpr int tb_krow_off(int q) {
    return G::BW == 1 ? G::TKPB_B * G::NW * q : G::TKPB_B * G::NW * (q / G::BW) + ((q % G::BW) * 256) / KRB_B;
  }
  __device__ __forceinline__ void init(const Operand& A, const Operand& B) {
    ra = rsrc_a(A);
    kmax_a = A.kmax;
    kmax_b = B.kmax;
    lda = A.ld * G::ESZ;
    const int lane = threadIdx.x & 63;
    w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rib = lane / G::SLOTS, phys = lane % G::SLOTS;
    // every load of this wave fills rows b * RPB + rib with b = i * NW + w,
    // whose swizzle does not depend on i
    kv = (phys ^ G::swz(w * G::RPB + rib)) * G::EPV;
    kr = lane >> 5;
    kt = lane / LPK_A;
    if constexpr (G::TB) {
      b_base = (const char*)B.base;
      ldb = B.ld;
      ncols_b = B.rows < G::BN ? B.rows : G::BN;
      kb = G::TKPB_B * w + (G::BW == 1 ? lane / LPK_B : 0);
      rb = ra;  // (per chunk: rsrc_b_chunk)
    } else {
      rb = rsrc_b(B);
    }
#pragma unroll
    for (int i = 0; i < G::IPW; ++i) {
      const int b = i * G::NW + w;
      if (G::GB && i < A_LOADS) {
        // blocked A: load i copies block (jb, ib) of the chunk, lane l its slot l
        int jb, ib;
        G::gb_block(b, jb, ib);
        voff[i] = (uint32_t)(((int64_t)jb * 32 * A.ld + ib * 512 + lane * 8) * 2);
      } else if (G::TA && i < A_LOADS) {
        // block b holds k-rows TKPB b .. + TKPB - 1 (within the chunk); lane l
        // fills slot l % LPK_A of k-row TKPB b + l / LPK_A
        const int krow = G::TKPB * b + kt;
        const int sw = G::ESZ == 2 ? 4 * (krow & 3) : G::swt32(krow);
        const int slot = (lane % LPK_A) ^ sw;
        voff[i] = (uint32_t)(((int64_t)krow * A.ld + slot * G::EPV) * G::ESZ);
      } else if (G::TB && i >= A_LOADS) {
        // transposed B (offsets from the chunk's first k-row)
        const int q = i - A_LOADS;
        int krow, pos;  // k-row in the chunk, float within it
        if (G::BW == 1) {
          krow = G::TKPB_B * (q * G::NW + w) + lane / LPK_B;
          pos = (lane % LPK_B) * 4;
        } else {
          const int byte = (q % G::BW) * 256 + 4 * lane;
          krow = G::TKPB_B * ((q / G::BW) * G::NW + w) + byte / KRB_B;
          pos = (byte % KRB_B) / 4;
        }
        const int lslot = (pos >> 2) ^ G::swt32(krow);
        voff[i] = (uint32_t)(((int64_t)krow * ldb + lslot * 4 + (pos & 3)) * G::ESZ);
      } else {
        const int r = b * G::RPB + rib;
        voff[i] = (uint32_t)(((i < A_LOADS ? (int64_t)r * A.ld : (int64_t)(r - G::BM) * B.ld) + kv) * G::ESZ);
      }
    }
  }
  // load i of the chunk starting at k0 into the A stage ad (loads i <
  // A_LOADS) or the B stage bd.  Chunks at or past kmax read as zeros
  // (out-of-range offsets), so loads may run past the last chunk.
  template <int I>
  __device__ __forceinline__ void issue(int k0, char* ad, char* bd) const {
    constexpr bool isa = I < A_LOADS;
    if constexpr (G::TB && !isa) {
      // transposed B: 16- or 4-byte lanes into block (q / BW) * NW + w, part q % BW
      constexpr int q = I - A_LOADS;
      constexpr int koff = tb_krow_off(q);
      const uint32_t off = (kb + koff < kmax_b - k0) ? voff[I] : OOB;
      char* dst = bd + ((q / G::BW) * G::NW + w) * 1024 + (q % G::BW) * 256;
      const __amdgpu_buffer_rsrc_t rc = make_rsrc_chunk<G::ESZ, G::BK>(b_base, ldb, kmax_b, ncols_b, k0);
      // (the size operand must be a literal)
      if constexpr (G::BW == 1)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (__attribute__((address_space(3))) void*)dst, 4, off, 0, 0, 0);
      return;
    }
    uint32_t off, soff;
    if (G::GB && isa) {
      int jb, ib;
      G::gb_block(I * G::NW + w, jb, ib);
      const int lane = threadIdx.x & 63;
      if (G::TA) {
        // k = j: this lane's row of the block; a chunk is k0 / 32 j-block rows down
        const int jj = (lane & 31) ^ (8 * kr + 4 * (ib & 1));
        off = (k0 + 32 * jb + jj < kmax_a) ? voff[I] : OOB;
        soff = (uint32_t)(k0 * lda);
      } else {
        // k = i: this lane's 8 columns; a chunk is k0 / 16 blocks along
        off = (k0 + 16 * ib + 8 * kr < kmax_a) ? voff[I] : OOB;
        soff = (uint32_t)k0 * 64;
      }
    } else if (G::TA && isa) {
      off = (k0 + G::TKPB * (I * G::NW + w) + kt < kmax_a) ? voff[I] : OOB;
      soff = (uint32_t)(k0 * lda);
    } else {
      off = (k0 + kv < (isa ? kmax_a : kmax_b)) ? voff[I] : OOB;
      soff = (uint32_t)k0 * G::ESZ;
    }
    // (four A half-stages: ad is the half-slot of load I's half, I / (A_LOADS / 2))
    char* dst = isa ? ad + ((G::SA == 4 ? I % (A_LOADS / 2) : I) * G::NW + w) * 1024
                    : bd + (I * G::NW + w - A_BLOCKS) * 1024;
    // the gradient-matrix operand (blocked A) streams from HBM once per side:
    // non-temporal (cache policy 2), so that it does not displace the
    // transposed-input panels the other tiles re-read
    if constexpr (G::GB && isa)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*)dst, 16, off, soff, 0, 2);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isa ? ra : rb, (__attribute__((address_space(3))) void*)dst, 16, off,
                                               soff, 0, 0);
  }
};

// One k-step's operand fragments: per 32-row block, this lane's 16-byte
// vector (8 16-bit or 4 fp32 values; the bits are moved as i16x8)
template <class G>
struct Frags {
  i16x8 a[G::FM], b[G::FN];
};

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

// Operand reads from LDS, as inline asm.  The compiler cannot tell these
// reads from the global->LDS loads still in flight into the other stages,
// and in some loop shapes it waits for every outstanding load (vmcnt(0))
// before each group of reads, which serialises the prefetch ring.  In asm
// they carry no such wait; the mainloop awaits their completion explicitly
// (lgkm_wait) before the MFMAs that use them, and wait_barrier orders them
// against the loads that refill their stage.
__device__ __forceinline__ uint32_t lds_off(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
template <int OFF>
__device__ __forceinline__ i16x8 lds_read_b128(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536 && OFF % 16 == 0, "ds_read_b128 offset");
  i16x8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
template <int OFF>
__device__ __forceinline__ float lds_read_b32(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536 && OFF % 4 == 0, "ds_read_b32 offset");
  float v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
// 4 k-rows of one column per lane (see the transposed-A note above)
__device__ __forceinline__ i16x4_t read_tr4(const char* p) {
  i16x4_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(lds_off(p)) : "memory");
  return v;
}

// Operand addresses of k-step s for this lane.  a_ptr: its A vector of
// fragment 0 (fragment i is 4 KB further: 32 rows of 128 bytes, or 4 blocks
// of the blocked layout), for A that is not transposed.  ta_ptr: the source
// address of transposed-A read `half` of fragment i: lane group g = lane / 16
// covers m0 + 16 (g & 1) .. + 15 and k-vector kvec(s, g >> 1); source lane j
// reads k-row kb + 4 half + j / 4, m-quad j % 4.  b_ptr: its B vector of
// fragment 0.
template <class G>
__device__ __forceinline__ const char* a_ptr(const char* stage, int s) {
  const int lane = threadIdx.x & 63, wm = G::KS == 1 ? (int)((threadIdx.x >> 6) / G::WN) : G::wave_m();
  const int q = lane & 31, h = lane >> 5;
  if constexpr (G::GB && G::SA == 4) {
    // four A half-stages: block (wm * TM / 32, s) of the half-slot of k-step s
    // at 2 KB per j-block and 1 KB per odd k-step
    return stage + ((wm * G::TM / 32) * 2 + (s & 1)) * 1024 + gb_slot(q, h, s & 1) * 16;
  } else if constexpr (G::GB) {
    // m = j: block (wm * TM / 32, s), row q, i-half h
    return stage + ((wm * G::TM / 32) * 4 + s) * 1024 + gb_slot(q, h, s & 1) * 16;
  } else {
    return stage + (wm * G::TM + q) * G::ROWB + ((G::kvec(s, h) ^ G::swz(q)) << 4);
  }
}
template <class G>
__device__ __forceinline__ const char* ta_ptr(const char* stage, int s, int i, int half) {
  const int lane = threadIdx.x & 63, wm = G::KS == 1 ? (int)((threadIdx.x >> 6) / G::WN) : G::wave_m();
  const int g = lane >> 4, j = lane & 15;
  const int kb = G::kvec(s, g >> 1) * 8;
  const int m = wm * G::TM + i * 32 + 16 * (g & 1) + 4 * (j & 3);
  const int krow = kb + 4 * half + (j >> 2);
  if constexpr (G::GB) {
    // krow = 32 (s >> 1) + 16 (s & 1) + r with r < 16, and the slot's XOR
    // touches bits 2-3 only: the k-step adds a constant to a per-lane offset
    const int ib = m >> 4, ih = (m >> 3) & 1, r = krow & 15;
    const int lane_off = ib * 1024 + ((r ^ (8 * ih + 4 * (ib & 1))) + 32 * ih) * 16 + (m & 7) * 2;
    return stage + lane_off + (s >> 1) * (G::BM / 16) * 1024 + (s & 1) * 256;
  } else {
    const int slot = (m >> 3) ^ (4 * (krow & 3));
    return stage + krow * (G::BM * 2) + slot * 16 + (m & 7) * 2;
  }
}
template <class G>
__device__ __forceinline__ const char* b_ptr(const char* bstage, int s) {
  const int lane = threadIdx.x & 63, wn = G::KS == 1 ? (int)((threadIdx.x >> 6) % G::WN) : G::wave_n();
  const int q = lane & 31, h = lane >> 5;
  return bstage + (wn * G::TN + q) * G::ROWB + ((G::kvec(s, h) ^ G::swz(q)) << 4);
}

// fp32 transposed operand (stage region of E floats per k-row): this lane's
// address of fragment i (32 m from m0 + 32 i), k-step s, k-value t = 0 (t
// adds t * E * 4 bytes): m = m0 + 32 i + lane % 32, k-row 16 h + 4 s + t
template <int E>
__device__ __forceinline__ uint32_t t32_addr(const char* region, int m0, int i, int s) {
  const int lane = threadIdx.x & 63, q = lane & 31, h = lane >> 5;
  const int m = m0 + 32 * i + q;
  const int krow = 16 * h + 4 * s;
  return lds_off(region) + krow * (E * 4) + (((m >> 2) ^ (8 * h)) << 4) + (m & 3) * 4;
}

// LDS reads per fragment set: A, B, and both
template <class G>
constexpr int frag_reads_a() {
  return G::TA ? (G::ESZ == 4 ? 4 : 2) * G::FM : G::FM;
}
template <class G>
constexpr int frag_reads_b() {
  return G::TB ? 4 * G::FN : G::FN;
}
template <class G>
constexpr int frag_reads() {
  return frag_reads_a<G>() + frag_reads_b<G>();
}

// One k-step's fragment reads, one read at a time: read R (of frag_reads) of
// k-step s.  16-bit transposed A takes two reads per fragment (its low and
// high four k-values), written into the halves of f.a[i]; fp32 transposed
// operands four (one k-value each).
template <class G>
struct FragReader {
  static constexpr bool TA32 = G::TA && G::ESZ == 4, TA16 = G::TA && G::ESZ == 2;
  uint32_t abase, bbase;
  uint32_t ta[TA16 ? G::FM : 1][2];  // 16-bit transposed A: per fragment and half
  uint32_t a32[TA32 ? G::FM : 1];     // fp32 transposed A: per fragment
  uint32_t b32[G::TB ? G::FN : 1];    // fp32 transposed B: per fragment
  __device__ __forceinline__ FragReader(const char* stage, const char* bstage, int s) {
    int wm, wn;
    if constexpr (G::KS == 1) {
      const int w = threadIdx.x >> 6;
      wm = w / G::WN;
      wn = w % G::WN;
    } else {
      wm = G::wave_m();
      wn = G::wave_n();
    }
    if constexpr (G::TB) {
      bbase = 0;
#pragma unroll
      for (int j = 0; j < G::FN; ++j) b32[j] = t32_addr<G::BN>(bstage, wn * G::TN, j, s);
    } else {
      bbase = lds_off(b_ptr<G>(bstage, s));
    }
    if constexpr (TA16) {
      abase = 0;
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int half = 0; half < 2; ++half) ta[i][half] = lds_off(ta_ptr<G>(stage, s, i, half));
    } else if constexpr (TA32) {
      abase = 0;
#pragma unroll
      for (int i = 0; i < G::FM; ++i) a32[i] = t32_addr<G::BM>(stage, wm * G::TM, i, s);
    } else {
      abase = lds_off(a_ptr<G>(stage, s));
    }
  }
  template <int R>
  __device__ __forceinline__ void read(Frags<G>& f) const {
    constexpr int NA = frag_reads_a<G>();
    if constexpr (R < NA) {
      if constexpr (TA16) {
        i16x4_t v;
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(ta[R / 2][R % 2]) : "memory");
        if constexpr (R % 2 == 0)
          f.a[R / 2].lo = v;
        else
          f.a[R / 2].hi = v;
      } else if constexpr (TA32) {
        f32x4 v = __builtin_bit_cast(f32x4, f.a[R / 4]);
        v[R % 4] = lds_read_b32<(R % 4) * G::BM * 4>(a32[R / 4]);
        f.a[R / 4] = __builtin_bit_cast(i16x8, v);
      } else {
        f.a[R] = lds_read_b128<R * 32 * G::ROWB>(abase);
      }
    } else {
      constexpr int RB = R - NA;
      if constexpr (G::TB) {
        f32x4 v = __builtin_bit_cast(f32x4, f.b[RB / 4]);
        v[RB % 4] = lds_read_b32<(RB % 4) * G::BN * 4>(b32[RB / 4]);
        f.b[RB / 4] = __builtin_bit_cast(i16x8, v);
      } else {
        f.b[RB] = lds_read_b128<RB * 32 * G::ROWB>(bbase);
      }
    }
  }
};

// every fragment of k-step s
template <class G>
__device__ __forceinline__ void read_frags(const char* stage, const char* bstage, int s, Frags<G>& f) {
  const FragReader<G> rd(stage, bstage, s);
  static_for<frag_reads<G>()>([&](auto r) { rd.template read<r>(f); });
}

// at most N LDS operations outstanding (the reads of `f` were issued before
// the last N), then f's registers are tied to the wait so that no MFMA using
// them is scheduled above it
template <int N, class G>
__device__ __forceinline__ void lgkm_wait(Frags<G>& f) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
  for (int i = 0; i < G::FM; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
  for (int j = 0; j < G::FN; ++j) asm volatile("" : "+v"(f.b[j]));
}

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// vmcnt <= N and lgkmcnt == 0, then a workgroup barrier.  __syncthreads()
// would also wait for every outstanding LDS DMA (its release fence counts them
// as LDS stores), which would serialise the prefetch ring; the explicit vmcnt
// covers the chunk that must have landed, lgkmcnt(0) the operand reads of the
// stage that is refilled after the barrier.
template <int N>
__device__ __forceinline__ void wait_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
  asm volatile("s_barrier" ::: "memory");
}

// Hook on the fp32 operand values as the MFMAs take them (the default of
// mainloop_core: none).  a(v, i, j, t) / b(v, i, j, t) return the value fed to
// MFMA t of block (i, j) from A fragment register v (fragment i) / B fragment
// register v (fragment j).
struct NoFragHook {
  __device__ __forceinline__ float a(const i16x8& v, int, int, int t) const { return __builtin_bit_cast(f32x4, v)[t]; }
  __device__ __forceinline__ float b(const i16x8& v, int, int, int t) const { return __builtin_bit_cast(f32x4, v)[t]; }
};

// Squared norms of the operand rows, accumulated from the fragments: each
// lane sees every k of its fragments' rows (m = 32 i + lane % 32 of the
// wave's A rows, n = 32 j + lane % 32 of its B rows) within its lane half
// (k = 16 h + 4 s + t of each chunk), so after the k-loop sa[i] + (the same
// of lane ^ 32) is the row's sum of squares over the k it took.  Each value
// is counted once per wave: A values at j = 0, B values at i = 0; and only
// at the k-values t % 2 == PA (A) and t % 2 == PB (B), so that two waves that
// share rows (the same wm, wn = 0 and 1, with PA = wn) split the work: one
// FMA per MFMA per wave on 2 x 2 waves, where every wave taking every k
// needed two.  The row's norm is the sum of the two waves' partials.
template <class G, int PA = -1, int PB = -1>
struct NormHook {
  static_assert(G::KIND == K_F32, "fp32 operands");
  mutable float sa[G::FM], sb[G::FN];
  __device__ __forceinline__ NormHook() {
#pragma unroll
    for (int i = 0; i < G::FM; ++i) sa[i] = 0.f;
#pragma unroll
    for (int j = 0; j < G::FN; ++j) sb[j] = 0.f;
  }
  __device__ __forceinline__ float a(const i16x8& v, int i, int j, int t) const {
    const float x = __builtin_bit_cast(f32x4, v)[t];
    if (j == 0 && (PA < 0 || t % 2 == PA)) sa[i] = fmaf(x, x, sa[i]);
    return x;
  }
  __device__ __forceinline__ float b(const i16x8& v, int i, int j, int t) const {
    const float x = __builtin_bit_cast(f32x4, v)[t];
    if (i == 0 && (PB < 0 || t % 2 == PB)) sb[j] = fmaf(x, x, sb[j]);
    return x;
  }
};

// MFMAs of one k-step with loads [L0, L1) interleaved, in program order.
// Loads [L0, L1) spread over the NMF MFMAs of a k-step: LPS loads after
// every EVERY-th MFMA (one load per slot while there are at most NMF loads)
// loads [I0, I1) in order
template <class G, int I0, int I1>
__device__ __forceinline__ void issue_loads(const LoadPlan<G>& lp, int k0, char* ad, char* bd) {
  if constexpr (I0 < I1) {
    lp.template issue<I0>(k0, ad, bd);
    issue_loads<G, I0 + 1, I1>(lp, k0, ad, bd);
  }
}
template <class G, int L0, int L1>
struct LoadSlots {
  static constexpr int NL = L1 - L0;
  static constexpr int LPS = NL > G::NMF ? (NL + G::NMF - 1) / G::NMF : 1;
  static constexpr int NSL = (NL + LPS - 1) / LPS;
  static constexpr int EVERY = NSL > 0 ? G::NMF / NSL : G::NMF + 1;
  // after MFMA m
  template <int M>
  static __device__ __forceinline__ void after(const LoadPlan<G>& lp, int k0, char* ad, char* bd) {
    if constexpr (NL > 0 && (M % EVERY) == EVERY - 1 && M / EVERY < NSL) {
      constexpr int I0 = L0 + (M / EVERY) * LPS;
      constexpr int I1 = I0 + LPS < L1 ? I0 + LPS : L1;
      sched_fence();
      issue_loads<G, I0, I1>(lp, k0, ad, bd);
      sched_fence();
    }
  }
};

template <class G, int L0, int L1, class FH = NoFragHook>
__device__ __forceinline__ void mfma_step(const Frags<G>& f, f32x16 (&acc)[G::FM][G::FN], const LoadPlan<G>& lp,
                                          int k0, char* ad, char* bd, const FH& fh = FH()) {
  static_for<G::NMF>([&](auto mc) {
    constexpr int m = mc;
    if constexpr (G::KIND == K_F32) {
      // block (i, j), sub-step t: lane half h supplies k = 16-byte vector's element t
      constexpr int blk = m / 4, t = m % 4, i = blk / G::FN, j = blk % G::FN;
      acc[i][j] = mfma_f32_32x32x2(fh.a(f.a[i], i, j, t), fh.b(f.b[j], i, j, t), acc[i][j]);
    } else {
      acc[m / G::FN][m % G::FN] =
          mfma16_32x32x16<G::F16>(f.a[m / G::FN], f.b[m % G::FN], acc[m / G::FN][m % G::FN]);
    }
    LoadSlots<G, L0, L1>::template after<m>(lp, k0, ad, bd);
  });
}

// mfma_step with the LDS reads of the next fragment set `nf` interleaved: two reads after each of the first MFMAs, so that the reads
// land during the step and the next step's MFMAs need not wait for them.
template <class G, int L0, int L1, class FH = NoFragHook>
__device__ __forceinline__ void mfma_step_rd(const Frags<G>& f, f32x16 (&acc)[G::FM][G::FN], const LoadPlan<G>& lp,
                                             int k0, char* ad, char* bd, const FragReader<G>& rd, Frags<G>& nf,
                                             const FH& fh = FH()) {
  constexpr int NR = frag_reads<G>();
  static_assert((NR + 1) / 2 <= G::NMF, "read slots");
  static_for<G::NMF>([&](auto mc) {
    constexpr int m = mc;
    if constexpr (G::KIND == K_F32) {
      // consecutive MFMAs on different blocks (the fences below keep program order)
      constexpr int NB = G::FM * G::FN, blk = m % NB, t = m / NB, i = blk / G::FN, j = blk % G::FN;
      acc[i][j] = mfma_f32_32x32x2(fh.a(f.a[i], i, j, t), fh.b(f.b[j], i, j, t), acc[i][j]);
    } else {
      acc[m / G::FN][m % G::FN] =
          mfma16_32x32x16<G::F16>(f.a[m / G::FN], f.b[m % G::FN], acc[m / G::FN][m % G::FN]);
    }
    if constexpr (2 * m < NR) {
      sched_fence();
      rd.template read<2 * m>(nf);
      if constexpr (2 * m + 1 < NR) rd.template read<2 * m + 1>(nf);
      sched_fence();
    }
    LoadSlots<G, L0, L1>::template after<m>(lp, k0, ad, bd);
  });
  sched_fence();  // the step's MFMAs stay above the caller's next wait
}

// acc[i][j] (this wave's sub-tile) = sum_k A(m, k) * B(n, k) over k in [0, K)
// (ZERO = false: added to acc), K > 0 (chunks past kmax read as zero).  Uses
// LDS_BYTES of `lds`; ends with every wave past its last LDS read of the ring
// and its loads landed (callers may reuse the ring after a barrier).
//
// Chunk kt+1 loads into the other stage, freed by the barrier at the start of
// chunk kt, spread over the first two of chunk kt's four k-steps (measured:
// issuing them all at the start of the chunk, or over all four steps, was
// slower).  The k-steps alternate fragment sets f0 / f1, each step's reads
// spread over the MFMAs of the step before.  Every iteration issues its
// loads, also past the last chunk (they read zeros into a stage nobody reads
// again), so the loop has no branches around them.

// Chunk 0 of a tile into stage 0: the loads before the first mainloop.
template <class G>
__device__ __forceinline__ void prologue(const Operand& A, const Operand& B, char* lds, LoadPlan<G>& lp) {
  lp.init(A, B);
  if constexpr (G::SA == 4) {
    // four A half-stages: A half 0, B of chunk 0, A halves 1 and 2 (the first
    // barrier waits for the first two, the k-step 1 one for half 1)
    constexpr int AH = LoadPlan<G>::A_LOADS / 2;
    static_for<AH>([&](auto i) { lp.template issue<i>(0, G::a_stage(lds, 0), nullptr); });
    static_for<G::IPW - 2 * AH>([&](auto i) { lp.template issue<2 * AH + i>(0, nullptr, G::b_stage(lds, 0)); });
    static_for<AH>([&](auto i) { lp.template issue<AH + i>(0, G::a_stage(lds, 1), nullptr); });
    static_for<AH>([&](auto i) { lp.template issue<i>(G::BK, G::a_stage(lds, 2), nullptr); });
    return;
  }
  static_for<G::IPW>([&](auto i) { lp.template issue<i>(0, G::a_stage(lds, 0), G::b_stage(lds, 0)); });
  // deeper rings: chunks 1 .. S - 2 as well
  if constexpr (G::S > 2) {
    for (int c = 1; c < G::S - 1; ++c)
      static_for<G::IPW>([&](auto i) { lp.template issue<i>(c * G::BK, G::a_stage(lds, c), G::b_stage(lds, c)); });
  }
  // three A stages: A's chunk 1 as well, issued last (the first barrier waits for all but it)
  if constexpr (G::SA == 3)
    static_for<LoadPlan<G>::A_LOADS>([&](auto i) { lp.template issue<i>(G::BK, G::a_stage(lds, 1), nullptr); });
}

// The k-loop of one tile whose chunk 0 was issued into stage p0 (chunk kt
// lives in stage (kt + p0) & 1).  With CHAIN and has_next, the last chunk's
// loads, which would otherwise read zeros past the end, fetch chunk 0 of the
// next tile instead: only the buffer descriptors differ between tiles of one
// launch (the per-lane offsets depend on the leading dimensions alone).  lp
// then describes the next tile and p0 names the stage its chunk 0 goes to;
// those loads are still in flight on return, and the caller keeps the ring
// untouched (and waits with wait_barrier, not __syncthreads) until the next
// call.  hook() runs once, after the first chunk's barrier: work issued there
// (the previous tile's global stores) is not waited for by that barrier.
// With VMF > 0 and vmf_first, the first chunk's barrier waits only until at
// most VMF vector-memory operations are outstanding: the caller issued at
// least VMF of them (the previous tile's global stores) after this tile's
// chunk-0 loads, and vector-memory operations complete in issue order, so the
// loads have landed while the stores still drain.
struct NoHook {
  __device__ __forceinline__ void operator()() const {}
};
template <class G, bool ZERO, bool CHAIN, class Hook = NoHook, int VMF = 0, class FH = NoFragHook>
__device__ __forceinline__ void mainloop_core(LoadPlan<G>& lp, __amdgpu_buffer_rsrc_t ra_next,
                                              __amdgpu_buffer_rsrc_t rb_next, bool has_next, int K, char* lds,
                                              int& p0, f32x16 (&acc)[G::FM][G::FN], const Hook& hook = Hook(),
                                              bool vmf_first = false, const FH& fh = FH()) {
  static_assert(G::NS == 4, "four k-steps per chunk");
  static_assert(G::SA == 2 || !CHAIN, "three A stages: one tile per call");
  static_assert(G::S == 2 || (!CHAIN && VMF == 0), "deeper rings: one tile per call");
  // S stages: at chunk kt's barrier the loads of chunks kt + 1 .. kt + S - 2
  // (issued later, all of them by now) may still be in flight
  constexpr int VMS = (G::S - 2) * G::IPW;
  static_assert(VMS < 64, "vmcnt range");
  static_assert(G::SA != 4, "four A half-stages: the rolling schedule only");
  if constexpr (ZERO) {
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int j = 0; j < G::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }
  constexpr int BK = G::BK;
  constexpr int LA = LoadPlan<G>::A_LOADS;
  constexpr int L1 = G::IPW / 2, L2 = G::IPW;  // loads issued in k-steps 0 and 1
  static_assert(G::IPW % 2 == 0 && (G::SA == 2 || LA == L1), "even load split");
  // Two A stages: chunk kt + 1's A loads in k-step 0, its B loads in k-step 1.
  // Three: chunk kt + 1's B loads in k-step 0, then chunk kt + 2's A loads in
  // k-step 1 (A streams from HBM: one chunk more of lead time).
  constexpr int S0A = G::SA == 2 ? 0 : LA, S0B = G::SA == 2 ? L1 : L2;
  constexpr int S1A = G::SA == 2 ? L1 : 0, S1B = G::SA == 2 ? L2 : LA;
  const int nk = (K + BK - 1) / BK;
  Frags<G> f0, f1;
  for (int kt = 0; kt < nk; ++kt) {
    // chunk kt landed (three A stages: all but the A loads of chunk kt + 1,
    // issued last); every wave is done with the stages refilled below
    if constexpr (G::SA == 3)
      wait_barrier<LA>();
    else if (VMF > 0 && kt == 0 && vmf_first)
      wait_barrier<VMF>();
    else
      wait_barrier<VMS>();
    lgkm_wait<0>(f1);   // f1 (the last step of chunk kt-1) landed before its MFMAs
    sched_fence();
    char *ca, *cb, *na, *nb;
    if constexpr (G::SA == 2 && G::S > 2) {
      // chunk kt in stage kt % S; this chunk loads chunk kt + S - 1 into
      // stage (kt - 1) % S, whose chunk every wave finished before the barrier
      ca = G::a_stage(lds, kt % G::S);
      cb = G::b_stage(lds, kt % G::S);
      na = G::a_stage(lds, (kt + G::S - 1) % G::S);
      nb = G::b_stage(lds, (kt + G::S - 1) % G::S);
    } else if constexpr (G::SA == 2) {
      ca = G::a_stage(lds, (kt + p0) & 1);
      cb = G::b_stage(lds, (kt + p0) & 1);
      na = G::a_stage(lds, (kt + p0 + 1) & 1);
      nb = G::b_stage(lds, (kt + p0 + 1) & 1);
    } else {
      ca = G::a_stage(lds, kt % 3);
      cb = G::b_stage(lds, kt & 1);
      na = G::a_stage(lds, (kt + 2) % 3);
      nb = G::b_stage(lds, (kt + 1) & 1);
    }
    int k1 = (kt + (G::S - 1)) * BK;  // (so grouped, S = 2 compiles as the two-stage loop did)
    if constexpr (CHAIN) {
      if (kt + 1 == nk && has_next) {
        lp.ra = ra_next;
        lp.rb = rb_next;
        k1 = 0;
      }
    }
    const int k2 = G::SA == 2 ? k1 : (kt + 2) * BK;  // the chunk k-step 1 loads
    const FragReader<G> r0(ca, cb, 0), r1(ca, cb, 1), r2(ca, cb, 2), r3(ca, cb, 3);
    if (kt > 0) {
      mfma_step_rd<G, S0A, S0B, FH>(f1, acc, lp, k1, na, nb, r0, f0, fh);
    } else {
      read_frags<G>(ca, cb, 0, f0);
      static_for<S0B - S0A>([&](auto i) { lp.template issue<S0A + i>(k1, na, nb); });
      hook();
    }
    lgkm_wait<0>(f0);
    sched_fence();
    mfma_step_rd<G, S1A, S1B, FH>(f0, acc, lp, k2, na, nb, r1, f1, fh);
    lgkm_wait<0>(f1);
    sched_fence();
    mfma_step_rd<G, 0, 0, FH>(f1, acc, lp, 0, lds, lds, r2, f0, fh);
    lgkm_wait<0>(f0);
    sched_fence();
    mfma_step_rd<G, 0, 0, FH>(f0, acc, lp, 0, lds, lds, r3, f1, fh);
    sched_fence();
  }
  lgkm_wait<0>(f1);
  sched_fence();
  mfma_step<G, 0, 0, FH>(f1, acc, lp, 0, lds, lds, fh);
  if constexpr (CHAIN) p0 = (p0 + nk) & 1;
}

// every outstanding global->LDS load landed (before the ring is reused for
// anything else, and before the workgroup ends)
__device__ __forceinline__ void drain_loads() {
  __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8) | (0 << 14));
}

// The k-loop with a split k (G::KS = 2): the waves of k-group g take k-steps
// 2g and 2g + 1 of every chunk, so that each SIMD runs two waves of one
// sub-tile.  One wave per SIMD serialises its MFMAs with its own operand
// reads, loads and address arithmetic (measured on the 64 x 64 fp32 tiles:
// the k-loop took the sum of the MFMA time and the time of the same loop with
// the MFMAs removed); with two, one wave's other work issues while the
// other's MFMAs run.  Otherwise mainloop_core's schedule for an S-stage ring:
// chunk kt in stage kt % S, chunk kt + S - 1 loaded during chunk kt (this
// wave's load 0 in its first k-step, load 1 in its second), fragment sets f0
// and f1 alternating, loads also past the last chunk (they read zeros).
template <class G, class FH = NoFragHook>
__device__ __forceinline__ void mainloop_ks2(LoadPlan<G>& lp, int K, char* lds, f32x16 (&acc)[G::FM][G::FN],
                                             const FH& fh = FH()) {
  static_assert(G::KS == 2 && G::NS == 4 && G::SA == 2 && G::IPW == 2, "split k: 2 x 2 k-steps, 2 loads a wave");
  constexpr int VMS = (G::S - 2) * G::IPW;
#pragma unroll
  for (int i = 0; i < G::FM; ++i)
#pragma unroll
    for (int j = 0; j < G::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  constexpr int BK = G::BK;
  const int s0 = 2 * G::wave_k();
  const int nk = (K + BK - 1) / BK;
  Frags<G> f0, f1;
  for (int kt = 0; kt < nk; ++kt) {
    wait_barrier<VMS>();
    lgkm_wait<0>(f1);
    sched_fence();
    char* ca = G::a_stage(lds, kt % G::S);
    char* cb = G::b_stage(lds, kt % G::S);
    char* na = G::a_stage(lds, (kt + G::S - 1) % G::S);
    char* nb = G::b_stage(lds, (kt + G::S - 1) % G::S);
    const int k1 = (kt + (G::S - 1)) * BK;
    const FragReader<G> r0(ca, cb, s0), r1(ca, cb, s0 + 1);
    if (kt > 0) {
      mfma_step_rd<G, 0, 1, FH>(f1, acc, lp, k1, na, nb, r0, f0, fh);
    } else {
      read_frags<G>(ca, cb, s0, f0);
      lp.template issue<0>(k1, na, nb);
    }
    lgkm_wait<0>(f0);
    sched_fence();
    mfma_step_rd<G, 1, 2, FH>(f0, acc, lp, k1, na, nb, r1, f1, fh);
    sched_fence();
  }
  lgkm_wait<0>(f1);
  sched_fence();
  mfma_step<G, 0, 0, FH>(f1, acc, lp, 0, lds, lds, fh);
}

// Split k: k-group 1's accumulators added to k-group 0's through LDS (over
// the ring, after every wave's last ring read and load), acc(0) + acc(1) in
// that order; the waves of group 0 then hold the tile's sums.  The ring is
// scratch afterwards (callers reuse it only after a barrier of their own).
template <class G>
__device__ __forceinline__ void ks_reduce(char* lds, f32x16 (&acc)[G::FM][G::FN]) {
  static_assert(G::KS == 2, "split k");
  constexpr int NB = G::FM * G::FN;
  static_assert(G::WM * G::WN * NB * 16 * 64 * 4 <= G::LDS_BYTES, "one k-group's accumulators fit the ring");
  float* buf = (float*)lds;
  const int lane = threadIdx.x & 63, wmn = G::wave_mn(), g = G::wave_k();
  __syncthreads();
  if (g == 1) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) buf[((wmn * NB + b) * 16 + r) * 64 + lane] = acc[b / G::FN][b % G::FN][r];
  }
  __syncthreads();
  if (g == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[b / G::FN][b % G::FN][r] += buf[((wmn * NB + b) * 16 + r) * 64 + lane];
  }
}

// One tile: chunk 0 into stage 0, the k-loop, and the zero loads past the
// last chunk awaited before the caller reuses the ring.  Split k: the k-loop
// of mainloop_ks2 and ks_reduce (the sums in k-group 0).
template <class G, bool ZERO = true>
__device__ __forceinline__ void mainloop(const Operand& A, const Operand& B, int K, char* lds,
                                         f32x16 (&acc)[G::FM][G::FN]) {
  LoadPlan<G> lp;
  prologue<G>(A, B, lds, lp);
  if constexpr (G::KS == 2) {
    static_assert(ZERO, "split k: fresh accumulators");
    mainloop_ks2<G>(lp, K, lds, acc);
    drain_loads();
    ks_reduce<G>(lds, acc);
  } else {
    int p0 = 0;
    mainloop_core<G, ZERO, false>(lp, lp.ra, lp.rb, false, K, lds, p0, acc);
    drain_loads();
  }
}

// ------------------------------------------------- rolling operand schedule
// For per-wave sub-tiles whose accumulators leave no room for two fragment
// sets (the 256 x 384 contraction tiles: 192 accumulator registers per wave):
// one fragment set.  A k-step's MFMAs run over the outer operand's fragments
// (the one with fewer fragments per wave), each against every inner fragment;
// the next k-step's read of a fragment is issued right after the MFMA that
// last uses it, into the same registers:
//   outer fragment o < NO - 1  after MFMA o NI + NI - 1,
//   inner fragment l           after MFMA (NO - 1) NI + l,
//   the last outer fragment    after the last MFMA,
// so every read is issued at least NI - 1 MFMAs before its first use, and
// each MFMA waits (lgkmcnt) only for the reads it needs.  The workgroup
// barriers sit in k-steps 1 and 3 after their first NI MFMAs (SPLIT), before
// the first read from the next A half-stage, and loads follow them.
template <class G>
struct RollSched {
  static constexpr int FM = G::FM, FN = G::FN, NMF = G::NMF;
  static constexpr int NA = G::TA ? 2 : 1;     // LDS reads per A fragment (transposed: low and high k)
  static constexpr bool AOUT = FM <= FN;       // A the outer operand (MFMA m = i FN + j), else B (m = j FM + i)
  static constexpr int NO = AOUT ? FM : FN, NI = AOUT ? FN : FM;
  static constexpr int RO = AOUT ? NA : 1, RI = AOUT ? 1 : NA;  // reads per outer / inner fragment
  static constexpr int NR = NO * RO + NI * RI;  // reads per k-step
  static constexpr int SPLIT = NI;              // MFMAs of k-step 3 before the barrier
  static_assert(NR <= 15, "lgkmcnt range");
  static_assert(G::KIND != K_F32 && NMF == FM * FN && NO >= 2, "16-bit MFMAs, one per 32 x 32 block");
  // MFMA m: blocks (i, j)
  static constexpr int mi(int m) { return AOUT ? m / FN : m % FM; }
  static constexpr int mj(int m) { return AOUT ? m % FN : m / FM; }
  // read r in issue order: outer fragments 0 .. NO - 2, the inner ones, the
  // last outer one; per fragment its reads (transposed A: half 0, 1)
  static constexpr int R1 = (NO - 1) * RO, R2 = R1 + NI * RI;
  static constexpr bool outer(int r) { return r < R1 || r >= R2; }
  static constexpr int frag(int r) { return r < R1 ? r / RO : (r < R2 ? (r - R1) / RI : NO - 1); }
  static constexpr int half(int r) { return r < R1 ? r % RO : (r < R2 ? (r - R1) % RI : (r - R2) % RO); }
  static constexpr bool is_a(int r) { return outer(r) == AOUT; }
  static constexpr int pos(int r) {
    return r < R1 ? frag(r) * NI + NI - 1 : (r < R2 ? (NO - 1) * NI + frag(r) : NMF - 1);
  }
  // index of the last read of outer fragment o / inner fragment l
  static constexpr int last_o(int o) { return o < NO - 1 ? (o + 1) * RO - 1 : NR - 1; }
  static constexpr int last_i(int l) { return R1 + (l + 1) * RI - 1; }
  static constexpr int last_a(int i) { return AOUT ? last_o(i) : last_i(i); }
  static constexpr int last_b(int j) { return AOUT ? last_i(j) : last_o(j); }
  // index of the last read that MFMAs 0..m need
  static constexpr int need(int m) {
    int l = -1;
    for (int u = 0; u <= m; ++u) {
      const int a = last_a(mi(u)), b = last_b(mj(u));
      l = a > l ? a : l;
      l = b > l ? b : l;
    }
    return l;
  }
  static constexpr int issued_before(int m) {
    int c = 0;
    for (int r = 0; r < NR; ++r) c += pos(r) < m ? 1 : 0;
    return c;
  }
};

// Per-lane LDS addresses of the rolling reads, for A's half-slot 0 and B's
// stage 0 (the reads add half-slot h's h * A_STAGE / 2 and stage p's p *
// B_STAGE); the k-step and the fragment are instruction offsets.
template <class G>
struct RollReader {
  static_assert(G::GB && G::ESZ == 2 && G::SA == 4 && G::NS == 4, "blocked 16-bit A, four A half-stages, four k-steps");
  uint32_t a[2];  // A: transposed, read half 0 / 1; else the slot of even / odd k-steps
  uint32_t b[4];  // B: k-step 0..3
  __device__ __forceinline__ explicit RollReader(char* lds) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (G::TA) {
        a[h] = lds_off(ta_ptr<G>(G::a_stage(lds, 0), 0, 0, h));
      } else {
        // a_ptr of k-step h (0 or 1); k-steps 2 and 3 are in the next half-slot
        a[h] = lds_off(a_ptr<G>(G::a_stage(lds, 0), h)) - h * 1024;
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) b[s] = lds_off(b_ptr<G>(G::b_stage(lds, 0), s));
  }
  template <int S, int R>
  __device__ __forceinline__ void read(Frags<G>& f, uint32_t sa, uint32_t sb) const {
    using RS = RollSched<G>;
    constexpr int fr = RS::frag(R);
    if constexpr (RS::is_a(R)) {
      if constexpr (G::TA) {
        // fragment i is 2 KB further, k-steps as in ta_ptr
        constexpr int off = fr * 2048 + (S & 1) * 256;
        static_assert(off < 65536, "ds offset");
        i16x4_t v;
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(a[RS::half(R)] + sa), "n"(off) : "memory");
        if constexpr (RS::half(R) == 0)
          f.a[fr].lo = v;
        else
          f.a[fr].hi = v;
      } else {
        f.a[fr] = lds_read_b128<(S & 1) * 1024 + fr * 2048>(a[S & 1] + sa);
      }
    } else {
      f.b[fr] = lds_read_b128<fr * 32 * G::ROWB>(b[S] + sb);
    }
  }
};

// MFMAs [M0, M1) of k-step `S` (fragments f), each after the wait for the
// reads it needs.  READ: the reads of k-step SN (A's and B's stage offsets
// sna, snb) are issued at their positions (and those at position M0 - 1
// first).  ld(q), q < NL: the range's loads, one after each of its first MFMAs.
template <class G, int S, bool READ, int SN, int M0, int M1, int NL, class LD>
__device__ __forceinline__ void roll_range(Frags<G>& f, f32x16 (&acc)[G::FM][G::FN], const RollReader<G>& rd,
                                           uint32_t sna, uint32_t snb, const LD& ld) {
  using RS = RollSched<G>;
  static_assert(NL <= M1 - M0, "one load per MFMA");
  if constexpr (READ && M0 > 0) {
    static_for<RS::NR>([&](auto rc) {
      if constexpr (RS::pos(rc) == M0 - 1) rd.template read<SN, rc>(f, sna, snb);
    });
  }
  static_for<M1 - M0>([&](auto mc) {
    constexpr int m = M0 + mc;
    constexpr int i = RS::mi(m), j = RS::mj(m);
    if constexpr (m == M0 || RS::need(m) > RS::need(m - 1)) {
      // reads of k-step S still allowed in flight, plus those of SN issued so far
      constexpr int n = RS::NR - 1 - RS::need(m) + (READ ? RS::issued_before(m) : 0);
      sched_fence();
      asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(n) : "memory");
      // every fragment tied to the wait: no MFMA is scheduled above it
#pragma unroll
      for (int u = 0; u < G::FM; ++u) asm volatile("" : "+v"(f.a[u]));
#pragma unroll
      for (int u = 0; u < G::FN; ++u) asm volatile("" : "+v"(f.b[u]));
      sched_fence();
    }
    acc[i][j] = mfma16_32x32x16<G::F16>(f.a[i], f.b[j], acc[i][j]);
    if constexpr (READ || (mc < NL)) {
      sched_fence();
      if constexpr (READ)
        static_for<RS::NR>([&](auto rc) {
          if constexpr (RS::pos(rc) == m) rd.template read<SN, rc>(f, sna, snb);
        });
      if constexpr (mc < NL) ld(mc);
      sched_fence();
    }
  });
}

// One tile on the rolling schedule (not chained): the first chunk and a
// half, the k-loop, the zero loads past the last chunk awaited (ZERO = false:
// added to acc).
//
// A (streamed from HBM) in four half-stages, B in two stages: half h of A
// (k-steps 2 (h % 2) and + 1 of chunk h / 2) lives in half-slot h % 4.  A
// second barrier, in k-step 1 of chunk kt, frees the half-slot of chunk kt's
// k-steps 0-1 for half 2 kt + 4; the barrier in k-step 3 also frees the other
// half-slot, for half 2 kt + 5, beside B's stage for chunk kt + 2.  Every A
// half then has a chunk and a half of lead.  Per wave the loads go out as
// groups [B(kt + 2), A(2 kt + 5)] (from the k-step 3 barrier of chunk kt on,
// the rest in k-step 0 of chunk kt + 1) and A(2 kt + 4) (after the k-step 1
// barrier); vector-memory loads complete in issue order, so the k-step 3
// barrier of chunk kt + 1, which needs B(kt + 1) and A(2 kt + 2), waits until
// at most A(2 kt + 3) and A(2 kt + 4) (A_LOADS loads) are outstanding,
// and the k-step 1 barrier of chunk kt + 1, which needs A(2 kt + 3), until at
// most A(2 kt + 4) and the group [B(kt + 2), A(2 kt + 5)] are.
template <class G, bool ZERO = true>
__device__ __forceinline__ void mainloop_roll(const Operand& A, const Operand& B, int K, char* lds,
                                              f32x16 (&acc)[G::FM][G::FN]) {
  using RS = RollSched<G>;
  constexpr int SPL = RS::SPLIT, NMF = G::NMF, BK = G::BK;
  if constexpr (ZERO) {
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int j = 0; j < G::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }
  LoadPlan<G> lp;
  prologue<G>(A, B, lds, lp);
  const RollReader<G> rd(lds);
  Frags<G> f;
  const int nk = (K + BK - 1) / BK;
  const auto none = [](auto) {};
  static_assert(G::SA == 4, "four A half-stages");
  {  // (scope of the schedule's constants)
    constexpr int AH = LoadPlan<G>::A_LOADS / 2, NB = G::IPW - 2 * AH;
    constexpr int NX = NB + AH;        // the k-step 3 barrier's group
    // its loads after the barrier, the rest in k-step 0 (a quarter after the
    // barrier measured best: the N = 262144, D = 1152 contraction 0.8-1.2%
    // faster than with half, 2-3% faster than with none or all)
    constexpr int XH = NX / 4;
    constexpr int WX = 2 * AH, WY = AH + NX;  // vmcnt of the two barriers
    static_assert(XH <= NMF - SPL && NX - XH <= NMF && AH <= NMF - SPL, "load slots");
    constexpr uint32_t HALF = G::A_STAGE / 2;
    // group load q of chunk kc (B first, then A's second half), half-slot / stage parity c
    const auto xload = [&](auto q, int kc, int c) {
      constexpr int I = q < NB ? 2 * AH + q : AH + (q - NB);
      lp.template issue<I>(kc * BK, G::a_stage(lds, 2 * c + 1), G::b_stage(lds, c));
    };
    // k-steps 0..2 and the first half of k-step 3 of chunk kt (parity c), the
    // first XH loads of chunk kt + 1's group already issued; then its barrier
    // and the second half of k-step 3, reading chunk kt + 1
    auto chunk = [&](int kt, int c) {
      const uint32_t a0 = 2 * c * HALF, a1 = a0 + HALF, sb = c * G::B_STAGE;
      roll_range<G, 0, true, 1, 0, NMF, NX - XH>(f, acc, rd, a0, sb,
                                                  [&](auto q) { xload(std::integral_constant<int, XH + q>{}, kt + 1, c ^ 1); });
      roll_range<G, 1, false, 2, 0, SPL, 0>(f, acc, rd, 0, 0, none);
      // every wave is done with half 2 kt; half 2 kt + 1 landed
      wait_barrier<WY>();
      sched_fence();
      roll_range<G, 1, true, 2, SPL, NMF, AH>(f, acc, rd, a1, sb, [&](auto q) {
        lp.template issue<q>((kt + 2) * BK, G::a_stage(lds, 2 * c), nullptr);
      });
      roll_range<G, 2, true, 3, 0, NMF, 0>(f, acc, rd, a1, sb, none);
      roll_range<G, 3, false, 0, 0, SPL, 0>(f, acc, rd, 0, 0, none);
      // chunk kt + 1's B and first A half landed; every wave is done with
      // chunk kt's B and A half 2 kt + 1
      wait_barrier<WX>();
      sched_fence();
      roll_range<G, 3, true, 0, SPL, NMF, XH>(f, acc, rd, a0 ^ (2 * HALF), sb ^ G::B_STAGE,
                                              [&](auto q) { xload(q, kt + 2, c); });
    };
    // chunk 0's B and first A half landed: its k-step 0 reads, then chunk 1's group
    wait_barrier<WX>();
    sched_fence();
    static_for<RS::NR>([&](auto rc) { rd.template read<0, rc>(f, 0, 0); });
    static_for<XH>([&](auto q) { xload(q, 1, 1); });
    sched_fence();
    for (int kt = 0; kt < nk - 1; ++kt) chunk(kt, kt & 1);
    {
      // the last chunk: no further barrier in k-step 3 (nothing else is read)
      const int kt = nk - 1, c = kt & 1;
      const uint32_t a0 = 2 * c * HALF, a1 = a0 + HALF, sb = c * G::B_STAGE;
      roll_range<G, 0, true, 1, 0, NMF, NX - XH>(f, acc, rd, a0, sb,
                                                  [&](auto q) { xload(std::integral_constant<int, XH + q>{}, kt + 1, c ^ 1); });
      roll_range<G, 1, false, 2, 0, SPL, 0>(f, acc, rd, 0, 0, none);
      wait_barrier<WY>();
      sched_fence();
      roll_range<G, 1, true, 2, SPL, NMF, 0>(f, acc, rd, a1, sb, none);
      roll_range<G, 2, true, 3, 0, NMF, 0>(f, acc, rd, a1, sb, none);
      roll_range<G, 3, false, 0, 0, NMF, 0>(f, acc, rd, 0, 0, none);
    }
  }
  drain_loads();
}

}  // namespace gdma
}  // namespace mec
