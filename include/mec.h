/*
 * mec.h — C ABI of the MI355X (gfx950) memory-efficient CLIP / LiT loss.
 *
 * This library replaces the four Triton kernels and the PyTorch glue of the
 * reference's autograd Functions (b0nce/MemoryEfficientCLIP):
 *   clip_sum_exp_kernel   clip_loss.py:9-64      -> mec_sumexp   (mode CLIP)
 *   lit_sum_exp_kernel    lit_loss.py:9-62       -> mec_sumexp   (mode LIT)
 *   forward epilogue      clip_loss.py:199-213,
 *                         lit_loss.py:192-205    -> mec_finalize
 *   clip_grad_kernel      clip_loss.py:67-156    -> mec_grad     (mode CLIP)
 *   lit_grad_kernel       lit_loss.py:65-148     -> mec_grad     (mode LIT)
 *   backward pro/epilogue clip_loss.py:234-256,
 *                         lit_loss.py:226-247    -> mec_postpass
 *   F.normalize(dim=1)    clip_loss.py:266-268,
 *                         lit_loss.py:257-259    -> fused: mec_prepass + mec_postpass
 *                                                   with normalize = 1
 *   Function.forward      clip_loss.py:159-213   -> mec_forward  (prepass+sumexp+finalize)
 *   Function.backward     clip_loss.py:215-256   -> mec_backward (grad+postpass)
 *
 * The reference has no FFI of its own: its boundary is the PyTorch
 * autograd.Function (clip_loss.py:159, lit_loss.py:151).  These entry points
 * are what that Function calls here, through ctypes
 * (memoryefficientclip_amd/_lib.py).
 *
 * Conventions
 *   - Every function returns MEC_OK (0) or a negative MEC_ERR_* code and never
 *     throws.  mec_last_error() returns a thread-local description of the
 *     last failure on the calling thread.
 *   - Pointers are device pointers.  x and y are row-major [n, d] with row
 *     strides ldx, ldy (in elements, >= d) and unit column stride.
 *     x is the row side of S = x^ y^T: image for CLIP, text for LiT.
 *   - dtype: MEC_DTYPE_F32 (float), MEC_DTYPE_BF16 (uint16 bfloat16 bits),
 *     MEC_DTYPE_F16 (uint16 IEEE binary16 bits), or float data with products
 *     formed from bf16 terms: MEC_DTYPE_F32_BF16X3, MEC_DTYPE_F32_BF16 (below).  All arithmetic
 *     accumulates in fp32; the loss is reduced in fp64.  Sizes: 1 <= d <= 2^20
 *     (MEC_ERR_INVALID beyond) and 1 <= n <= 2^22 for every dtype
 *     (MEC_ERR_UNSUPPORTED beyond, returned before any launch).  Memory
 *     bounds n further: the caller holds the inputs, the workspace, two fp32
 *     n x d accumulators and the gradient scratch (mec_grad_scratch_bytes;
 *     16 GiB at n = 2^21, d = 1152, fp32).  Rows that are 16-byte aligned
 *     (x, y 16-byte aligned, d, ldx, ldy multiples of 8 elements for the
 *     16-bit types, 4 for fp32) use the direct-to-LDS tiles; other layouts
 *     are supported at lower speed.
 *   - mode: MEC_MODE_CLIP or MEC_MODE_LIT, optionally OR
 *     MEC_FLAG_DETERMINISTIC (every function accepts it; only the forward
 *     sums, mec_sumexp and mec_forward, depend on it) and MEC_FLAG_KEEP_EXP
 *     (small fp32 problems; see there).
 *   - All work is enqueued on `stream` (a hipStream_t; NULL = default
 *     stream), which must belong to the current HIP device (the device of
 *     the data; the forward sizes its persistent launches by that device's
 *     compute units).  No function synchronises the host and none allocates
 *     device memory: the workspace and the gradient scratch are caller-owned.
 *   - HIP graph capture is not supported: a function called on a stream that
 *     is being captured (hipStreamIsCapturing, including a legacy default
 *     stream joined to another stream's capture) returns
 *     MEC_ERR_UNSUPPORTED before any launch.  A captured step of this loss
 *     ended in a host segmentation fault during graph instantiation on
 *     MI355X, with no cause found in these launches.
 *   - Argument validation is pure host code; invalid arguments are reported
 *     before anything touches the GPU.
 *   - Resident device memory: the library's code object holds the
 *     MEC_NOALLOC_SCRATCH_BYTES (256 MiB) array of mec_backward_noalloc, so
 *     every GPU on which any function of this library runs carries those
 *     256 MiB for the life of the process, whether or not
 *     mec_backward_noalloc is ever called.  PyTorch's allocator statistics do
 *     not include it.
 */
#ifndef MEC_H_
#define MEC_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MEC_OK 0
#define MEC_ERR_INVALID (-1)     /* bad argument (null pointer, size, enum) */
#define MEC_ERR_UNSUPPORTED (-2) /* valid but not supported by this build */
#define MEC_ERR_HIP (-3)         /* a HIP runtime call failed */

#define MEC_DTYPE_F32 0
#define MEC_DTYPE_BF16 1
#define MEC_DTYPE_F16 2
/* fp32 inputs and outputs (as MEC_DTYPE_F32), with every product of the
 * similarity GEMMs and the gradient contractions formed as
 * hi_a hi_b + lo_a hi_b + hi_a lo_b on the bf16 MFMA, where hi = bf16(v) and
 * lo = bf16(v - hi) (about 16 significant bits per operand; the error of one
 * product is at most about 3 * 2^-16 of it), accumulated in fp32.  The norms,
 * the diagonal and the post-pass stay in fp32.  This is PyTorch's "high"
 * float32 matmul precision (torch.set_float32_matmul_precision), and plays
 * the role of the TF32 dot products the reference gets from Triton on NVIDIA
 * (clip_loss.py:53,113,148-149 pass no input_precision).  No counterpart
 * dtype in the reference.  The workspace is larger (mec_workspace_floats_for)
 * and must be 16-byte aligned; mec_sumexp and mec_grad_step read split copies
 * of x and y that mec_prepass writes into it. */
#define MEC_DTYPE_F32_BF16X3 3
/* fp32 inputs and outputs with the products of the similarity GEMMs and the
 * contractions in plain bf16 (bf16(a) bf16(b), fp32 accumulate): PyTorch's
 * "medium" float32 matmul precision.  Errors are those of bf16 inputs (the
 * bf16 tolerances); the norms, the diagonal and the post-pass stay fp32.
 * Workspace and scratch as for MEC_DTYPE_F32_BF16X3 (one term instead of
 * three). */
#define MEC_DTYPE_F32_BF16 4

#define MEC_MODE_CLIP 0 /* symmetric image<->text loss, gradients for x and y */
#define MEC_MODE_LIT 1  /* text->image only (x = text), gradient for x only */
#define MEC_MODE_MASK 0xff
/* OR into `mode`: the forward sums are formed without atomics across
 * workgroups, in a fixed order, so the loss and (through the sums) the
 * gradients are bitwise reproducible for the same inputs on the same device.
 * The backward is deterministic in either mode.  The similarity tiles are
 * still visited once (in P x Q blocks), with the partial sums combined in a
 * fixed order by a second, O(n) launch.  The 16-bit forward with 16-byte rows
 * and normalize = 0, and the forward of MEC_DTYPE_F32_BF16X3 /
 * MEC_DTYPE_F32_BF16 (on normalized copies), always run this way (chained
 * tiles; faster than the atomic forward there), with or without the flag. */
#define MEC_FLAG_DETERMINISTIC 0x100
/* OR into `mode` of mec_forward and of the matching mec_grad / mec_backward
 * (mec_backward_noalloc) for a small problem that mec_keep_exp_supported
 * accepts: the forward keeps the similarity matrix in the workspace, np x np
 * floats (np = n rounded up to 64), and turns it into H = diag(rx) G'
 * diag(ry) once the sums are known, together with per-block sums of
 * G'_ij cos_ij for the normalisation backward; the backward contracts H
 * instead of recomputing the similarity tiles.  The forward is then two
 * launches (similarity tiles, which also form the norms and the diagonal;
 * finalize), mec_backward one (the contractions with the post-pass in their
 * epilogue; mec_grad + mec_postpass: two), and the backward needs no
 * gradient scratch.  Both passes are deterministic
 * (fixed-order sums) with or without MEC_FLAG_DETERMINISTIC.  The workspace
 * must hold mec_workspace_floats_mode(n, d, dtype, mode) floats and be 16-byte
 * aligned; the flag must be passed to both calls or to neither.  No
 * counterpart in the reference, whose backward always recomputes
 * (clip_loss.py:96-124): this trades np^2 floats of workspace, held from the
 * forward to the backward, for one similarity GEMM, and is limited to
 * n <= MEC_KEEP_EXP_MAX_N.  The functions that run one stage (mec_sumexp,
 * mec_finalize, mec_grad_step) reject the flag. */
#define MEC_FLAG_KEEP_EXP 0x200
#define MEC_KEEP_EXP_MAX_N 2048

/* Sides of the backward, for the size queries: the x side (acc_x, dx) and
 * the y side (acc_y, dy; CLIP only).  mec_grad and friends compute the sides
 * whose accumulators are non-NULL. */
#define MEC_SIDE_X 1
#define MEC_SIDE_Y 2

/* Thread-local message for the last error on this thread ("" if none). */
const char* mec_last_error(void);

/* Library version string. */
const char* mec_version(void);

/* Number of floats of the per-call workspace: 8 vectors of length n
 * (inverse norms rx, ry; raw diagonal x_i.y_i; off-diagonal row/column sums
 * of E = exp((S-1)/T); 1/R; 1/C; diagonal gradient coefficient), then
 * ceil(n/256) doubles of loss partials (mec_finalize), then 48 x n floats
 * of partial sums (the deterministic forward, MEC_FLAG_DETERMINISTIC).  The
 * workspace must be 8-byte aligned.  The same workspace must be passed to
 * mec_forward and the matching mec_backward (it replaces
 * ctx.save_for_backward of the sums, clip_loss.py:199).  Enough for
 * MEC_DTYPE_F32, MEC_DTYPE_BF16 and MEC_DTYPE_F16 only: the two bf16-product
 * dtypes (MEC_DTYPE_F32_BF16X3, MEC_DTYPE_F32_BF16) keep bf16 copies of x and
 * y in the workspace as well and need mec_workspace_floats_for(n, d, dtype),
 * which is correct for every dtype.  Returns < 0 for n outside [1, 2^22]. */
int64_t mec_workspace_floats(int64_t n);

/* Number of floats of the workspace for (n, d, dtype): mec_workspace_floats(n)
 * for fp32, bf16 and fp16; for MEC_DTYPE_F32_BF16X3 (MEC_DTYPE_F32_BF16) that,
 * rounded up to 4 floats, plus split copies of x and y: 2 n rows of
 * 3 * round8(d) (round8(d)) bf16.  Returns < 0 on bad args.  No counterpart
 * in the reference. */
int64_t mec_workspace_floats_for(int64_t n, int64_t d, int dtype);

/* Number of floats of the workspace for (n, d, dtype, mode):
 * mec_workspace_floats_for(n, d, dtype), plus, with MEC_FLAG_KEEP_EXP in
 * mode, the kept matrix (np x np floats), 4 np^2 / 64 floats of per-tile
 * row and column sums (of E, and of G'_ij cos_ij) and one 64-bit loss
 * accumulator (np = n rounded up to 64), each part 256-byte aligned.
 * Returns < 0 on bad
 * args, or for MEC_FLAG_KEEP_EXP with a dtype other than MEC_DTYPE_F32 or
 * n > MEC_KEEP_EXP_MAX_N.  No counterpart in the reference. */
int64_t mec_workspace_floats_mode(int64_t n, int64_t d, int dtype, int mode);

/* 1 if mec_forward / mec_backward accept MEC_FLAG_KEEP_EXP for these inputs
 * (MEC_DTYPE_F32, n <= MEC_KEEP_EXP_MAX_N, 16-byte aligned rows: x and y
 * 16-byte aligned, d, ldx and ldy multiples of 4), else 0 (also for invalid
 * arguments).  Host-only.  No counterpart in the reference. */
int mec_keep_exp_supported(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                           int dtype);

/* Bytes of gradient scratch that mec_grad / mec_grad_step / mec_backward
 * need for (n, d, dtype, mode, sides), sides a mask of MEC_SIDE_X and
 * MEC_SIDE_Y (LiT: the x side only).  The layout, in the scratch element type
 * (fp32 for MEC_DTYPE_F32, 16 bits for every other dtype):
 *   - the gradient-matrix buffers: one block diagonal of the off-diagonal
 *     gradient matrix (nb blocks of bs x bs), double-buffered (one buffer
 *     when a single block covers n).  fp32 keeps H = diag(rx) G' diag(ry)
 *     once, row-major; the 16-bit types keep G'^T in a blocked layout
 *     (bf16x3: hi and lo planes);
 *   - the 16-bit types (and the bf16-product modes) only: transposed
 *     normalised copies of the inputs, [d][n rounded up to 128], one for each
 *     side computed (bf16x3: hi and lo planes).  fp32 reads its raw inputs.
 * bs targets ~4d rows for fp32 and ~8d for the other dtypes (~16d when
 * n >= 8192 and 8d would give fewer than 16 blocks; at most 16384 rows for
 * fp32 and 32512 for the 16-bit kernels), and is shortened, never below 128
 * (fp32) or 256 rows, until the gradient-matrix buffers fit
 * min(16 GiB, max(64 n d elem, 256 MiB)): O(n*d).  Examples: n = 32768,
 * d = 1152 fp32 CLIP 1.07 GB; LiT the same; n = 1024, d = 512 fp32 4.2 MB.
 * With MEC_FLAG_KEEP_EXP in mode: 0 (the backward contracts the kept
 * matrix); < 0 where the flag does not apply (dtype, n).
 * Returns < 0 on bad args or n outside [1, 2^22]. */
int64_t mec_grad_scratch_bytes_for(int64_t n, int64_t d, int dtype, int mode, int sides);

/* mec_grad_scratch_bytes_for(n, d, dtype, MEC_MODE_CLIP, MEC_SIDE_X | MEC_SIDE_Y):
 * enough for every mode and side. */
int64_t mec_grad_scratch_bytes(int64_t n, int64_t d, int dtype);

/* The backward's plan for (n, d, dtype, mode, sides) on a device of
 * `compute_units` CUs (<= 0: the current device's), for 16-byte aligned rows.
 * No counterpart in the reference; for callers sizing buffers and for tests
 * of the selection rules without a GPU. */
typedef struct mec_backward_plan_t {
  int64_t block_rows;            /* rows per block of the gradient matrix */
  int64_t num_blocks;            /* blocks (mec_grad runs num_blocks + 1 steps) */
  int64_t scratch_bytes;         /* mec_grad_scratch_bytes_for */
  int64_t noalloc_block_rows;    /* mec_backward_noalloc's block rows, -1 if it refuses the problem */
  int64_t noalloc_scratch_bytes; /* bytes of its array that it uses, -1 if it refuses the problem */
  int32_t contract_tile_rows;    /* contraction tile: output rows ... */
  int32_t contract_tile_features;/* ... and features (16-bit: 256 or 384) */
  int32_t narrow_tiles;          /* 16-bit: 512 x 128 tiles for a last column of <= 128 features */
  int32_t reserved;
} mec_backward_plan_t;
int mec_backward_plan(int64_t n, int64_t d, int dtype, int mode, int sides, int compute_units,
                      mec_backward_plan_t* plan);

/* Block decomposition of the backward for (n, d, dtype): the n x n gradient
 * matrix is cut into num_blocks^2 blocks of block_rows rows (the last block
 * may be short); mec_grad runs num_blocks + 1 pipeline steps.  No counterpart
 * in the reference (its backward grid is fixed at 64 x 64 tiles,
 * clip_loss.py:239-249); exposed so callers can size and drive the steps. */
int mec_grad_blocking(int64_t n, int64_t d, int dtype, int64_t* block_rows, int64_t* num_blocks);

/* rx, ry (1 if !normalize), diag; clears the sum accumulators.
 * MEC_DTYPE_F32_BF16X3, MEC_DTYPE_F32_BF16: also writes the bf16 (split)
 * copies of x and y into the workspace, normalized (x_i rx_i, y_j ry_j) when
 * normalize is set; mec_sumexp and the backward then run their GEMMs on
 * those copies, so every stage of one step takes the same normalize. */
int mec_prepass(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                int dtype, int normalize, float* workspace, void* stream);

/* Accumulates the off-diagonal sums sum_{j!=i} E_ij (and sum_{i!=j} E_ij for
 * CLIP) into the workspace.  Requires mec_prepass first. */
int mec_sumexp(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
               int dtype, int mode, int normalize, float temperature, float* workspace,
               void* stream);

/* Loss (fp32 scalar at *loss, device pointer) and the backward's per-row
 * vectors.  CLIP: mean over i of (CE_row_i + CE_col_i)/2; LiT: mean CE_row_i. */
int mec_finalize(int64_t n, int mode, float temperature, float* workspace, float* loss,
                 void* stream);

/* prepass + sumexp + finalize.  With MEC_FLAG_KEEP_EXP: the similarity
 * tiles (with the norms and the diagonal) and the finalize of the kept
 * matrix, two launches; the workspace then holds the scaled gradient matrix
 * for the backward. */
int mec_forward(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                int dtype, int mode, int normalize, float temperature, float* workspace,
                float* loss, void* stream);

/* Off-diagonal gradient contractions into fp32 accumulators [n, d]
 * (row stride d):  acc_x_i = sum_{j!=i} G'_ij y^_j,  acc_y_j = sum_{i!=j} G'_ij x^_i
 * with G'_ij = E_ij (1/R_i + 1/C_j) (LiT: E_ij / R_i; acc_y is ignored).
 * Replaces clip_grad_kernel (clip_loss.py:67-156) and lit_grad_kernel
 * (lit_loss.py:65-148).  A NULL accumulator skips that side (e.g. a frozen
 * tower); at least one is required.  scratch must hold
 * mec_grad_scratch_bytes_for(n, d, dtype, mode, sides) bytes for the sides
 * requested, 16-byte aligned.  MEC_DTYPE_F32: the accumulators hold the
 * contractions of H = diag(rx) G' diag(ry) with the raw inputs, i.e. row i of
 * acc_x is rx_i sum_j G'_ij y^_j (and acc_y's row j ry_j sum_i G'_ij x^_i;
 * rx = ry = 1 when normalize = 0), which mec_postpass expects for that dtype;
 * row strides up to 2^24 elements (MEC_ERR_UNSUPPORTED beyond).
 * Equivalent to mec_grad_step for step = 0 .. num_blocks in order.  With
 * MEC_FLAG_KEEP_EXP (as passed to mec_forward): one launch that contracts the
 * kept matrix, the same accumulators; scratch is not used and may be NULL. */
int mec_grad(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
             int dtype, int mode, int normalize, float temperature, const float* workspace,
             void* scratch, int64_t scratch_bytes, float* acc_x, float* acc_y, void* stream);

/* One pipeline step of mec_grad (one kernel launch): step t in
 * [0, num_blocks] recomputes the similarity blocks of block diagonal t and
 * stores their gradient-matrix blocks in scratch buffer t % 2, and contracts
 * diagonal t - 1 from the other buffer into the accumulators (step 1
 * overwrites them, later steps add).  Steps must run in order on one
 * stream with the same scratch. */
int mec_grad_step(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                  int dtype, int mode, int normalize, float temperature, const float* workspace,
                  int64_t step, void* scratch, int64_t scratch_bytes, float* acc_x, float* acc_y,
                  void* stream);

/* Final gradients from the accumulators (as mec_grad leaves them for the same
 * dtype and normalize): scale a = grad_scale/(2n) (LiT:
 * grad_scale/n), exact diagonal term, F.normalize backward when normalize,
 * times *grad_output (device fp32 scalar, NULL = 1), cast to dtype.
 * grad_scale is 1/T for the standard loss and sqrt(n/T) for the Stable
 * variants (clip_loss.py:182, :299).  dx/dy are row-major [n, d] (row
 * stride d) and may alias acc_x/acc_y when the data are fp32, i.e. for
 * MEC_DTYPE_F32, MEC_DTYPE_F32_BF16X3 and MEC_DTYPE_F32_BF16 (one wave
 * handles a row and reads each accumulator element before it writes that
 * element of the output).  A
 * side is skipped when both its accumulator and its output are NULL (LiT:
 * always y). */
int mec_postpass(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                 int dtype, int mode, int normalize, float grad_scale, const float* workspace,
                 const float* grad_output, const float* acc_x, const float* acc_y, void* dx,
                 void* dy, void* stream);

/* mec_grad + mec_postpass.  With MEC_FLAG_KEEP_EXP (as passed to
 * mec_forward): one launch, the contraction tiles applying the post-pass in
 * their epilogue; acc_x and acc_y are then not written (they may alias dx
 * and dy as above), and the normalisation backward's <x^_i, dx^_i> comes from
 * the finalize's block sums of G'_ij cos_ij rather than from a sum over the
 * features, so dx and dy equal mec_grad + mec_postpass's to fp32 rounding
 * (not bitwise). */
int mec_backward(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                 int dtype, int mode, int normalize, float temperature, float grad_scale,
                 const float* workspace, const float* grad_output, void* scratch,
                 int64_t scratch_bytes, float* acc_x, float* acc_y, void* dx, void* dy,
                 void* stream);

/* Bytes of the gradient scratch array of mec_backward_noalloc (256 MiB). */
#define MEC_NOALLOC_SCRATCH_BYTES (256LL << 20)

/* mec_backward without caller scratch and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc; not HIP graph
 * capture, which every function here refuses).  The gradient scratch is a
 * file-scope device array of MEC_NOALLOC_SCRATCH_BYTES on each GPU the
 * library runs on, held until the process ends (resident from the library's
 * first use on that GPU, see above); its address is resolved once per device
 * on the first call.  The blocking is mec_backward's when its scratch fits
 * the array, else shorter blocks (down to 128 rows for fp32, 256 for the
 * other dtypes); problems whose scratch does not fit even then return
 * MEC_ERR_UNSUPPORTED before any launch.  mec_backward_plan reports, for any
 * shape, whether it fits and with which blocks (the largest n at d = 1152,
 * CLIP: see the integration notes).  Nothing in the array needs to start at
 * zero.  Every call on one GPU uses the same array: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialised by the
 * caller.  Arguments and results otherwise as mec_backward. */
int mec_backward_noalloc(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                         int mode, int normalize, float temperature, float grad_scale, const float* workspace,
                         const float* grad_output, float* acc_x, float* acc_y, void* dx, void* dy, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MEC_H_ */
