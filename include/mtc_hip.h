/*
 * C-ABI of libmtc_hip.so: MI355X (gfx950) kernels for Y = X * W_hat, where
 * W_hat is a quadtree-tiled, per-leaf mixed-precision weight packed into a
 * device-resident "panel stream" (format below).
 *
 * Plain C types only; every device buffer is caller-owned; no entry point
 * allocates device memory. Launches are asynchronous on the given HIP stream
 * (NULL = default stream). Functions return 0 on success and a negative
 * MTC_E* code on failure; mtc_last_error() returns a thread-local message.
 * Calls that share one GEMV workspace must not overlap in time.
 *
 * Reference interfaces replaced (Sharexi/TensorPack, Python + numba, no FFI):
 *   mtc_gemv_f32   <- mtc/kernels/gemm.py:124-210 (mtc_gemm_core_kernel) as
 *                     driven by mtc_gemm, gemm.py:541-574, for decode shapes
 *   mtc_gemv_f32_group <- several LinearMTCAdaptive.forward calls on one input,
 *                     mtc/nn/layers.py:150-151 (X @ W per layer), e.g. the q/k/v or
 *                     gate/up projections of a decoder layer, in one launch
 *   mtc_gemm_bf16_group <- the same layer calls at prefill shapes
 *   mtc_gemm_bf16  <- same kernel/entry point, prefill shapes (bf16 MFMA), over
 *                     the tile stream (mtc_tile_desc)
 *   mtc_dequant    <- MTCMatrix.to_array, gemm.py:510-538, and
 *                     qt_dequant / permuted_qt_dequant, mtc/core/quadtree.py:157-171,
 *                     mtc/core/permutation.py:76-79
 *   mtc_rd_search  (libmtc_rd.so, host) <- _search_kernel, mtc/core/allocation.py:106-136
 */
#ifndef MTC_HIP_H
#define MTC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTC_ABI_VERSION 11

enum {
  MTC_OK = 0,
  MTC_E_NULL = -1,        /* a required pointer is NULL */
  MTC_E_DESC = -2,        /* malformed stream descriptor */
  MTC_E_SHAPE = -3,       /* M / leading dimension / chunk geometry not supported */
  MTC_E_DTYPE = -4,       /* unsupported dtype code */
  MTC_E_WORKSPACE = -5,   /* workspace missing or too small */
  MTC_E_LAUNCH = -6,      /* HIP launch / runtime error */
  MTC_E_VERSION = -7      /* descriptor from another ABI version */
};

enum { MTC_DTYPE_F32 = 0, MTC_DTYPE_BF16 = 1 };

/* Descriptor flags */
#define MTC_FLAG_FP32_SCALES 0x1u   /* leaf scales come from `leaf_scale`, not the descriptor word */
#define MTC_FLAG_MX_LAYOUT 0x2u     /* payload in the matrix-core decode layout (see below); decoded one X
                                       row per block on v_mfma_f32_4x4x4_16b_f16 */
#define MTC_FLAG_COLS_GATHERED 0x4u /* tile stream: columns in the original order, 8-word cells with a bf16
                                       scale pair per column, no col_perm (see mtc_tile_desc) */

/*
 * Panel stream. The (permuted) weight Wp is K x N (reduction x output). It is
 * cut into work units u = panel * n_chunks + chunk: panel = 32 output columns
 * = 8 column groups (cg) of 4 columns, chunk = `chunk_rows` reduction rows
 * (multiple of 32, at most 4096). Within a unit, lane chunks are grouped by cg
 * and bucketed by (leaf size S in {4,8,16,32}, code width P in
 * {2,3,4,5,6,8,16}); a unit's buckets, payload and leaf words are contiguous.
 *
 *  unit_hdr[32*u + 0..1]   : payload dword range [begin, end) of the unit (begin % 4 == 0)
 *  unit_hdr[32*u + 2..3]   : leaf-word range [begin, end)
 *  unit_hdr[32*u + 4..5]   : bucket range [begin, end)
 *  unit_hdr[32*u + 7]      : dwords a decode block stages on chip: max over the unit's column-group
 *                            pairs of (pair payload + 4 per pair bucket) + the unit's leaf words
 *  unit_hdr[32*u + 8..16]  : bucket offset of cg 0..8, relative to the unit's first bucket
 *  unit_hdr[32*u + 17..25] : payload offset of cg 0..8 in dwords, relative to the unit's payload
 *  unit_hdr[32*u + 26]     : as word 7 for blocks of four column groups
 *  unit_hdr[32*u + 27..28] : overflow start (a record index) and record count of decode block 0
 *                            (column groups 0-3)
 *  unit_hdr[32*u + 29..30] : the same for decode block 1 (column groups 4-7)
 *  buckets[4*b + 0] : payload offset of the bucket in dwords, relative to the unit (multiple of 4)
 *  buckets[4*b + 1] : first leaf word of the bucket, relative to the unit
 *  buckets[4*b + 2] : lane chunks in the bucket (bits 0-15) | first chunk within its cg (bits 16-31)
 *  buckets[4*b + 3] : log2(S) | P << 8
 *  leaf_word[l]     : bits 0-9 row offset in the unit / 4, bit 13 pad leaf (ignored),
 *                     bits 16-31 bf16 scale
 *  leaf_scale[l]    : fp32 scale (only with MTC_FLAG_FP32_SCALES)
 *  steps[8*r + ..]  : decode step records. Decode block B = 2*u + b (unit u, block b of 4
 *                     column groups) owns count = unit_hdr[32*u + 28 + 2b] records, ordered by
 *                     bucket kind, then 16-chunk step j. Its record i < F = fixed_steps is
 *                     steps record B*F + i; record i >= F is record overflow_start + i - F.
 *                     Record n_blocks*F (n_blocks = 2 * n_units) and unused fixed places are
 *                     null records (no chunks). Word 2g (g = 0..3, column group 4b + g) names
 *                     the step's first chunk, chunk 16j of the kind's bucket in that column
 *                     group, relative to the unit: bits 0-15 its payload offset in dwords / 4
 *                     (from unit_hdr[32*u + 0]), bits 16-31 its first leaf word (from
 *                     unit_hdr[32*u + 2]; the bucket's first leaf + 32j for S = 4, + 16j >>
 *                     (log2 S - 3) otherwise); 0 when the slot has no chunks. Words 2g + 1
 *                     (all four equal): bits 0-2 log2 S, bits 3-7 P, bits 8+5g .. 12+5g the
 *                     chunks of slot g in this step, min(max(n - 16j, 0), 16) for a bucket
 *                     of n chunks (0 without one).

 * The payload array extends at least 4 dwords past the last bucket (the kernels read
 * chunks with 16-byte loads that may run up to 3 dwords past a chunk's end); leaf_word
 * holds at least one word.
 *
 * A lane chunk is 32 codes in P dwords, stored offset-binary (u = q + 2^(P-1), so
 * the signed code q = u - 2^(P-1)). For P != 3 code i occupies bits [i*P, i*P+P)
 * of the chunk's little-endian bit string. For P = 3 the codes sit in byte lanes:
 * byte b of dwords 0, 1, 2 (dword 0's byte lowest) is a 24-bit string holding
 * codes 8b .. 8b+7, code 8b + a at bits [3a, 3a+3). Every chunk lands in the 4
 * columns of its cg: for S >= 8 it is 4 columns x 8 rows of one leaf, code i
 * at column i/8, row i%8, and chunk t of a bucket is leaf t/(S/8), row block
 * t%(S/8); for S = 4 it is leaves 2t and 2t+1 (16 codes each, column-major; an
 * odd group ends with a pad leaf). A leaf's word is shared by every cg it spans.
 *
 * With MTC_FLAG_MX_LAYOUT the buckets hold whole quads of chunks: a bucket of n chunks has
 * ceil(n / 4) * 4 * P payload dwords (the last quad padded with zero codes; step records and
 * counts name the real chunks). Quad q's 4P dwords are 4 lanes of P dwords; lane j holds
 * column j of the quad's chunks 4q .. 4q+3 as 32 offset-binary codes: for o = 0..15, code o of
 * the "low" string is chunk o/4, chunk row 2(o%4), column j, and code o of the "high" string
 * is the row after it (chunk rows 0-7 are the leaf's 8 rows for S >= 8; for S = 4 rows 0-3 are
 * the chunk's first leaf and 4-7 its second). The low string is the concatenation of the low
 * 16-bit halves of the lane's dwords (dword d holds string bits [16d, 16d+16)), the high string
 * that of the high halves, and code o sits at bits [o*W, o*W+W) of its string, W = P; for
 * P = 16 the low bytes of the codes form such strings with W = 8 in dwords 0-7 and the high
 * bytes in dwords 8-15.
 *
 * Y[:, col_perm[n]] = X[:, row_perm] * Wp[:, n]; NULL perms mean identity.
 * payload and row_perm must be 16-byte aligned.
 */
typedef struct mtc_stream_desc {
  uint32_t abi_version;
  uint32_t flags;
  int32_t K;
  int32_t N;
  int32_t chunk_rows;
  int32_t n_panels;
  int32_t n_chunks;
  int32_t n_buckets;
  int32_t max_unit_words;  /* max over units of unit_hdr[32*u + 7] */
  int32_t max_unit_words4; /* max over units of unit_hdr[32*u + 26] */
  int32_t fixed_steps;     /* step records per decode block at fixed positions: 0, 16, 32 or 48 */
  int32_t reserved;        /* 0 */
  int64_t n_leaves;
  int64_t payload_dwords;
  const uint32_t* payload;
  const uint32_t* buckets;
  const int32_t* unit_hdr;
  const uint32_t* leaf_word;
  const float* leaf_scale;
  const int32_t* row_perm;
  const int32_t* col_perm;
  const uint32_t* steps;   /* n_steps step records of 8 words */
  int64_t n_steps;
} mtc_stream_desc;

int mtc_abi_version(void);
const char* mtc_last_error(void);

/* Host-side validation of a descriptor (pointer presence and geometry only). */
int mtc_check_desc(const mtc_stream_desc* d);

/* W_out (K x N fp32, row-major, ORIGINAL channel order) = W_hat, bit-exact,
 * with +0.0 wherever a P0 leaf lies. */
int mtc_dequant(const mtc_stream_desc* d, float* W_out, void* hip_stream);

/* LDS bytes one decode block needs for M rows of X over a stream with these K and
 * chunk_rows (has_row_perm: the stream has a row permutation); a packer shrinks
 * chunk_rows until this fits the device's per-block LDS. Host arithmetic only (no HIP
 * call, no GPU needed); 0 for non-positive arguments. */
size_t mtc_gemv_lds_bytes(int K, int chunk_rows, int has_row_perm, int M);

/* Bytes of GEMV workspace needed for M rows: split-K partials and counters when the stream has
 * several row chunks, and, for M >= 5 (matrix-core M tiles of 8 or 16 rows), X gathered through
 * the row permutation once per call (M tiles x chunk-padded K x tile rows fp32); 0 for a
 * single-chunk stream at M <= 4. The workspace must be zero-filled once before first use; the
 * kernels leave its counters at zero again after every call. */
size_t mtc_gemv_workspace_bytes(const mtc_stream_desc* d, int M);

/* fp32 path: Y (M x N fp32, leading dim ldy) = X (M x K fp32, leading dim ldx) * W_hat.
 * Any M >= 1; tuned for decode (M <= 16): M <= 4 on the vector units, M >= 5 on the matrix
 * core (v_mfma_f32_4x4x1_16b_f32, fp32 products and sums) after a small X staging launch.
 * Deterministic; the rows of a call at any M >= 5 equal those of any other call at M >= 5
 * bit for bit. */
int mtc_gemv_f32(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                 void* workspace, size_t workspace_bytes, void* hip_stream);

/* mtc_gemv_f32 for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference. It takes no
 * workspace: what mtc_gemv_workspace_bytes counts (split-K partials and counters, staged X) lives in
 * a static per-device array of MTC_NOALLOC_SCRATCH_BYTES that the library holds until the
 * process ends; a call that needs more fails with MTC_E_WORKSPACE before any launch. The
 * call allocates nothing and clears the counters itself (a small fill kernel on hip_stream
 * before the decode kernel). Every call on one GPU shares that GPU's array: calls that
 * overlap in time on one GPU (two streams, or two threads) race. Y equals, bit for bit, what
 * mtc_gemv_f32 writes. */
#define MTC_NOALLOC_SCRATCH_BYTES (8u << 20)
size_t mtc_gemv_noalloc_scratch_bytes(void);
int mtc_gemv_f32_noalloc(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                         void* hip_stream);

/* fp32 path for n (1..MTC_MAX_GROUP) matrices that read the same X, in one launch:
 * Y[i] (M x N_i, leading dim ldy[i]) = X (M x K, leading dim ldx) * W_hat_i.
 * No workspace: at M >= 5 each block gathers its own X rows (no staging launch).
 * Every stream must have a single row chunk (n_chunks == 1), the
 * same K, and the same scale format and row-permutation presence. Each Y[i] equals,
 * bit for bit, what mtc_gemv_f32 writes for matrix i alone. */
#define MTC_MAX_GROUP 4
int mtc_gemv_f32_group(const mtc_stream_desc* const* descs, int n, const float* X, int64_t ldx,
                       float* const* Y, const int64_t* ldy, int M, void* hip_stream);

/* Batched decode: any number of matrices, each with its own X and Y (the same M), in ONE
 * launch per block shape (plus one X staging launch for M >= 5). Replaces a loop of mtc_gemv_f32 calls (the reference's per-layer
 * LinearMTCAdaptive.forward, mtc/nn/layers.py:150-151, once per matrix of a decoder stack)
 * when the inputs are known together. Each Y equals, bit for bit, what mtc_gemv_f32 writes
 * for its matrix alone (same block code and chunking, fixed reduction order).
 *
 * 1. mtc_gemv_batch_plan(items, n, M, NULL, 0, NULL, 0, &plan_bytes, &ws_bytes) reports the
 *    sizes (host only).
 * 2. The caller provides a zero-filled device workspace of ws_bytes (256-byte aligned; split-K
 *    partials and counters of the members with several row chunks, and X staged for M >= 5;
 *    the kernels leave the counters at zero again) and a 64-byte aligned host buffer of plan_bytes, and calls
 *    mtc_gemv_batch_plan again with both: it writes the plan (descriptors, X/Y pointers,
 *    workspace slices, the member of each grid block) into the host buffer.
 * 3. The caller copies the plan byte for byte into a 64-byte aligned device buffer (and keeps
 *    every array, X, Y and the workspace alive and unmoved while the plan is used).
 * 4. mtc_gemv_f32_batch(host_plan, device_plan, stream) launches it (asynchronous; the host
 *    plan is read during the call only). Launches that share a workspace must not overlap.
 * All members must have the same scale format. */
typedef struct mtc_gemv_batch_item {
  const mtc_stream_desc* desc;   /* read while the plan is built */
  const float* X;                /* M x K fp32, leading dim ldx */
  int64_t ldx;
  float* Y;                      /* M x N fp32, leading dim ldy */
  int64_t ldy;
} mtc_gemv_batch_item;

int mtc_gemv_batch_plan(const mtc_gemv_batch_item* items, int n, int M, void* workspace, size_t workspace_bytes,
                        void* plan, size_t plan_bytes, size_t* plan_needed, size_t* workspace_needed);
int mtc_gemv_f32_batch(const void* host_plan, const void* device_plan, void* hip_stream);

/*
 * Tile stream (prefill). Wp (K x N) is cut into steps of 64 reduction rows x
 * 256 output columns; step = col_tile * n_ksteps + kstep. A step holds 512
 * cells of 8 rows x 4 columns (column group c = 0..63 of the tile, row block
 * r = 0..7), each covered by one leaf of size >= 8 or by two 4x4 leaves (top
 * rows 0-3, bottom rows 4-7), so a cell has a (code width, scale) pair per half.
 * A cell is stored in the class of its wider half, as offset-binary codes
 * u = q + 2^(w-1):
 *   class 0 (P <= 4):  4 dwords; column j in dword j, byte k = u[row k] | u[row k+4] << 4
 *   class 1 (P <= 8):  8 dwords; column j in dwords 2j (rows 0-3) and 2j+1 (rows 4-7), byte per row
 *   class 2 (P = 16): 16 dwords; column j in dwords 4j+h: rows 2h (bits 0-15), 2h+1 (bits 16-31)
 *   class 3 (P0):      no payload (zeros)
 * cells[step*512 + i] (2 words, or 4 with MTC_FLAG_FP32_SCALES):
 *   word 0 : payload offset within the step in dwords (bits 0-13) | class << 14 | (c*8 + r) << 16
 *   word 1 : bf16 scale of the top half | bf16 scale of the bottom half << 16
 *            (fp32 scales: word 1 top, word 2 bottom, word 3 unused)
 * Within a step, cells are sorted by class, then position.
 * step_off[step] : payload offset of the step in dwords (n_steps + 1 entries); the
 *   payload array extends at least 8 dwords past step_off[n_steps] (the kernel reads
 *   32 bytes per cell whatever its class).
 * The device stages bf16(q * s) per weight (q * s is exact in fp32).
 */
typedef struct mtc_tile_desc {
  uint32_t abi_version;
  uint32_t flags;          /* MTC_FLAG_FP32_SCALES: 4-word cells with fp32 scales;
                              MTC_FLAG_COLS_GATHERED: 8-word cells (word 0, then per column j a
                              bf16 top scale | bf16 bottom scale << 16, 3 zero words) whose
                              columns are Y's own (a QT-P matrix packed with its columns back in
                              the original order), so col_perm must be NULL */
  int32_t K;
  int32_t N;
  int32_t n_ksteps;        /* ceil(K / 64) */
  int32_t n_col_tiles;     /* ceil(N / 256) */
  int64_t payload_dwords;
  const uint32_t* cells;
  const uint32_t* step_off;
  const uint32_t* payload;
  const int32_t* row_perm;
  const int32_t* col_perm;
} mtc_tile_desc;

int mtc_check_tile_desc(const mtc_tile_desc* d);

/* Bytes of prefill workspace for M rows of X of dtype x_dtype (256-byte aligned
 * workspace; contents need no initialisation): M*K*2 (rounded up to 256) when X may
 * be staged as bf16 first (fp32 X, or a row permutation to gather; fp32 X without a
 * permutation, with 16-byte aligned rows, in the 64- and 128-row tiles of short X is
 * rounded to bf16 by the tile kernel itself and leaves that area unused), plus
 * splits*M*N*4 when the output has too few 256 x 256 tiles to fill the chip and the
 * K steps are split over blocks (fp32 partial tiles, summed in a fixed order).
 * For a call eligible for the decode-once path (below) at least N*64*ceil(K/64)*2
 * (W_hat in bf16) + the staged X (the GEMM itself runs without a workspace). */
size_t mtc_gemm_workspace_bytes(const mtc_tile_desc* d, int M, int x_dtype);

/* bf16 MFMA path (prefill): Y (M x N, fp32 or bf16, leading dim ldy) =
 * X (M x K, fp32 or bf16, leading dim ldx) * W_hat with bf16 operands and
 * fp32 accumulation. bf16 X read in place must have 16-byte aligned rows
 * (ldx % 8 == 0). Any M >= 1.
 * Decode-once path: a call with M >= max(512, K / 8), M * K * N >= 2^28 and no col_perm
 * decodes W_hat once
 * into bf16 in the workspace (the values the tile kernel would multiply) and runs
 * hipBLASLt's bf16 GEMM with fp32 accumulation on it, instead of the tile kernel, which
 * decodes each weight step once per 256-row tile. The same shape always runs the same GEMM
 * algorithm, so results are deterministic. Without hipBLASLt, or with no algorithm for the
 * shape, the call runs the tile kernel; so does a call made while its stream is captured into a
 * graph before any call outside a capture has set the library up on the device (that allocates),
 * whose graph then holds the tile kernel. */
int mtc_gemm_bf16(const mtc_tile_desc* d, const void* X, int x_dtype, int64_t ldx, void* Y, int y_dtype,
                  int64_t ldy, int M, void* workspace, size_t workspace_bytes, void* hip_stream);

/* Switches the decode-once paths of mtc_gemm_bf16 / mtc_gemm_bf16_group / mtc_gemm_f32 on (1, the default)
 * or off (0: every call runs the tile kernel) for the process; -1 only queries. Returns the
 * previous setting. No counterpart in the reference: for callers and tests that measure or
 * check the fused tile kernel at shapes the decode-once path would take. A prefill batch
 * plan keeps the choice made when it was built. Not synchronised with calls in flight on
 * other threads. */
int mtc_set_prefill_decode_once(int enable);

/* fp32 matrix-core path over the tile stream: Y (M x N fp32, leading dim ldy) = X (M x K
 * fp32, leading dim ldx) * W_hat with the exact fp32 W_hat and fp32 products and sums
 * (v_mfma_f32_16x16x4f32), in 16-row tiles with K split over blocks until the chip is full;
 * within the fp32 tolerance of the reference's float32 block loop (mtc/kernels/gemm.py:124-210,
 * the same operation as mtc_gemv_f32, for callers at 5..16 rows and beyond). X read in place
 * must have 16-byte aligned rows (ldx % 4 == 0); a stream with a row permutation gathers X
 * into the workspace first. Workspace (mtc_gemm_f32_workspace_bytes, 256-byte aligned, no
 * initialisation): the gathered X (M*K*4) and the split-K partials.
 * Decode-once path: a call with M >= 256, M * K * N >= 2^32 and no col_perm decodes the exact
 * W_hat once into fp32 in the workspace (N*64*ceil(K/64)*4 bytes, then the gathered X) and runs
 * hipBLASLt's fp32 GEMM on it (fp32 products and sums); deterministic, one algorithm per shape;
 * without hipBLASLt, or with the path switched off (mtc_set_prefill_decode_once), the tile
 * kernel runs. */
size_t mtc_gemm_f32_workspace_bytes(const mtc_tile_desc* d, int M);
int mtc_gemm_f32(const mtc_tile_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                 void* workspace, size_t workspace_bytes, void* hip_stream);

/* Prefill for n (1..MTC_MAX_GROUP) matrices that read the same X, one launch per kernel
 * (X staging, tile GEMM, split-K reduction) instead of one per matrix:
 * Y[i] (M x N_i, leading dim ldy[i]) = X * W_hat_i. Every tile stream must have the same
 * K and scale format. The workspace (mtc_gemm_group_workspace_bytes, 256-byte aligned, no
 * initialisation) holds, per member, its staged X and its split-K partials, then one area
 * for the members a single call would run on the decode-once path, which run on it here too,
 * one after another. Each Y[i] equals, bit for bit, what mtc_gemm_bf16 writes for matrix i
 * alone. */
size_t mtc_gemm_group_workspace_bytes(const mtc_tile_desc* const* descs, int n, int M, int x_dtype);
int mtc_gemm_bf16_group(const mtc_tile_desc* const* descs, int n, const void* X, int x_dtype, int64_t ldx,
                        void* const* Y, int y_dtype, const int64_t* ldy, int M, void* workspace,
                        size_t workspace_bytes, void* hip_stream);

/* Batched prefill: any number of matrices, each with its own X and Y (the same M, X dtype and
 * Y dtype, and one scale format), in one X-staging launch, one tile launch and, if any
 * member's K is split, one reduction launch. Replaces a loop of mtc_gemm_bf16 calls (the
 * reference's per-layer LinearMTCAdaptive.forward, mtc/nn/layers.py:150-151, at prefill
 * shapes) when the inputs are known together. The protocol is that of the decode batch:
 * query sizes with plan == NULL, give a 256-byte aligned device workspace (staged bf16 X and
 * split-K partials; no initialisation) and a 64-byte aligned host buffer, copy the plan byte
 * for byte to a 64-byte aligned device buffer, launch with mtc_gemm_bf16_batch. When the
 * members' output tiles together fill the chip no K is split; otherwise each member splits K
 * as mtc_gemm_bf16 would, and its Y then equals that call's bit for bit. Results are
 * deterministic. In a batch that does not fill the chip, members that mtc_gemm_bf16 alone
 * would run on the decode-once path run on it here too, one after another after the tile
 * launches (in one more workspace area), so their Y also equals the single call's; a batch
 * that fills the chip runs every member on the tile kernel. Launches that share a workspace
 * must not overlap. */
typedef struct mtc_gemm_batch_item {
  const mtc_tile_desc* desc;     /* read while the plan is built */
  const void* X;                 /* M x K, x_dtype, leading dim ldx */
  int64_t ldx;
  void* Y;                       /* M x N, y_dtype, leading dim ldy */
  int64_t ldy;
} mtc_gemm_batch_item;

int mtc_gemm_batch_plan(const mtc_gemm_batch_item* items, int n, int M, int x_dtype, int y_dtype, void* workspace,
                        size_t workspace_bytes, void* plan, size_t plan_bytes, size_t* plan_needed,
                        size_t* workspace_needed);
int mtc_gemm_bf16_batch(const void* host_plan, const void* device_plan, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* MTC_HIP_H */
