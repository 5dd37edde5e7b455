// gfx950 decode kernels and C-ABI for Y = X * W_hat over the panel stream,
// plus the host error state shared with mtc_gemm.hip.
//
//   k_fill_zero  : zero an fp32 buffer (used before dequant; no memset nodes)
//   k_dequant    : stream -> dense W_hat (bit-exact q*s, +0.0 for P0)
//   k_gemv<MT,FS,LG,NW>: fp32 decode path for M tiles of MT rows (FS: fp32 leaf
//                  scales, LG: X rows gathered in LDS, NW waves). One block per
//                  (unit, 4 column groups); waves walk the block's step records,
//                  streaming payload into registers, and accumulate 4 columns per
//                  lane; one reduction at the end.
//   k_gemv_group : the same blocks for up to 4 matrices that share X, one launch
//   (the prefill path, k_gemm_tile over the tile stream, is in mtc_gemm.hip)
//
// Reference behaviour: mtc/kernels/gemm.py:124-210 (block loop: skip P0
// blocks, unpack codes, scale, fp32 multiply-accumulate) for a dense X and a
// quadtree weight; W_hat as defined by mtc/core/quadtree.py:157-171.

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "mtc_hip.h"
#include "mtc_decode.h"
#include "mtc_host.h"

using namespace mtc;
using mtc::host::check_launch;
using mtc::host::fail;
using mtc::host::ok;


#define MTC_API extern "C" __attribute__((visibility("default")))

namespace {

// Bucket entry fields.
struct Bucket {
  uint32_t pay;      // payload offset, dwords, unit-relative
  uint32_t leaf;     // first leaf word, unit-relative
  uint32_t n;        // lane chunks
  uint32_t cstart;   // first chunk within the column group
  uint32_t key;
};

__device__ __forceinline__ Bucket read_bucket(const uint32_t* e) {
  Bucket b;
  b.pay = e[0];
  b.leaf = e[1];
  b.n = e[2] & 0xFFFFu;
  b.cstart = e[2] >> 16;
  b.key = e[3];
  return b;
}

// ---------------------------------------------------------------------------
// zero fill
// ---------------------------------------------------------------------------
__global__ void k_fill_zero(float* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// dequant: one block (8 waves) per unit, wave g decodes column group g
// ---------------------------------------------------------------------------
template <int S, int P, int T>
__device__ __forceinline__ void mx_codes_t(const uint32_t* q, float (&out)[32]);
template <int S, int P>
__device__ __forceinline__ void mx_codes(const uint32_t* q, uint32_t t, float (&out)[32]);

// Chunk t of a bucket into W_hat; src: the chunk's dwords (v1 layout) or its quad's (mx).
template <int S, int P>
__device__ __forceinline__ void dequant_chunk(const mtc_stream_desc& d, const uint32_t* src, bool mx,
                                              const uint32_t* lw, uint32_t lg0, uint32_t t, int kb, int col0,
                                              float* __restrict__ W) {
  float q[32];
  if (mx) {
    mx_codes<S, P>(src, t & 3u, q);
  } else {
    uint32_t w[P];
    load_chunk<P, true>(src, w);
    decode_chunk<P>(w, q);
  }
  constexpr int R = (S == 4) ? 4 : 8;
#pragma unroll
  for (int h = 0; h < (S == 4 ? 2 : 1); ++h) {
    uint32_t leaf;
    int rrel;
    if constexpr (S == 4) {
      leaf = 2 * t + h;
      rrel = 0;
    } else {
      leaf = t / (S / 8);
      rrel = 8 * (int)(t % (S / 8));
    }
    const LeafInfo li = leaf_info(lw[leaf], d.leaf_scale, lg0 + leaf);
    if (li.pad) continue;
#pragma unroll
    for (int c = 0; c < kGroup; ++c) {
      int col = col0 + c;
      if (d.col_perm) col = d.col_perm[col];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        int k = kb + li.row + rrel + r;
        if (d.row_perm) k = d.row_perm[k];
        float v = q[16 * h + R * c + r] * li.scale;
        // quadtree W_hat is summed into a +0.0 buffer (no -0.0); the uniform-block
        // arena rebuild assigns q*s as is
        if (!d.leaf_scale) v += 0.0f;
        W[(int64_t)k * d.N + col] = v;
      }
    }
  }
}

__global__ __launch_bounds__(512) void k_dequant(const mtc_stream_desc d, float* __restrict__ W) {
  const int u = blockIdx.x;
  const int g = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int panel = u / d.n_chunks, chunk = u - panel * d.n_chunks;
  const int kb = chunk * d.chunk_rows;
  const int32_t* hdr = d.unit_hdr + kUnitHdr * u;
  const uint32_t* bk = d.buckets + 4 * (hdr[4] + hdr[8 + g]);
  const int nb = hdr[9 + g] - hdr[8 + g];
  const uint32_t* pay = d.payload + hdr[0];
  const int col0 = panel * kPanel + g * kGroup;
  const bool mx = (d.flags & MTC_FLAG_MX_LAYOUT) != 0;
  for (int b = 0; b < nb; ++b) {
    const Bucket e = read_bucket(bk + 4 * b);
    const uint32_t* lw = d.leaf_word + hdr[2] + e.leaf;
    const uint32_t lg0 = hdr[2] + e.leaf;
    for (uint32_t t = lane; t < e.n; t += 64) {
      switch (e.key) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): \
    dequant_chunk<S, P>(d, mx ? pay + e.pay + (t / 4) * 4 * P : pay + e.pay + t * P, mx, lw, lg0, t, kb, col0, W); \
    break;
        MTC_FOR_EACH_BUCKET(MTC_CASE)
#undef MTC_CASE
        default: break;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 decode GEMV
//
// Block = (unit, block of 4 column groups), W waves (16, or 8 for 4-row M tiles and for
// streams whose blocks hold at most 16 records). The block's work is its list of
// step records; wave w executes records w, w + W, w + 2W, ... (round robin, so the
// waves of each SIMD get near-equal counts). In a step, lane 16g + i decodes chunk
// 16j + i of column-group slot g's bucket of the step's kind: one kind per step, so
// the decode is a scalar (readfirstlane) switch into fully unrolled code. Each lane
// streams its chunk's payload dwords and leaf word(s) straight from memory into
// registers, the first three steps' loads before anything else, and accumulates its
// column group's 4 columns (times MT rows) in registers. X (gathered through
// row_perm) and its 4- and 8-row sums are staged in LDS. Lanes and waves are
// combined once at the end (no atomics unless K is split over units). Blocks of one
// unit are mapped to the same XCD so the unit's leaf words stay in one L2.
// ---------------------------------------------------------------------------
constexpr int kMaxP = 16;
typedef uint32_t u32x16_t __attribute__((ext_vector_type(16)));   // a step's payload words (one SSA value)

typedef const __attribute__((address_space(4))) int32_t* ci32p;

// Loads of one step into a lane's registers: its chunk's payload dwords (w[0..P)), its
// leaf word(s) and, for fp32-scale streams, the leaf scale(s). Every step issues the same
// kStepLoads vector loads into the same registers whatever its kind: four 16-byte payload
// loads at offsets 0, 4, 8, 12 dwords, where the loads a P-dword chunk does not need read
// one wave-uniform stand-in address instead (the words they fill are read only by wider
// kinds). The compiler's waits before decoding a step then stay partial.
// Chunks are dword aligned; a 16-byte load past a chunk reads the next chunk or the
// stream's tail padding. Lanes past the bucket's end re-read its last chunk and are
// masked when accumulating.
constexpr int kStepLoads = 8;
typedef uint32_t u32x4u_t __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ u32x4_t ldu4(const uint32_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4u_t*>(p));
}

typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));

// Workgroup barrier that orders LDS only: waits for this wave's LDS accesses, not for its
// global loads, which may stay in flight across it (__syncthreads() waits for both).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Buffer resources: a wave-uniform base and byte size in scalar registers, so every load
// is one instruction with a 32-bit per-lane byte offset, and an offset past the end
// reads zeros instead of faulting.
constexpr int kBufferFormat = 0x00020000;            // dword 3 of a raw gfx9 buffer resource
constexpr int kNT = 2;                               // load cache policy: nontemporal
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)min(bytes, (int64_t)0x7FFFFFFF), kBufferFormat);
}

// A step's loads into a lane's registers. Every kind issues the same number of load
// instructions (2 payload, 2 leaf-word and, with fp32 scales, 2 scale loads), so the
// compiler's in-order wait counts stay exact across steps of different kinds; each load
// reads only what the kind needs (the vector memory pipeline's cost grows with lanes x
// bytes even when lanes share an address), and a load a kind does not need reads past
// the buffer's end, which returns zeros without a memory access. Payload dwords 8-15 of
// a P = 16 chunk are loaded when the chunk is decoded (gemv_load_p16_tail).
constexpr uint32_t kOutOfRange = 0xFFFFFF00u;        // byte offset past any buffer's end
constexpr int64_t kMaxArrayBytes = 0x7FFFFFFF;       // largest stream array a buffer resource covers

// The payload part of a step's loads: P dwords at dword pay + t * P (two load instructions for
// every width; the tail of a P = 16 chunk comes from gemv_load_p16_tail).
__device__ __forceinline__ void gemv_load_payload(__amdgpu_buffer_rsrc_t pay_r, uint32_t P, uint32_t pay, uint32_t t,
                                                  u32x16_t& w, uint32_t& ob) {
  ob = (pay + t * P) << 2;                           // payload byte offset of the chunk
  if (P <= 4) {
    if (P == 2) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(pay_r, ob, 0, kNT);
      w[0] = v.x; w[1] = v.y;
    } else if (P == 3) {
      const u32x3_t v = __builtin_amdgcn_raw_buffer_load_b96(pay_r, ob, 0, kNT);
      w[0] = v.x; w[1] = v.y; w[2] = v.z;
    } else {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(pay_r, ob, 0, kNT);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
    w[15] = __builtin_amdgcn_raw_buffer_load_b32(pay_r, kOutOfRange, 0, 0);   // count keeper
  } else {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(pay_r, ob, 0, kNT);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    if (P == 5) {
      w[4] = __builtin_amdgcn_raw_buffer_load_b32(pay_r, ob + 16, 0, kNT);
    } else if (P == 6) {
      const u32x2_t e = __builtin_amdgcn_raw_buffer_load_b64(pay_r, ob + 16, 0, kNT);
      w[4] = e.x; w[5] = e.y;
    } else {
      const u32x4_t e = __builtin_amdgcn_raw_buffer_load_b128(pay_r, ob + 16, 0, kNT);
      w[4] = e.x; w[5] = e.y; w[6] = e.z; w[7] = e.w;
    }
  }
}

template <bool FS>
__device__ __forceinline__ void gemv_load(__amdgpu_buffer_rsrc_t pay_r, __amdgpu_buffer_rsrc_t lw_r,
                                          __amdgpu_buffer_rsrc_t fs_r, uint32_t key, uint32_t pay, uint32_t leaf,
                                          uint32_t t, u32x16_t& w, uint32_t& ob, uint32_t& lw0, uint32_t& lw1,
                                          float& fs0, float& fs1) {
  const uint32_t P = key >> 8, ls = key & 0xFFu;
  gemv_load_payload(pay_r, P, pay, t, w, ob);
  const uint32_t l0 = leaf + (ls == 2 ? 2 * t : t >> (ls - 3));
  const uint32_t b1 = ls == 2 ? (l0 + 1) << 2 : kOutOfRange;   // second 4x4 leaf, if any
  lw0 = __builtin_amdgcn_raw_buffer_load_b32(lw_r, l0 << 2, 0, 0);
  lw1 = __builtin_amdgcn_raw_buffer_load_b32(lw_r, b1, 0, 0);
  if constexpr (FS) {
    fs0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(fs_r, l0 << 2, 0, 0));
    fs1 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(fs_r, b1, 0, 0));
  } else {
    fs0 = fs1 = 0.0f;
  }
}

__device__ __forceinline__ u32x16_t gemv_load_p16_tail(__amdgpu_buffer_rsrc_t pay_r, u32x16_t w, uint32_t ob) {
  const u32x4_t f = __builtin_amdgcn_raw_buffer_load_b128(pay_r, ob + 32, 0, kNT);
  const u32x4_t h = __builtin_amdgcn_raw_buffer_load_b128(pay_r, ob + 48, 0, kNT);
  w[8] = f.x; w[9] = f.y; w[10] = f.z; w[11] = f.w;
  w[12] = h.x; w[13] = h.y; w[14] = h.z; w[15] = h.w;
  return w;
}

// X rows of a unit as staged in LDS: xs[m][r] = X[m0 + m, row_perm[kb + r]], plus the
// sums of each 4-row and 8-row block (xs4[m][r / 4], xs8[m][r / 8]) that turn a chunk's
// offset-binary dot product into the signed one: sum_r x_r q_r = sum_r x_r u_r - 2^(P-1) sum_r x_r.
// Blocks of 4 M rows keep no 4-row sums (they add them from the x values instead), so
// that two blocks of a 4096-row unit fit one CU's LDS.
__host__ __device__ constexpr bool gemv_sum4(int MT) { return MT <= 2; }

// Whole X rows are staged and gathered in LDS when there is a row permutation, the M tile
// has 1-2 rows and K <= 4096 (at most 32 KB per block).
__host__ __device__ constexpr int gemv_lds_gather_rows(int MT) { return MT <= 2 ? MT : 1; }
__host__ __device__ constexpr bool gemv_lds_gather(int MT, bool perm, int K) {
  return perm && MT <= 2 && K <= kMaxChunkRows;
}

struct XStage {
  const float* xs;
  const float* xs4;
  const float* xs8;
  int kc;
};

// One lane chunk (payload in registers) into the lane's 4-column accumulators:
// acc[m][c] += s * (sum_r x[m][r] * u[r][c] - off * sum_r x[m][r]) per leaf.
// S = 4: two 4x4 leaves. S = 8 stands for every leaf size of 8 or more: chunk t is row
// block t & rb_mask of its leaf (rb_mask = S / 8 - 1, wave-uniform), so the three sizes
// share one code path.
template <int S, int P, int MT>
__device__ __forceinline__ void gemv_chunk(const u32x16_t rw, uint32_t lw0, uint32_t lw1, float fs0, float fs1,
                                           bool fp32_scales, uint32_t t, uint32_t rb_mask, const XStage& xt,
                                           float (&acc)[MT][kGroup]) {
  static_assert(S == 4 || S == 8, "leaf sizes 16 and 32 take the S = 8 path");
  constexpr float off = (float)(1 << (P - 1));
  uint32_t w[P];
#pragma unroll
  for (int i = 0; i < P; ++i) w[i] = rw[i];
  float u[32];
  decode_chunk_u<P>(w, u);
  if constexpr (S == 4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const LeafInfo li = leaf_info_v(h ? lw1 : lw0, fp32_scales, h ? fs1 : fs0);
      if (li.pad) continue;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 x = *reinterpret_cast<const float4*>(xt.xs + m * xt.kc + li.row);
        float x4;
        if constexpr (gemv_sum4(MT)) {
          x4 = xt.xs4[m * (xt.kc / 4) + (li.row >> 2)];
        } else {
          x4 = (x.x + x.y) + (x.z + x.w);
        }
        const float init = -off * x4;
#pragma unroll
        for (int c = 0; c < kGroup; ++c) {
          const float* q = u + 16 * h + 4 * c;
          float dsum = __builtin_fmaf(x.x, q[0], init);
          dsum = __builtin_fmaf(x.y, q[1], dsum);
          dsum = __builtin_fmaf(x.z, q[2], dsum);
          dsum = __builtin_fmaf(x.w, q[3], dsum);
          acc[m][c] = __builtin_fmaf(li.scale, dsum, acc[m][c]);
        }
      }
    }
  } else {
    const LeafInfo li = leaf_info_v(lw0, fp32_scales, fs0);
    const int row = li.row + 8 * (int)(t & rb_mask);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float4 x0 = *reinterpret_cast<const float4*>(xt.xs + m * xt.kc + row);
      const float4 x1 = *reinterpret_cast<const float4*>(xt.xs + m * xt.kc + row + 4);
      const float init = -off * xt.xs8[m * (xt.kc / 8) + (row >> 3)];
#pragma unroll
      for (int c = 0; c < kGroup; ++c) {
        const float* q = u + 8 * c;
        float dsum = __builtin_fmaf(x0.x, q[0], init);
        dsum = __builtin_fmaf(x0.y, q[1], dsum);
        dsum = __builtin_fmaf(x0.z, q[2], dsum);
        dsum = __builtin_fmaf(x0.w, q[3], dsum);
        dsum = __builtin_fmaf(x1.x, q[4], dsum);
        dsum = __builtin_fmaf(x1.y, q[5], dsum);
        dsum = __builtin_fmaf(x1.z, q[6], dsum);
        dsum = __builtin_fmaf(x1.w, q[7], dsum);
        acc[m][c] = __builtin_fmaf(li.scale, dsum, acc[m][c]);
      }
    }
  }
}

constexpr int kStepGroups = 4;              // column groups one decode step covers
constexpr int kStepLanes = 16;              // lanes per column group in a step
constexpr int kStepWords = 8;               // words per step record: (slot word, kind and counts) x 4

// Slot g's word of record r and the record's kind-and-counts word (words 2g, 2g + 1).
__device__ __forceinline__ u32x2_t record_slot(__amdgpu_buffer_rsrc_t rec_r, uint32_t r, int g) {
  return __builtin_amdgcn_raw_buffer_load_b64(rec_r, r * (kStepWords * 4) + 8 * g, 0, 0);
}
// Bucket key (log2 S | P << 8) of a record's kind field (log2 S | P << 3); wave-uniform.
__device__ __forceinline__ uint32_t record_key(uint32_t kc) {
  const uint32_t k = __builtin_amdgcn_readfirstlane(kc);
  return (k & 7u) | (((k >> 3) & 31u) << 8);
}
// Chunks of slot g in the record's step (0-16).
__device__ __forceinline__ uint32_t record_count(uint32_t kc, int g) { return (kc >> (8 + 5 * g)) & 31u; }
// Most waves a decode block has (the LDS of the cross-wave reduction is sized for it).
__host__ __device__ constexpr int gemv_waves(int MT) { return MT == 4 ? 8 : 16; }
constexpr int kFewSteps = 16;
constexpr int kSmallRows = 1024;
constexpr int kGemvBlocksPerUnit = kGroups / kStepGroups;

// Block shape of a matrix's decode blocks. The single, grouped and batched launches all take it
// from gemv_shape, so a matrix's blocks run the same code (same waves, hence the same
// summation order) in every launch:
// - M tiles of 4 rows: 8 waves, three steps prefetched;
// - 1-2 rows, units of at most kSmallRows rows: 4 waves with two steps prefetched, which
//   keeps a wave near 69 registers so that seven blocks share a CU; the X staging is sized
//   for kSmallRows rows (with the LDS gather when K fits it too);
// - 1-2 rows, larger units with more than kFewSteps records per block: 16 waves (one block
//   fills a CU), three steps prefetched, X rows gathered in LDS when there is a row
//   permutation and K <= 4096;
// - 1-2 rows, larger units with at most kFewSteps records per block: 4 waves, X staging
//   for kMaxChunkRows rows without the LDS gather.
struct GemvShape {
  int nw;        // waves per block
  int kc;        // rows the X staging covers (kSmallRows or kMaxChunkRows)
  bool lg_code;  // the kernel has the LDS-gather code
  bool lg;       // this matrix gathers X in LDS
  bool mx;       // the stream has the mx payload layout (one X row per block, matrix core)
};
inline bool is_mx(const mtc_stream_desc* d) { return (d->flags & MTC_FLAG_MX_LAYOUT) != 0; }
inline GemvShape gemv_shape(int MT, const mtc_stream_desc* d) {
  const bool perm = d->row_perm != nullptr, mx = is_mx(d);
  if (MT > 4) return {16, kMaxChunkRows, false, false, false};   // matrix core
  if (MT > 2) return {8, kMaxChunkRows, false, false, false};
  if (d->chunk_rows <= kSmallRows) return {4, kSmallRows, true, perm && d->K <= kSmallRows, mx};
  if (d->fixed_steps > kFewSteps) return {16, kMaxChunkRows, true, perm && d->K <= kMaxChunkRows, mx};
  return {4, kMaxChunkRows, false, false, mx};
}
// Column halves of its unit per vector-path block. A batched launch of one-row M tiles over small
// units (4 waves, kSmallRows) gives a block both halves of its unit, two waves per half, so that
// the unit's X rows are staged once and the blocks' fixed costs are spread over twice the
// records (the batch's blocks fill the chip anyway); every other launch, and a single or grouped
// call of any shape, runs a block per half, whose four waves keep each wave's chain of records
// short. A two-half block's waves each run two accumulator sets that stand for the four waves of
// a one-half block (records wh, wh + 4, ... and wh + 2, wh + 6, ...), so both give the same Y bit
// for bit.
__host__ __device__ constexpr int gemv_batch_halves(int MT, int NW, int KC, bool MX) {
  return MT == 1 && NW == 4 && KC == kSmallRows && !MX ? 2 : 1;
}
__host__ __device__ constexpr int gemv_prefetch(int NW) { return NW == 4 ? 2 : 3; }
constexpr int kMaxFixedSteps = 48;          // step records per block at block-computable positions
constexpr int kXcds = 8;

// Sum over the 16 lanes of a column-group slot (one DPP row): row shifts by 1, 2, 4 and 8
// build an inclusive prefix sum, so the row's last lane ends with the total.
constexpr int kSlotSumLane = kStepLanes - 1;
template <int kRowShr>
__device__ __forceinline__ float row_shr(float v) {   // DPP row_shr; lanes shifted in read 0
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x110 + kRowShr, 0xF,
                                                                0xF, true));
}
__device__ __forceinline__ float slot_sum(float v) {
  v += row_shr<1>(v);
  v += row_shr<2>(v);
  v += row_shr<4>(v);
  v += row_shr<8>(v);
  return v;
}


// The block's outputs from the cross-wave reduction buffer red[partial][slot][m][c] (all
// partials in place, after a barrier; W threads' waves store them). The block covers H column
// halves of its unit's panel (16 columns each, from half cb), WH partials per half, summed in
// order: Y directly for a single-chunk stream; otherwise the block's partial, and the last
// block of each (M tile, panel) sums the unit partials into Y.
template <int MT, int W, int H, int WH = W / H>
__device__ __forceinline__ void gemv_store(const mtc_stream_desc& d, const float* red, const int u, const int cb,
                                           float* __restrict__ Y, int64_t ldy, int M, float* __restrict__ part,
                                           uint32_t* __restrict__ counters) {
  constexpr int T = 64 * W, CH = kStepGroups * kGroup;   // threads; partials (WH) and columns per half
  constexpr int blocks_per_chunk = kGemvBlocksPerUnit / H;
  const int tid = threadIdx.x;
  const int mt = blockIdx.y, m0 = mt * MT;
  const int n_units = d.n_panels * d.n_chunks;
  const int panel = u / d.n_chunks;
  constexpr int nout = MT * H * CH;
  auto sum_of = [&](int i, int& m, int& pc) __attribute__((always_inline)) {
    m = i / (H * CH);
    const int rest = i - m * (H * CH);
    const int hh = rest / CH, gc = rest - hh * CH;
    const int g2 = gc / kGroup, c = gc - g2 * kGroup;
    pc = (cb + hh) * CH + gc;                          // column within the panel
    float v = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < WH; ++w2) v += red[(((hh * WH + w2) * kStepGroups + g2) * MT + m) * kGroup + c];
    return v;
  };

  if (d.n_chunks == 1) {
    for (int i = tid; i < nout; i += T) {
      int m, pc;
      const float v = sum_of(i, m, pc);
      if (m0 + m < M) {
        int col = panel * kPanel + pc;
        if (d.col_perm) col = d.col_perm[col];
        Y[(int64_t)(m0 + m) * ldy + col] = v;
      }
    }
    return;
  }

  // split-K over chunks: deterministic last-block reduction per (M tile, panel).
  // Partials and the counter use relaxed device-scope atomics, which the hardware performs
  // past the XCD-private L2s; ordering comes from waiting for the partial stores to complete
  // before the counter add. (Acquire/release fences at device scope would write back and
  // invalidate the whole L2 of the XCD instead, costing tens of microseconds per call.)
  constexpr int n_part = MT * kPanel;
  float* mine = part + ((size_t)mt * n_units + u) * n_part;
  for (int i = tid; i < nout; i += T) {
    int m, pc;
    const float v = sum_of(i, m, pc);
    __hip_atomic_store(mine + m * kPanel + pc, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are complete
  __syncthreads();
  __shared__ int last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[mt * d.n_panels + panel], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last = (prev == (uint32_t)(d.n_chunks * blocks_per_chunk - 1));
  }
  __syncthreads();
  if (!last) return;
  const float* pp = part + ((size_t)mt * n_units + (size_t)panel * d.n_chunks) * n_part;
  for (int i = tid; i < n_part; i += T) {
    float v = 0.0f;
    for (int c = 0; c < d.n_chunks; ++c)
      v += __hip_atomic_load(pp + (size_t)c * n_part + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int m = i / kPanel, cc = i - m * kPanel;
    if (m0 + m < M) {
      int col = panel * kPanel + cc;
      if (d.col_perm) col = d.col_perm[col];
      Y[(int64_t)(m0 + m) * ldy + col] = v;
    }
  }
  if (tid == 0)
    __hip_atomic_store(&counters[mt * d.n_panels + panel], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One decode block of matrix `d`: block id `bid` along the grid's x (the y index is the M tile),
// NW waves. LG: the code for X rows gathered in LDS is present; lg: this matrix uses it
// (gemv_lds_gather on the host; a constant true for kernels instantiated per matrix).
// KC: rows the X staging covers (chunk_rows <= KC, and K <= KC when X is gathered in LDS).
// PF (gemv_prefetch): steps whose loads a wave issues before the X staging; a wave executes
// its records in the same order whatever PF is.
template <int MT, bool FS, bool LG, int NW, int KC, int H>
__device__ __forceinline__ void gemv_block(const mtc_stream_desc& d, const int bid, const float* __restrict__ X,
                                           int64_t ldx, float* __restrict__ Y, int64_t ldy, int M,
                                           float* __restrict__ part, uint32_t* __restrict__ counters,
                                           const bool lg = true) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  static_assert(H == 1 || (H == 2 && NW == 4), "two-half blocks have four waves");
  constexpr int W = NW, T = 64 * W, BPU = kGemvBlocksPerUnit;
  constexpr int WH = W / H, BPB = BPU / H;           // real waves per half, blocks per unit
  const int kc = d.chunk_rows;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: keeps per-wave control scalar
  const int wh = wave % WH;                           // the wave's place among its half's waves
  const int n_units = d.n_panels * d.n_chunks;
  // block -> (unit, block of 4 column groups) with both blocks of a unit on one XCD; in a block
  // of both halves, wave w takes half w / WH
  const int xcd = bid % kXcds, slot = bid / kXcds;
  const int u = (slot / BPB) * kXcds + xcd;
  if (u >= n_units) return;                           // padding block of the XCD mapping
  const int cb = H == 2 ? wave / WH : slot % BPU;
  const int mt = blockIdx.y;
  const int panel = u / d.n_chunks, chunk = u - panel * d.n_chunks;
  const int m0 = mt * MT;
  const int kb = chunk * kc;
  const int rows = min(kc, d.K - kb);

  float* xs = smem;                                   // [MT][kc]
  float* xs4 = xs + MT * kc;                          // [MT][kc / 4] (MT <= 2 only)
  float* xs8 = xs4 + (gemv_sum4(MT) ? MT * (kc / 4) : 0);   // [MT][kc / 8]
  float* red = xs8 + MT * (kc / 8);                   // [H x W partials][4 slots][MT][4] (H W <= gemv_waves)
  float* xraw = red + H * W * kStepGroups * MT * kGroup;   // [MT][K] whole X rows (LDS gather only)

  const ci32p hdr = (ci32p)(d.unit_hdr + kUnitHdr * u);

  // ---- X first: its loads depend on nothing, so their latency overlaps the record ->
  //      payload chain below. With a row permutation and X rows that fit on chip (M tiles
  //      of 1-2 rows, K <= 4096), the rows are read whole and gathered in LDS, so X is one
  //      load level away and the decode can start before the last payload arrives;
  //      otherwise the permuted row indices are read here and X is gathered from memory
  //      after the payload loads are out. ----
  static_assert(KC % T == 0, "the X staging loops cover KC rows");
  constexpr int XG = (KC + 4 * T - 1) / (4 * T);     // 4-row groups per thread (kc <= KC)
  constexpr int XR = KC / T;                         // whole-row X values per thread and M row (K <= KC)
  constexpr int PF = gemv_prefetch(NW);
  const bool perm = d.row_perm != nullptr;
  const bool lds_gather = LG && lg;                  // host: gemv_lds_gather(MT, perm, K)
  int4 kk[XG];
#pragma unroll
  for (int i = 0; i < XG; ++i) {
    const int r = 4 * (i * T + tid);                  // first of 4 rows, unit-relative
    if (perm && r < rows) {
      kk[i] = *reinterpret_cast<const int4*>(d.row_perm + kb + r);   // kb, r multiples of 4
    } else {
      kk[i] = make_int4(kb + r, kb + r + 1, kb + r + 2, kb + r + 3);
    }
  }
  float xr[gemv_lds_gather_rows(MT)][XR];
  if (lds_gather) {
#pragma unroll
    for (int m = 0; m < gemv_lds_gather_rows(MT); ++m) {
      const float* xrow = X + (int64_t)min(m0 + m, M - 1) * ldx;
#pragma unroll
      for (int i = 0; i < XR; ++i) {
        const int k = i * T + tid;
        xr[m][i] = (k < d.K && m0 + m < M) ? xrow[k] : 0.0f;
      }
    }
  }

  // ---- this wave's step records: records wh, wh + WH, wh + 2WH, ... of its half's list.
  //      A block's first F records sit at block-computable places, so the first three steps'
  //      records are read while the unit header (whose payload and leaf-word starts the
  //      records' offsets are relative to) is still in flight. ----
  const int F = d.fixed_steps;
  const int blk = u * BPU + cb;
  const uint32_t null_rec = (uint32_t)(d.n_panels * d.n_chunks * BPU) * (uint32_t)F;
  const int g = lane / kStepLanes, li = lane % kStepLanes;   // column-group slot, lane in slot

  // A lane's view of a record: its slot's word (where the step starts in the column group's
  // bucket, relative to the unit) and the record's kind-and-counts word; the 16 lanes of a
  // slot read the same words.
  const __amdgpu_buffer_rsrc_t rec_r = buffer_of(d.steps, d.n_steps * kStepWords * 4);
  const __amdgpu_buffer_rsrc_t pay_r = buffer_of(d.payload, d.payload_dwords * 4);
  const __amdgpu_buffer_rsrc_t lw_r = buffer_of(d.leaf_word, d.n_leaves * 4);
  const __amdgpu_buffer_rsrc_t fs_r =
      buffer_of(FS ? static_cast<const void*>(d.leaf_scale) : static_cast<const void*>(d.leaf_word), d.n_leaves * 4);
  const uint32_t pay0 = (uint32_t)hdr[0], leaf0 = (uint32_t)hdr[2];   // the unit's payload and leaf words
  auto slot_of = [&](uint32_t r) __attribute__((always_inline)) { return record_slot(rec_r, r, g); };
  // A step's per-lane view: chunk t = li of the step in this slot's column group, active if
  // li is below the slot's chunk count. Inactive lanes load the step's chunk 0 (a slot without
  // chunks names the unit's first payload dword and leaf word) and use nothing they load.
  struct Regs {
    u32x16_t w;
    uint32_t ob, lw0, lw1;
    float fs0, fs1;
    uint32_t t, key;
    bool on;
  };
  auto fetch = [&](const u32x2_t f, Regs& r) __attribute__((always_inline)) {
    r.key = record_key(f.y);                          // one kind per record
    r.on = (uint32_t)li < record_count(f.y, g);
    r.t = r.on ? (uint32_t)li : 0u;
    gemv_load<FS>(pay_r, lw_r, fs_r, r.key, pay0 + ((f.x & 0xFFFFu) << 2), leaf0 + (f.x >> 16), r.t, r.w, r.ob,
                  r.lw0, r.lw1, r.fs0, r.fs1);
  };

  // The first three steps: record wh + k*WH of the wave's half is a fixed record (or the null
  // record: a block with records past F has F = 48 >= 3W, so those indices are all fixed; 8-wave
  // blocks of 1-2 rows run only streams with F <= 16, whose blocks have no records past F). Their
  // records are read together with X; all of them are waited for here, before any payload
  // load, so that no later wait (the compiler counts loads in issue order, and the payload
  // load count varies with the kind) has to include payload that is still in flight.
  Regs r0, r1, r2;
  {
    auto fixed = [&](int k) __attribute__((always_inline)) {
      const int i = wh + k * WH;
      return slot_of(i < F ? (uint32_t)(blk * F + i) : null_rec);
    };
    static_assert(PF >= 1 && PF <= 3, "one to three prefetched steps");
    const u32x2_t f0 = fixed(0);
    u32x2_t f1 = {}, f2 = {};
    if constexpr (PF >= 2) f1 = fixed(1);
    if constexpr (PF >= 3) f2 = fixed(2);
    asm volatile("" ::"v"(f0.x));
    if constexpr (PF >= 2) asm volatile("" ::"v"(f1.x));
    if constexpr (PF >= 3) asm volatile("" ::"v"(f2.x));
    asm volatile("" ::"s"(pay0), "s"(leaf0));         // the unit's starts, read beside the records
#pragma unroll
    for (int i = 0; i < XG; ++i) asm volatile("" ::"v"(kk[i].x));
    if (lds_gather) {
#pragma unroll
      for (int m = 0; m < gemv_lds_gather_rows(MT); ++m)
#pragma unroll
        for (int i = 0; i < XR; ++i) asm volatile("" ::"v"(xr[m][i]));
    }
    fetch(f0, r0);
    if constexpr (PF >= 2) fetch(f1, r1);
    if constexpr (PF >= 3) fetch(f2, r2);
  }

  // ---- X rows of the unit (gathered) and their 4- and 8-row sums into LDS ----
  if (lds_gather) {
#pragma unroll
    for (int m = 0; m < gemv_lds_gather_rows(MT); ++m)
#pragma unroll
      for (int i = 0; i < XR; ++i) {
        const int k = i * T + tid;
        if (k < d.K) xraw[m * d.K + k] = xr[m][i];
      }
    lds_barrier();
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float* xrow = X + (int64_t)min(m0 + m, M - 1) * ldx;
    const bool mv = m0 + m < M;
    float4 xv[XG];
    if (lds_gather) {
      const float* xl = xraw + m * d.K;
#pragma unroll
      for (int i = 0; i < XG; ++i) {
        const int r = 4 * (i * T + tid);
        xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r < rows && mv) xv[i] = make_float4(xl[kk[i].x], xl[kk[i].y], xl[kk[i].z], xl[kk[i].w]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < XG; ++i) {
        const int r = 4 * (i * T + tid);
        xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r < rows && mv) xv[i] = make_float4(xrow[kk[i].x], xrow[kk[i].y], xrow[kk[i].z], xrow[kk[i].w]);
      }
    }
#pragma unroll
    for (int i = 0; i < XG; ++i) {
      const int r = 4 * (i * T + tid);
      if (i * 4 * T < kc) {                           // wave-uniform: the loop covers kc rows
        const float s4 = (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
        const float s8 = s4 + __shfl_xor(s4, 1, 64);  // rows r & ~7 .. +7: this lane and its pair
        if (r < kc) {
          *reinterpret_cast<float4*>(xs + m * kc + r) = xv[i];
          if constexpr (gemv_sum4(MT)) xs4[m * (kc / 4) + (r >> 2)] = s4;
          if ((r & 7) == 0) xs8[m * (kc / 8) + (r >> 3)] = s8;
        }
      }
    }
  }
  lds_barrier();                                      // payload loads stay in flight
  const XStage xt{xs, xs4, xs8, kc};

  // ---- decode: the prefetched steps, then any further steps one at a time. The wave's k-th
  //      record (wh + k WH of its half) accumulates into set k % H: set s holds what wave
  //      wh + s WH of a one-half block sums (its records wh + s WH + j W). ----
  float acc[H][MT][kGroup];
#pragma unroll
  for (int s = 0; s < H; ++s)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < kGroup; ++c) acc[s][m][c] = 0.0f;
  auto compute = [&](const Regs& cur, float (&acc)[MT][kGroup]) __attribute__((always_inline)) {
    if (cur.on) {
      const uint32_t key = cur.key;
      const uint32_t ls = key & 0xFFu;
      const uint32_t rb_mask = ls > 3 ? (1u << (ls - 3)) - 1u : 0u;
      switch (ls == 2 ? key : (key & ~0xFFu) | 3u) {   // sizes 8, 16, 32 share a case
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): \
    gemv_chunk<S, P, MT>(P == 16 ? gemv_load_p16_tail(pay_r, cur.w, cur.ob) : cur.w, cur.lw0, cur.lw1, cur.fs0, \
                         cur.fs1, FS, cur.t, rb_mask, xt, acc); \
    break;
        MTC_FOR_EACH_WIDTH(8, MTC_CASE)
        MTC_FOR_EACH_WIDTH(4, MTC_CASE)
#undef MTC_CASE
        default: break;
      }
    }
  };
  // Records past the prefetched ones, in the same order: each one's slot is loaded a record
  // ahead (while the previous record computes), so only its payload load is waited for.
  const int nrec = hdr[28 + 2 * cb];
  const uint32_t ovf = (uint32_t)hdr[27 + 2 * cb];
  auto rec = [&](int i) __attribute__((always_inline)) {
    return i < F ? (uint32_t)(blk * F + i) : ovf + (uint32_t)(i - F);
  };
  static_assert(H == 1 || PF == 2, "two accumulator sets alternate from the third record on");
  int i = wh + PF * WH;
  compute(r0, acc[0]);                                // null records have no active lanes
  u32x2_t nxt = {};                                   // loaded once r0's registers are free
  if (i < nrec) nxt = slot_of(rec(i));
  if constexpr (PF >= 2) compute(r1, acc[1 % H]);
  if constexpr (PF >= 3) compute(r2, acc[2 % H]);
  if constexpr (H == 1) {
    for (; i < nrec; i += WH) {
      fetch(nxt, r0);
      if (i + WH < nrec) nxt = slot_of(rec(i + WH));
      compute(r0, acc[0]);
    }
  } else {
    for (; i < nrec; i += 2 * WH) {
      fetch(nxt, r0);
      if (i + WH < nrec) nxt = slot_of(rec(i + WH));
      compute(r0, acc[0]);
      if (i + WH >= nrec) break;
      fetch(nxt, r0);
      if (i + 2 * WH < nrec) nxt = slot_of(rec(i + 2 * WH));
      compute(r0, acc[1]);
    }
  }

  // ---- reduce: the 16 lanes of each slot, then the block's partials (set s of wave wh of half
  //      cb is partial wh + s WH of the half, the place of that wave in a one-half block) ----
#pragma unroll
  for (int s = 0; s < H; ++s)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < kGroup; ++c) acc[s][m][c] = slot_sum(acc[s][m][c]);
  if (li == kSlotSumLane) {
    const int p0 = (H == 2 ? cb * W : 0) + wh;       // this wave's first partial
#pragma unroll
    for (int s = 0; s < H; ++s)
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < kGroup; ++c)
          red[(((p0 + s * WH) * kStepGroups + g) * MT + m) * kGroup + c] = acc[s][m][c];
  }
  __syncthreads();
  gemv_store<MT, W, H, W>(d, red, u, H == 2 ? 0 : cb, Y, ldy, M, part, counters);
}

// ---------------------------------------------------------------------------
// Decode blocks for M tiles of 8 or 16 rows, on the matrix core.
// v_mfma_f32_4x4x1_16b_f32 runs 16 independent 4x4 outer products per wave: block b (lanes
// 4b .. 4b+3) adds A_b (x) B_b to its 4x4 accumulator, with A_b[i] from lane 4b + i, B_b[j]
// from lane 4b + j, and D_b[i][j] held by lane 4b + j in accumulator register i. A lane
// chunk (8 rows x 4 columns of one column group, rows chosen by its leaf) is one such block:
// lane 4b + j decodes the chunk's column j (8 codes) into weights s * q and, for row r =
// 0..7 in turn, multiplies them with X[m0 + 4h + j][row r] for every 4-row slice h of the M
// tile (one accumulator per slice, so consecutive MFMAs are independent). A step record's
// 4 slots x 16 chunks take four passes of 16 chunks: in pass p, lane (slot g, li) takes
// chunk 4p + li / 4 of slot g's bucket, column li % 4. The weights equal the dequantized
// W_hat (one fma rounding of s * (u - 2^(P-1)), exact in q), and every product accumulates
// in fp32. The lane -> chunk order, and so every sum, is the same for M tiles of 8 and 16
// rows: the tile height only sets how many X rows one block stages.
// X is staged in LDS as xs[r][j][h] = X[m0 + 4h + j][row r of the unit], so the slices a
// lane needs for one row are adjacent (one 16- or 8-byte read). A staging launch writes X
// transposed into that order once per call (xt[k][j][h], in the workspace), so a block
// gathers each of its rows (through row_perm) as one 32- or 64-byte piece; without it
// (grouped launches) each block gathers its rows from X itself, 4 bytes at a time.
// One block covers a whole unit (both 16-column halves of its panel, waves 0-7 and 8-15),
// so that a unit's X rows are staged once.
// ---------------------------------------------------------------------------
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kMfmaWaves = 16;
// 16-byte X pieces per thread when a block stages its rows: kc * MT floats fit the LDS next to
// the reduction buffer (at most 144 KB for 16-row tiles), over 1024 threads.
constexpr int kMfmaStageIters = 9;

// X of one M tile transposed for the matrix core: xt[k][j][h] = X[m0 + 4h + j][k] (original
// row order, k < K; M rows past M are zero). Thread k of the launch writes row k's MT values.
__device__ __forceinline__ int mfma_slot(int m, int MT) { return (m & 3) * (MT / 4) + (m >> 2); }
constexpr int kStageThreads = 64;

template <int MT>
__device__ __forceinline__ void stage_xt_block(int K, const float* __restrict__ X, int64_t ldx,
                                               const int32_t* __restrict__ row_perm, int M, float* __restrict__ xt) {
  // one thread per 16-byte piece of xt: row k, slots 4i .. 4i+3 of its MT (consecutive threads
  // write consecutive pieces); slot s holds M row 4 (s % Q) + s / Q (the inverse of mfma_slot)
  constexpr int Q = MT / 4;
  const int64_t t = (int64_t)blockIdx.x * kStageThreads + (int)threadIdx.x;
  if (t >= (int64_t)K * Q) return;
  const int k = (int)(t / Q), i = (int)(t - (int64_t)k * Q);
  const int m0 = (int)blockIdx.y * MT;
  const int src = row_perm ? row_perm[k] : k;         // xt row k holds X[:, row_perm[k]]
  float v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int sl = 4 * i + u, m = 4 * (sl % Q) + sl / Q;
    v[u] = m0 + m < M ? X[(int64_t)(m0 + m) * ldx + src] : 0.0f;
  }
  *reinterpret_cast<float4*>(xt + ((size_t)blockIdx.y * K + k) * MT + 4 * i) = make_float4(v[0], v[1], v[2], v[3]);
}

template <int MT>
__global__ __launch_bounds__(kStageThreads) void k_gemv_stage_x(int K, const float* __restrict__ X, int64_t ldx,
                                                                const int32_t* __restrict__ row_perm, int M,
                                                                float* __restrict__ xt) {
  stage_xt_block<MT>(K, X, ldx, row_perm, M, xt);
}

// A lane's loads of one pass: the 64-bit window(s) holding its column's codes (two loads for
// every kind: leaf 0's and leaf 1's windows for two 4x4 leaves; the two halves of a 128-bit
// window for P = 16; the whole 3-dword chunk and the dword after it for P = 3, whose codes sit
// in byte lanes; the window and a load past the buffer's end, which reads zeros, for other
// widths), the leaf word(s) and, with fp32 scales, the leaf scale(s). Same load count for
// every kind, so the compiler's in-order waits stay exact.
struct MfmaPass {
  u32x4_t w;
  uint32_t lw0, lw1;
  float fs0, fs1;
};

// The loads of a record's four passes. Pass p of lane (slot, chunk cq, column j) takes chunk
// t0 + 4p of the step (t0 = cq; pay and leaf name the step's first chunk and its first leaf
// word in the slot's column group), so every offset is pass 0's plus a
// wave-uniform step per pass: 4 chunks of P dwords of payload, and the leaf words of 4
// chunks (8 for two 4x4 leaves per chunk, 4 >> (log2 S - 3) for larger leaves). Chunks past the bucket's
// end are read in place (the stream's next chunks, or zeros past a buffer's end) and masked
// by the caller.
template <bool FS, int NP>
__device__ __forceinline__ void mfma_load_rec(__amdgpu_buffer_rsrc_t pay_r, __amdgpu_buffer_rsrc_t lw_r,
                                              __amdgpu_buffer_rsrc_t fs_r, uint32_t key, uint32_t pay,
                                              uint32_t leaf, uint32_t t0, uint32_t j, MfmaPass (&r)[NP]) {
  const uint32_t P = key >> 8, ls = key & 0xFFu;
  const uint32_t ob = (pay + t0 * P) << 2;           // payload byte offset of pass 0's chunk
  const bool two = ls == 2;                          // two 4x4 leaves per chunk
  uint32_t o0, o1;
  if (P == 3) {                                      // byte lanes: every column spans the chunk
    o0 = ob;
    o1 = ob + 8;
  } else if (two) {                                  // codes 4j.. of leaf 0 and 16 + 4j.. of leaf 1
    o0 = ob + (((4 * j * P) >> 5) << 2);
    o1 = ob + ((((16 + 4 * j) * P) >> 5) << 2);
  } else if (P == 16) {                              // codes 8j .. 8j + 7: 128 bits at dword 4j
    o0 = ob + 16 * j;
    o1 = o0 + 8;
  } else {                                           // codes 8j .. 8j + 7: 8P <= 64 bits
    o0 = ob + (((8 * j * P) >> 5) << 2);
    o1 = kOutOfRange;
  }
  const bool o1_used = two || P == 16 || P == 3;
  const uint32_t sh = ls >= 3 ? ls - 3 : 0u;         // leaf sizes 8, 16, 32 (the null record has ls = 0)
  const uint32_t l0 = leaf + (two ? 2 * t0 : t0 >> sh);
  const uint32_t pstep = 16 * P;                     // bytes of 4 chunks (P dwords each)
  const uint32_t lstep = 4 * (two ? 8u : 4u >> sh);  // bytes of the leaf words of 4 chunks
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const uint32_t a = o0 + p * pstep, b = o1_used ? o1 + p * pstep : kOutOfRange;
    const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(pay_r, a, 0, kNT);
    const u32x2_t y = __builtin_amdgcn_raw_buffer_load_b64(pay_r, b, 0, kNT);
    r[p].w = u32x4_t{x.x, x.y, y.x, y.y};
    const uint32_t w0 = (l0 << 2) + p * lstep, w1 = two ? w0 + 4 : kOutOfRange;
    r[p].lw0 = __builtin_amdgcn_raw_buffer_load_b32(lw_r, w0, 0, 0);
    r[p].lw1 = __builtin_amdgcn_raw_buffer_load_b32(lw_r, w1, 0, 0);
    if constexpr (FS) {
      r[p].fs0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(fs_r, w0, 0, 0));
      r[p].fs1 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(fs_r, w1, 0, 0));
    } else {
      r[p].fs0 = r[p].fs1 = 0.0f;
    }
  }
}

// NC codes of width P, the first at bit `o` (0..31) of the 64-bit window (lo, hi), as floats.
// Z: o is known to be 0 for this kind.
template <int P, int NC, bool Z>
__device__ __forceinline__ void window_codes(uint32_t lo, uint32_t hi, uint32_t o, float* u) {
  const uint32_t a = Z ? lo : __builtin_amdgcn_alignbit(hi, lo, o);   // window bits o .. o + 31
  const uint32_t b = Z ? hi : hi >> o;                                // window bits o + 32 .. 63
  constexpr uint32_t mask = (1u << P) - 1u;
#pragma unroll
  for (int r = 0; r < NC; ++r) {
    const int s = r * P;
    uint32_t v;
    if (s + P <= 32) v = (a >> s) & mask;
    else if (s >= 32) v = (b >> (s - 32)) & mask;
    else v = __builtin_amdgcn_alignbit(b, a, s) & mask;
    u[r] = (float)v;
  }
}

// Byte lane b (0..3) of a 3-bit chunk (dwords w0, w1, w2) as one 24-bit string: codes 8b ..
// 8b + 7 at bits 0, 3, .., 21. Two byte permutes.
__device__ __forceinline__ uint32_t p3_lane(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t b) {
  const uint32_t lo = __builtin_amdgcn_perm(w1, w0, b | ((4u + b) << 8) | 0x0C0C0000u);   // w0.b, w1.b, 0, 0
  return __builtin_amdgcn_perm(w2, lo, 0x0C000100u | ((4u + b) << 16));                   // lo.0, lo.1, w2.b, 0
}

// A lane's column of its chunk in one pass of kind (S, P): the 8 weights (zero when the
// lane's chunk is not in the bucket, `on` false, or its leaf is padding) and the unit rows
// they sit on (rows row0 .. row0 + 3 and row1 .. row1 + 3; row_off: the chunk's 8-row block
// within a leaf of 16 or 32 rows).
template <int S, int P>
__device__ __forceinline__ void mfma_decode(const MfmaPass& r, bool on, int row_off, uint32_t j, bool fp32_scales,
                                            float (&wq)[8], int& row0, int& row1) {
  static_assert(S == 4 || S == 8, "leaf sizes 16 and 32 take the S = 8 path");
  constexpr float off = (float)(1 << (P - 1));
  float u[8];
  float s0, s1;
  // the column's 8 codes
  if constexpr (P == 3) {
    if constexpr (S == 4) {
      // codes 4j + k (leaf 0) and 16 + 4j + k (leaf 1): byte lanes j/2 and 2 + j/2, from bit 12 (j & 1)
      const uint32_t l0 = p3_lane(r.w.x, r.w.y, r.w.z, j >> 1), l1 = p3_lane(r.w.x, r.w.y, r.w.z, 2u + (j >> 1));
      const uint32_t o = 12u * (j & 1u);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        u[k] = (float)__builtin_amdgcn_ubfe(l0, o + 3u * k, 3u);
        u[4 + k] = (float)__builtin_amdgcn_ubfe(l1, o + 3u * k, 3u);
      }
    } else {
      const uint32_t l = p3_lane(r.w.x, r.w.y, r.w.z, j);   // codes 8j .. 8j + 7: byte lane j
#pragma unroll
      for (int k = 0; k < 8; ++k) u[k] = (float)((l >> (3 * k)) & 7u);
    }
  } else if constexpr (S == 4) {
    window_codes<P, 4, (P >= 8)>(r.w.x, r.w.y, (4 * j * P) & 31u, u);
    window_codes<P, 4, (P >= 8)>(r.w.z, r.w.w, ((16 + 4 * j) * P) & 31u, u + 4);
  } else if constexpr (P == 16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      u[2 * k] = (float)(r.w[k] & 0xFFFFu);
      u[2 * k + 1] = (float)(r.w[k] >> 16);
    }
  } else {
    window_codes<P, 8, (P == 4 || P == 8)>(r.w.x, r.w.y, (8 * j * P) & 31u, u);
  }
  // their leaves: rows and scales
  if constexpr (S == 4) {
    const LeafInfo a = leaf_info_v(r.lw0, fp32_scales, r.fs0), b = leaf_info_v(r.lw1, fp32_scales, r.fs1);
    row0 = on ? a.row : 0;                           // a masked lane's leaf may be any unit's
    row1 = on ? b.row : 0;
    s0 = (on && !a.pad) ? a.scale : 0.0f;
    s1 = (on && !b.pad) ? b.scale : 0.0f;
  } else {
    const LeafInfo a = leaf_info_v(r.lw0, fp32_scales, r.fs0);
    row0 = on ? a.row + row_off : 0;                 // a masked lane's leaf may be any unit's
    row1 = row0 + 4;
    s0 = s1 = (on && !a.pad) ? a.scale : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float s = k < 4 ? s0 : s1;
    wq[k] = __builtin_fmaf(u[k], s, -(s * off));     // s * (u - off): s * off is exact
  }
}

// LDS of a matrix-core decode block: X rows [kc][MT] and the cross-wave reduction.
__host__ __device__ constexpr size_t gemv_mfma_lds_floats(int MT, int kc) {
  return (size_t)MT * kc + (size_t)kMfmaWaves * kStepGroups * MT * kGroup;
}

template <int MT, bool FS>
__device__ __forceinline__ void gemv_block_mfma(const mtc_stream_desc& d, const int bid, const float* __restrict__ X,
                                                int64_t ldx, float* __restrict__ Y, int64_t ldy, int M,
                                                float* __restrict__ part, uint32_t* __restrict__ counters,
                                                const float* __restrict__ xt) {
  static_assert(MT == 8 || MT == 16, "M tiles of 8 or 16 rows");
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int W = kMfmaWaves, T = 64 * W, BPU = kGemvBlocksPerUnit, NP = kStepLanes / 4, Q = MT / 4;
  constexpr int WH = W / BPU;                         // waves per column half
  const int kc = d.chunk_rows;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_units = d.n_panels * d.n_chunks;
  const int u = bid;                                  // grid x: one block per unit
  if (u >= n_units) return;                           // padding block of the XCD rounding
  const int cb = wave / WH, wl = wave % WH;           // this wave's column half, its index there
  const int m0 = blockIdx.y * MT;
  const int chunk = u % d.n_chunks;
  const int kb = chunk * kc;
  const int rows = min(kc, d.K - kb);
  float* xs = smem;                                   // [kc][4 j][Q h]
  float* red = xs + MT * kc;                          // [waves][4 slots][MT][4]
  const ci32p hdr = (ci32p)(d.unit_hdr + kUnitHdr * u);

  const int F = d.fixed_steps;
  const int blk = u * BPU + cb;
  const uint32_t null_rec = (uint32_t)(n_units * BPU) * (uint32_t)F;
  const int g = lane / kStepLanes, li = lane % kStepLanes;
  const uint32_t j = (uint32_t)(li & 3), cq = (uint32_t)(li >> 2);   // column in the chunk, chunk in the pass
  const __amdgpu_buffer_rsrc_t rec_r = buffer_of(d.steps, d.n_steps * kStepWords * 4);
  const __amdgpu_buffer_rsrc_t pay_r = buffer_of(d.payload, d.payload_dwords * 4);
  const __amdgpu_buffer_rsrc_t lw_r = buffer_of(d.leaf_word, d.n_leaves * 4);
  const __amdgpu_buffer_rsrc_t fs_r =
      buffer_of(FS ? static_cast<const void*>(d.leaf_scale) : static_cast<const void*>(d.leaf_word), d.n_leaves * 4);
  const int nrec = hdr[28 + 2 * cb];
  const uint32_t ovf = (uint32_t)hdr[27 + 2 * cb];
  // record index of the block's i-th record: the first F at block-computable places, the rest
  // (F = 48 only) in the unit's overflow list; past the block's end, the null record
  auto rec_of = [&](int i) __attribute__((always_inline)) {
    return i < F ? (uint32_t)(blk * F + i) : i < nrec ? ovf + (uint32_t)(i - F) : null_rec;
  };
  const uint32_t pay0 = (uint32_t)hdr[0], leaf0 = (uint32_t)hdr[2];   // the unit's payload and leaf words
  auto slot_of = [&](uint32_t r) __attribute__((always_inline)) { return record_slot(rec_r, r, g); };
  struct Rec {
    MfmaPass p[NP];
    uint32_t key, valid;
  };
  auto fetch = [&](const u32x2_t f, Rec& r) __attribute__((always_inline)) {
    r.key = record_key(f.y);
    r.valid = record_count(f.y, g);
    mfma_load_rec<FS, NP>(pay_r, lw_r, fs_r, r.key, pay0 + ((f.x & 0xFFFFu) << 2), leaf0 + (f.x >> 16), cq, j, r.p);
  };

  // ---- X rows of the unit into LDS, overlapped with the first records' loads. The compiler
  //      waits for loads in issue order, so the order is: record slots, X pieces, then the
  //      first record's payload; the LDS stores wait for the X pieces only and the payload
  //      stays in flight. xt holds X[:, row_perm] (the staging launch gathered it), so the
  //      unit's rows are one contiguous slab of MT-float pieces (16 bytes per thread); kc * MT
  //      fits the LDS, so a thread has at most kMfmaStageIters pieces. ----
  constexpr int L = MT / 4;                           // threads per row
  int kr[kMfmaStageIters];
  if (xt) {
#pragma unroll
    for (int it = 0; it < kMfmaStageIters; ++it) {
      const int r = (it * T + tid) / L;
      kr[it] = r < rows ? kb + r : -1;
    }
  }
  const u32x2_t f0 = slot_of(rec_of(wl));
  u32x2_t f1 = slot_of(rec_of(wl + WH));
  float4 v[kMfmaStageIters];
  if (xt) {
    const float* src = xt + (size_t)blockIdx.y * d.K * MT;
#pragma unroll
    for (int it = 0; it < kMfmaStageIters; ++it) {
      const int part4 = (it * T + tid) % L;
      v[it] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (kr[it] >= 0) v[it] = *reinterpret_cast<const float4*>(src + (size_t)kr[it] * MT + 4 * part4);
    }
  }
  Rec cur, nxt;
  fetch(f0, cur);
  if (xt) {
#pragma unroll
    for (int it = 0; it < kMfmaStageIters; ++it) {
      const int i = it * T + tid;
      if (i < kc * L) *reinterpret_cast<float4*>(xs + 4 * i) = v[it];
    }
  } else {
    const int r4 = 4 * tid;                           // this thread's 4 rows (kc <= 4096 = 4T)
    if (r4 < kc) {
      int4 kk = make_int4(kb + r4, kb + r4 + 1, kb + r4 + 2, kb + r4 + 3);
      if (d.row_perm && r4 < rows) kk = *reinterpret_cast<const int4*>(d.row_perm + kb + r4);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float* xrow = X + (int64_t)min(m0 + m, M - 1) * ldx;
        float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r4 < rows && m0 + m < M) xv = make_float4(xrow[kk.x], xrow[kk.y], xrow[kk.z], xrow[kk.w]);
        float* o = xs + r4 * MT + mfma_slot(m, MT);
        o[0] = xv.x;
        o[MT] = xv.y;
        o[2 * MT] = xv.z;
        o[3 * MT] = xv.w;
      }
    }
  }
  lds_barrier();                                      // record loads stay in flight

  f32x4_t acc[Q];
#pragma unroll
  for (int h = 0; h < Q; ++h) acc[h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const float* xl = xs + (int)j * Q;                  // this lane's M rows m0 + 4h + j
  auto compute = [&](const Rec& r) __attribute__((always_inline)) {
    // passes holding any chunk of the record (slots share a kind, not a chunk count)
    const uint32_t vmax = max(max(__builtin_amdgcn_readlane(r.valid, 0), __builtin_amdgcn_readlane(r.valid, 16)),
                              max(__builtin_amdgcn_readlane(r.valid, 32), __builtin_amdgcn_readlane(r.valid, 48)));
    const uint32_t key = r.key, ls = key & 0xFFu;
    // 8-row block of the chunk within its leaf (chunk t of the bucket is block t & (S/8 - 1);
    // t = 16 step + 4p + cq, so only cq matters)
    const int row_off = ls > 3 ? 8 * (int)(cq & ((1u << (ls - 3)) - 1u)) : 0;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if ((uint32_t)(4 * p) >= vmax) break;
      const bool on = 4 * p + cq < r.valid;
      float wq[8];
      int row0 = 0, row1 = 0;
      switch (ls == 2 ? key : (key & ~0xFFu) | 3u) {   // sizes 8, 16, 32 share a case
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): \
    mfma_decode<S, P>(r.p[p], on, row_off, j, FS, wq, row0, row1); \
    break;
        MTC_FOR_EACH_WIDTH(8, MTC_CASE)
        MTC_FOR_EACH_WIDTH(4, MTC_CASE)
#undef MTC_CASE
        default:
#pragma unroll
          for (int k = 0; k < 8; ++k) wq[k] = 0.0f;
          break;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int row = k < 4 ? row0 + k : row1 + (k - 4);
        if constexpr (Q == 4) {
          const float4 xq = *reinterpret_cast<const float4*>(xl + row * MT);
          acc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq.x, wq[k], acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq.y, wq[k], acc[1], 0, 0, 0);
          acc[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq.z, wq[k], acc[2], 0, 0, 0);
          acc[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq.w, wq[k], acc[3], 0, 0, 0);
        } else {
          const float2 xq = *reinterpret_cast<const float2*>(xl + row * MT);
          acc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq.x, wq[k], acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq.y, wq[k], acc[1], 0, 0, 0);
        }
      }
    }
  };
  // two records in flight: while one is computed the next one's loads (and the record
  // after that's slot) are outstanding
  for (int i = wl; i < nrec; i += 2 * WH) {
    u32x2_t f2 = slot_of(rec_of(i + 2 * WH));
    if (i + WH < nrec) fetch(f1, nxt);
    compute(cur);
    if (i + WH >= nrec) break;
    f1 = slot_of(rec_of(i + 3 * WH));
    if (i + 2 * WH < nrec) fetch(f2, cur);
    compute(nxt);
  }

  // ---- reduce: the 4 chunks of each slot (lanes li, li + 4, li + 8, li + 12), then the waves ----
#pragma unroll
  for (int h = 0; h < Q; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[h][i];
      v += row_shr<4>(v);
      v += row_shr<8>(v);
      acc[h][i] = v;
    }
  if (li >= kStepLanes - 4) {
#pragma unroll
    for (int h = 0; h < Q; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * kStepGroups + g) * MT + 4 * h + i) * kGroup + (int)j] = acc[h][i];
  }
  __syncthreads();
  gemv_store<MT, W, BPU>(d, red, u, 0, Y, ldy, M, part, counters);
}

#include "mtc_gemv_mx.h"

// The block code of an M tile: over an mx stream (MX) one X row on the matrix core with
// f16 operands; else the matrix core for tiles of 8 or 16 rows (X staged transposed in xt, or
// gathered by the block from X when xt is null), else the vector path with H column halves per
// block.
template <int MT, bool FS, bool LG, int NW, int KC, bool MX = false, int H = 1>
__device__ __forceinline__ void gemv_any(const mtc_stream_desc& d, const int bid, const float* __restrict__ X,
                                         int64_t ldx, float* __restrict__ Y, int64_t ldy, int M,
                                         float* __restrict__ part, uint32_t* __restrict__ counters, const bool lg,
                                         const float* __restrict__ xt) {
  if constexpr (MX) {
    static_assert(MT == 1, "the mx layout decodes one X row per block");
    gemv_block_mx<FS, LG, NW, KC>(d, bid, X, ldx, Y, ldy, M, part, counters, lg);
  } else if constexpr (MT >= 8) {
    static_assert(NW == kMfmaWaves, "matrix-core decode blocks have 16 waves");
    gemv_block_mfma<MT, FS>(d, bid, X, ldx, Y, ldy, M, part, counters, xt);
  } else {
    gemv_block<MT, FS, LG, NW, KC, H>(d, bid, X, ldx, Y, ldy, M, part, counters, lg);
  }
}

// At least 4 waves per SIMD: a 16-wave block fills a CU's 4 SIMDs; two 8-wave blocks
// (M tiles of 4 rows) share one only if each wave keeps to 128 VGPRs. 4-wave blocks over mx
// streams ask for 7 per CU, as the vector path's 4-wave blocks reach: a decode block's time is
// mostly memory latency, so the blocks in flight set the throughput.
__host__ __device__ constexpr int gemv_min_blocks(int NW, bool MX) { return MX && NW == 4 ? 7 : 4; }

template <int MT, bool FS, bool LG, int NW, int KC, bool MX>
__global__ __launch_bounds__(64 * NW, gemv_min_blocks(NW, MX)) void k_gemv(const mtc_stream_desc d, const float* __restrict__ X,
                                                  int64_t ldx, float* __restrict__ Y, int64_t ldy, int M,
                                                  float* __restrict__ part, uint32_t* __restrict__ counters,
                                                  const float* __restrict__ xt) {
  gemv_any<MT, FS, LG, NW, KC, MX>(d, blockIdx.x, X, ldx, Y, ldy, M, part, counters, true, xt);
}

// Up to kMaxGroup single-chunk matrices of one block shape that read the same X, in one launch:
// matrix i owns grid blocks [start[i], start[i + 1]) (each range a whole number of XCD rounds, so
// a block's XCD is the same as in a launch of its own).
constexpr int kMaxGroup = MTC_MAX_GROUP;
struct GemvGroup {
  mtc_stream_desc d[kMaxGroup];
  float* Y[kMaxGroup];
  int64_t ldy[kMaxGroup];
  int start[kMaxGroup + 1];
};

template <int MT, bool FS, bool LG, int NW, int KC, bool MX>
__global__ __launch_bounds__(64 * NW, gemv_min_blocks(NW, MX)) void k_gemv_group(const GemvGroup g, const float* __restrict__ X,
                                                        int64_t ldx, int M) {
  int i = 0;
#pragma unroll
  for (int k = 1; k < kMaxGroup; ++k) i += (int)blockIdx.x >= g.start[k];
  gemv_any<MT, FS, LG, NW, KC, MX>(g.d[i], (int)blockIdx.x - g.start[i], X, ldx, g.Y[i], g.ldy[i], M, nullptr,
                                   nullptr, true, nullptr);
}

// Any number of matrices, each with its own X and Y. The plan (built on the host by
// mtc_gemv_batch_plan and copied byte for byte to the device by the caller) holds one BatchItem
// per matrix and, per grid block, the index of its item. The members of each block shape
// (gemv_shape) run in one launch of that shape's kernel, so each block runs the block code of a
// launch of its own: every Y is bit-identical to the matrix's single call. Item i owns blocks
// [start, start + its blocks) of its shape's launch, a multiple of the XCD count, so each block
// also runs on the XCD it would run on alone.
struct BatchItem {
  mtc_stream_desc d;
  const float* X;
  float* Y;
  float* part;          // split-K partials and counters in the caller's workspace (n_chunks > 1)
  uint32_t* counters;
  float* xt;            // X staged for the matrix core (M tiles of 8 or 16 rows)
  int64_t ldx;
  int64_t ldy;
  int32_t start;        // first block of the item in its shape's launch
  int32_t lg;           // X rows gathered in LDS
};

// Shape classes of a batch, in the order of their blocks in the plan's block table:
// 0: 4 waves, X staging of kSmallRows rows (LDS gather per member); 1: 4 waves, kMaxChunkRows
// rows, no gather; 2: 16 waves, kMaxChunkRows rows (gather per member); 3: 8 waves (M tiles of
// 4 rows), no gather; 4, 5, 6: classes 0, 1, 2 over mx streams.
constexpr int kShapeClasses = 7;
inline int shape_class(const GemvShape& s) {
  const int c = s.nw == 8 ? 3 : s.nw == 16 ? 2 : s.kc == kSmallRows ? 0 : 1;
  return s.mx ? 4 + c : c;
}
inline int class_waves(int cls) { return cls == 3 ? 8 : (cls == 2 || cls == 6) ? 16 : 4; }

struct BatchHeader {
  uint32_t magic;
  uint32_t abi_version;
  int32_t n_items;
  int32_t n_blocks;
  int32_t M;
  int32_t mt;           // rows per M tile
  int32_t fs;           // fp32 leaf scales
  int32_t stage_blocks_x;   // grid x of the X staging (matrix-core M tiles)
  int32_t class_blocks[kShapeClasses];
  uint64_t lds_bytes;
  uint64_t items_off;   // byte offset of the BatchItem array
  uint64_t block_item_off;
  uint64_t plan_bytes;
  uint64_t ws_bytes;
  const void* workspace;
};
constexpr uint32_t kBatchMagic = 0x4D544342u;   // "BCTM"

template <int MT, bool FS, bool LG, int NW, int KC, bool MX>
__global__ __launch_bounds__(64 * NW, gemv_min_blocks(NW, MX)) void k_gemv_batch(const BatchItem* __restrict__ items,
                                                        const uint32_t* __restrict__ block_item, int M) {
  const int b = blockIdx.x;
  const BatchItem& it = items[block_item[b]];
  gemv_any<MT, FS, LG, NW, KC, MX, gemv_batch_halves(MT, NW, KC, MX)>(
      it.d, b - it.start, it.X, it.ldx, it.Y, it.ldy, M, it.part, it.counters, it.lg != 0, it.xt);
}

// X of every member staged for the matrix core (grid z: the member).
template <int MT>
__global__ __launch_bounds__(kStageThreads) void k_gemv_stage_x_batch(const BatchItem* __restrict__ items, int M) {
  const BatchItem& it = items[blockIdx.z];
  stage_xt_block<MT>(it.d.K, it.X, it.ldx, it.d.row_perm, M, it.xt);
}

// The batch kernel of a shape class (the LDS gather is a per-member flag there).
template <int MT>
const void* gemv_batch_kernel(bool fs, int cls) {
#define MTC_BATCH_K(LG_, NW_, KC_, MX_) \
  (fs ? reinterpret_cast<const void*>(&k_gemv_batch<MT, true, LG_, NW_, KC_, MX_>) \
      : reinterpret_cast<const void*>(&k_gemv_batch<MT, false, LG_, NW_, KC_, MX_>))
  if constexpr (MT > 4) {
    return MTC_BATCH_K(false, 16, kMaxChunkRows, false);
  } else if constexpr (MT > 2) {
    return MTC_BATCH_K(false, 8, kMaxChunkRows, false);
  } else {
    if constexpr (MT == 1) {
      if (cls == 4) return MTC_BATCH_K(true, 4, kSmallRows, true);
      if (cls == 5) return MTC_BATCH_K(false, 4, kMaxChunkRows, true);
      if (cls == 6) return MTC_BATCH_K(true, 16, kMaxChunkRows, true);
    }
    if (cls == 0) return MTC_BATCH_K(true, 4, kSmallRows, false);
    if (cls == 1) return MTC_BATCH_K(false, 4, kMaxChunkRows, false);
    return MTC_BATCH_K(true, 16, kMaxChunkRows, false);
  }
#undef MTC_BATCH_K
}

// The single-matrix (Group = false) or group kernel of an M tile, scale format and block shape.
template <int MT, bool Group>
const void* gemv_kernel(bool fs, const GemvShape& s) {
#define MTC_GEMV_K(LG_, NW_, KC_, MX_) \
  (Group ? (fs ? reinterpret_cast<const void*>(&k_gemv_group<MT, true, LG_, NW_, KC_, MX_>) \
               : reinterpret_cast<const void*>(&k_gemv_group<MT, false, LG_, NW_, KC_, MX_>)) \
         : (fs ? reinterpret_cast<const void*>(&k_gemv<MT, true, LG_, NW_, KC_, MX_>) \
               : reinterpret_cast<const void*>(&k_gemv<MT, false, LG_, NW_, KC_, MX_>)))
  if constexpr (MT > 4) {
    return MTC_GEMV_K(false, 16, kMaxChunkRows, false);
  } else if constexpr (MT > 2) {
    return MTC_GEMV_K(false, 8, kMaxChunkRows, false);
  } else {
    if constexpr (MT == 1) {
      if (s.mx) {
        if (s.nw == 16) return s.lg ? MTC_GEMV_K(true, 16, kMaxChunkRows, true) : MTC_GEMV_K(false, 16, kMaxChunkRows, true);
        if (s.kc == kSmallRows) return s.lg ? MTC_GEMV_K(true, 4, kSmallRows, true) : MTC_GEMV_K(false, 4, kSmallRows, true);
        return MTC_GEMV_K(false, 4, kMaxChunkRows, true);
      }
    }
    if (s.nw == 16) return s.lg ? MTC_GEMV_K(true, 16, kMaxChunkRows, false) : MTC_GEMV_K(false, 16, kMaxChunkRows, false);
    if (s.kc == kSmallRows) return s.lg ? MTC_GEMV_K(true, 4, kSmallRows, false) : MTC_GEMV_K(false, 4, kSmallRows, false);
    return MTC_GEMV_K(false, 4, kMaxChunkRows, false);
  }
#undef MTC_GEMV_K
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
int check_desc(const mtc_stream_desc* d) {
  if (!d) return fail(MTC_E_NULL, "descriptor is NULL");
  if (d->abi_version != MTC_ABI_VERSION)
    return fail(MTC_E_VERSION, "descriptor ABI %u, library ABI %d", d->abi_version, MTC_ABI_VERSION);
  if (d->K <= 0 || d->N <= 0 || d->N % kPanel || d->K % 8)
    return fail(MTC_E_DESC, "bad shape K=%d N=%d (N must be a multiple of %d, K of 8)", d->K, d->N, kPanel);
  if (d->chunk_rows <= 0 || d->chunk_rows % 32 || d->chunk_rows > kMaxChunkRows)
    return fail(MTC_E_DESC, "chunk_rows=%d must be a multiple of 32 in [32, %d]", d->chunk_rows, kMaxChunkRows);
  if (d->n_panels != d->N / kPanel) return fail(MTC_E_DESC, "n_panels=%d != N/32=%d", d->n_panels, d->N / kPanel);
  if (d->n_chunks != (d->K + d->chunk_rows - 1) / d->chunk_rows)
    return fail(MTC_E_DESC, "n_chunks=%d inconsistent with K=%d chunk_rows=%d", d->n_chunks, d->K, d->chunk_rows);
  if (!d->unit_hdr) return fail(MTC_E_NULL, "unit_hdr is NULL");
  if (d->max_unit_words < 0 || d->max_unit_words4 < d->max_unit_words)
    return fail(MTC_E_DESC, "max_unit_words=%d max_unit_words4=%d", d->max_unit_words, d->max_unit_words4);
  if (d->n_buckets > 0 && (!d->buckets || !d->payload || !d->leaf_word))
    return fail(MTC_E_NULL, "stream arrays missing for %d buckets", d->n_buckets);
  if (d->flags & ~(MTC_FLAG_FP32_SCALES | MTC_FLAG_MX_LAYOUT))
    return fail(MTC_E_DESC, "unknown descriptor flags 0x%x", d->flags);
  if ((d->flags & MTC_FLAG_FP32_SCALES) && !d->leaf_scale && d->n_leaves > 0)
    return fail(MTC_E_NULL, "fp32-scale stream without leaf_scale");
  if (!(d->flags & MTC_FLAG_FP32_SCALES) && d->leaf_scale)
    return fail(MTC_E_DESC, "leaf_scale given but MTC_FLAG_FP32_SCALES not set");
  if (d->n_steps < 0 || (d->n_buckets > 0 && (!d->steps || d->n_steps == 0)))
    return fail(MTC_E_NULL, "decode step records missing (n_steps=%lld)", (long long)d->n_steps);
  if (d->fixed_steps < 0 || d->fixed_steps > kMaxFixedSteps || d->fixed_steps % kStepLanes || d->reserved)
    return fail(MTC_E_DESC, "fixed_steps=%d must be 0, 16, 32 or 48 (reserved=%d must be 0)", d->fixed_steps,
                d->reserved);
  if (d->n_buckets > 0 &&
      d->n_steps < (int64_t)d->n_panels * d->n_chunks * kGemvBlocksPerUnit * d->fixed_steps + 1)
    return fail(MTC_E_DESC, "n_steps=%lld is less than the fixed record area plus the null record",
                (long long)d->n_steps);
  if ((reinterpret_cast<uintptr_t>(d->payload) | reinterpret_cast<uintptr_t>(d->row_perm)) % 16)
    return fail(MTC_E_DESC, "payload and row_perm must be 16-byte aligned");
  // the kernels address payload, leaf words and step records with 32-bit byte offsets
  if (d->payload_dwords < 0 || d->n_leaves < 0 || d->payload_dwords > kMaxArrayBytes / 4 ||
      d->n_leaves > kMaxArrayBytes / 4 || d->n_steps > kMaxArrayBytes / (4 * kStepWords))
    return fail(MTC_E_DESC, "stream arrays exceed 2 GiB (payload_dwords=%lld n_leaves=%lld n_steps=%lld)",
                (long long)d->payload_dwords, (long long)d->n_leaves, (long long)d->n_steps);
  return ok();
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

using mtc::host::device_lds_limit;

// Rows per M tile: 1, 2 or 4 on the vector path; 8, or 16 when 16 staged X rows of a unit fit
// on chip (chunk_rows <= kMfmaTile16Rows), on the matrix core (the sums are the same for both).
constexpr int kMfmaTile16Rows = 2048;
int gemv_mt(int M, int chunk_rows) {
  return M <= 2 ? M : M <= 4 ? 4 : (M <= 8 || chunk_rows > kMfmaTile16Rows) ? 8 : 16;
}
// Rows per M tile for a stream: one for the mx layout (its blocks decode one X row), else gemv_mt.
int gemv_mt_of(const mtc_stream_desc* d, int M) { return is_mx(d) ? 1 : gemv_mt(M, d->chunk_rows); }

// Workspace of a decode call: split-K counters (counters_bytes, from offset 0) and partials when
// K is split over row chunks, then, for matrix-core M tiles, X staged per M tile (from xt_off).
size_t gemv_ws_layout(const mtc_stream_desc* d, int M, int mt, size_t* counters_bytes, size_t* xt_off = nullptr) {
  const size_t n_mt = (size_t)((M + mt - 1) / mt);
  const size_t cb = ((n_mt * d->n_panels * sizeof(uint32_t)) + 255) & ~(size_t)255;
  if (counters_bytes) *counters_bytes = cb;
  size_t end = d->n_chunks == 1 ? 0 : cb + n_mt * (size_t)d->n_panels * d->n_chunks * mt * kPanel * sizeof(float);
  if (mt > 4) {
    end = (end + 255) & ~(size_t)255;
    if (xt_off) *xt_off = end;
    end += n_mt * (size_t)d->K * mt * sizeof(float);
  }
  return end;
}

// A matrix-core block stages at most kMfmaStageIters 16-byte X pieces per thread.
bool mfma_rows_fit(int mt, int chunk_rows) {
  return mt <= 4 || (size_t)chunk_rows * (mt / 4) <= (size_t)kMfmaStageIters * 64 * kMfmaWaves;
}

// Grid x of the X staging of one M tile.
// Grid x of the matrix-core X staging: one thread per 16-byte piece of xt (K * MT / 4).
unsigned stage_x_blocks(const mtc_stream_desc* d, int mt) {
  return (unsigned)(((int64_t)d->K * (mt / 4) + kStageThreads - 1) / kStageThreads);
}

// Decode blocks of one M tile: one per unit on the matrix core; on the vector path one per
// column half, or in a batched launch one per unit where gemv_batch_halves gives blocks both
// halves; the unit count rounded up to whole XCD rounds.
int gemv_blocks(const mtc_stream_desc* d, int mt, bool batch = false) {
  const int n_units = d->n_panels * d->n_chunks;
  if (mt > 4) return n_units;
  const GemvShape s = gemv_shape(mt, d);
  const int h = batch ? gemv_batch_halves(mt, s.nw, s.kc, s.mx) : 1;
  return (n_units + kXcds - 1) / kXcds * kXcds * (kGemvBlocksPerUnit / h);
}

// LDS of a decode block: X rows, their 4- and 8-row sums, the cross-wave reduction and,
// for the LDS gather, whole X rows.
size_t gemv_lds_bytes(int K, int chunk_rows, bool perm, int MT) {
  if (MT > 4) return gemv_mfma_lds_floats(MT, chunk_rows) * 4;
  const size_t kc = (size_t)chunk_rows;
  const size_t raw = gemv_lds_gather(MT, perm, K) ? (size_t)MT * K : 0;
  return ((size_t)MT * (kc + (gemv_sum4(MT) ? kc / 4 : 0) + kc / 8) +
          (size_t)gemv_waves(MT) * kStepGroups * MT * kGroup + raw) * 4;
}
size_t gemv_lds_bytes(const mtc_stream_desc* d, int MT) {
  if (is_mx(d))
    return gemv_mx_lds_bytes(d->chunk_rows, gemv_waves(1), gemv_lds_gather(1, d->row_perm != nullptr, d->K), d->K);
  return gemv_lds_bytes(d->K, d->chunk_rows, d->row_perm != nullptr, MT);
}

// The decode block of an M tile of MT rows fits the device (LDS, matrix-core X staging).
int check_gemv_fits(const mtc_stream_desc* d, int MT) {
  const size_t shmem = gemv_lds_bytes(d, MT);
  const size_t limit = device_lds_limit();
  if (shmem > limit || !mfma_rows_fit(MT, d->chunk_rows))
    return fail(MTC_E_SHAPE, "fp32 path: %d rows x chunk_rows=%d needs %zu B of LDS (limit %zu); "
                "use a stream with smaller chunk_rows", MT, d->chunk_rows, shmem, limit);
  return MTC_OK;
}

template <int MT>
int launch_gemv(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M, void* ws,
                hipStream_t st) {
  const int fits = check_gemv_fits(d, MT);          // before any launch
  if (fits) return fits;
  size_t cb = 0, xt_off = 0;
  gemv_ws_layout(d, M, MT, &cb, &xt_off);
  uint32_t* counters = reinterpret_cast<uint32_t*>(ws);
  float* part = ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + cb) : nullptr;
  float* xt = nullptr;
  if constexpr (MT > 4) {
    xt = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + xt_off);
    hipLaunchKernelGGL(k_gemv_stage_x<MT>, dim3(stage_x_blocks(d, MT), (M + MT - 1) / MT), dim3(kStageThreads), 0, st,
                       d->K, X, ldx, d->row_perm, M, xt);
    const int rc = check_launch("k_gemv_stage_x");
    if (rc) return rc;
  }
  const size_t shmem = gemv_lds_bytes(d, MT);
  const bool fs = d->leaf_scale != nullptr;
  const GemvShape shape = gemv_shape(MT, d);
  const void* kern = gemv_kernel<MT, false>(fs, shape);
  if (shmem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
    if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  }
  dim3 grid(gemv_blocks(d, MT), (M + MT - 1) / MT);
  const dim3 block(64 * shape.nw);
  void* args[] = {const_cast<mtc_stream_desc*>(d), &X, &ldx, &Y, &ldy, &M, &part, &counters, &xt};
  const hipError_t e = hipLaunchKernel(kern, grid, block, args, shmem, st);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "k_gemv launch: %s", hipGetErrorString(e));
  return check_launch("k_gemv");
}

// One launch for group members of one block shape (g holds only those members).
template <int MT>
int launch_gemv_group(const GemvGroup& g, int n, const GemvShape& shape, const float* X, int64_t ldx, int M,
                      hipStream_t st) {
  size_t shmem = 0;
  for (int i = 0; i < n; ++i) {
    shmem = std::max(shmem, gemv_lds_bytes(&g.d[i], MT));
    if (!mfma_rows_fit(MT, g.d[i].chunk_rows)) shmem = SIZE_MAX;
  }
  const size_t limit = device_lds_limit();
  if (shmem > limit)
    return fail(MTC_E_SHAPE, "fp32 group: %d rows need %zu B of LDS (limit %zu)", MT, shmem, limit);
  const void* kern = gemv_kernel<MT, true>(g.d[0].leaf_scale != nullptr, shape);
  if (shmem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
    if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  }
  dim3 grid(g.start[n], (M + MT - 1) / MT);
  const dim3 block(64 * shape.nw);
  void* args[] = {const_cast<GemvGroup*>(&g), &X, &ldx, &M};
  const hipError_t e = hipLaunchKernel(kern, grid, block, args, shmem, st);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "k_gemv_group launch: %s", hipGetErrorString(e));
  return check_launch("k_gemv_group");
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Plan of a batched decode launch (layout: BatchHeader, BatchItem[n], uint32 block_item[n_blocks]).
// With plan == NULL only the sizes are reported.
int build_batch_plan(const mtc_gemv_batch_item* items, int n, int M, void* workspace, size_t ws_bytes, void* plan,
                     size_t plan_bytes, size_t* plan_needed, size_t* ws_needed) {
  if (!items) return fail(MTC_E_NULL, "items is NULL");
  if (n < 1) return fail(MTC_E_SHAPE, "batch of %d matrices", n);
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  int max_rows = 0;
  for (int i = 0; i < n; ++i)
    if (items[i].desc) max_rows = std::max(max_rows, items[i].desc->chunk_rows);
  const bool mx = items[0].desc && is_mx(items[0].desc);
  for (int i = 1; i < n; ++i)
    if (items[i].desc && is_mx(items[i].desc) != mx)
      return fail(MTC_E_SHAPE, "batch item %d differs from item 0 in payload layout (MTC_FLAG_MX_LAYOUT)", i);
  const int mt = mx ? 1 : gemv_mt(M, max_rows);
  if (mt > 4 && n > 65535) return fail(MTC_E_SHAPE, "batch of %d matrices at M=%d (at most 65535 above M=4)", n, M);
  bool fs = false;
  size_t ws = 0, lds = 0;
  int64_t blocks = 0, class_blocks[kShapeClasses] = {};
  for (int i = 0; i < n; ++i) {
    const mtc_stream_desc* d = items[i].desc;
    int rc = check_desc(d);
    if (rc) {
      char why[400];
      snprintf(why, sizeof(why), "%s", mtc::host::last_error());
      return fail(rc, "batch item %d: %s", i, why);
    }
    if (!items[i].X || !items[i].Y) return fail(MTC_E_NULL, "batch item %d: X or Y is NULL", i);
    if (items[i].ldx < d->K || items[i].ldy < d->N)
      return fail(MTC_E_SHAPE, "batch item %d: ldx=%lld < K or ldy=%lld < N", i, (long long)items[i].ldx,
                  (long long)items[i].ldy);
    if ((M - 1) > (INT64_MAX / items[i].ldx)) return fail(MTC_E_SHAPE, "batch item %d: M * ldx overflows", i);
    const bool fsi = d->leaf_scale != nullptr;
    if (i == 0) fs = fsi;
    if (fsi != fs) return fail(MTC_E_SHAPE, "batch item %d differs from item 0 in scale format", i);
    lds = std::max(lds, mfma_rows_fit(mt, d->chunk_rows) ? gemv_lds_bytes(d, mt) : SIZE_MAX);
    ws += align_up(gemv_ws_layout(d, M, mt, nullptr), 256);
    const int64_t nb = gemv_blocks(d, mt, true);
    blocks += nb;
    class_blocks[shape_class(gemv_shape(mt, d))] += nb;
  }
  if (blocks > (1 << 30)) return fail(MTC_E_SHAPE, "batch of %lld blocks", (long long)blocks);
  const size_t items_off = align_up(sizeof(BatchHeader), 64);
  const size_t block_off = align_up(items_off + (size_t)n * sizeof(BatchItem), 64);
  const size_t need = block_off + (size_t)blocks * sizeof(uint32_t);
  if (plan_needed) *plan_needed = need;
  if (ws_needed) *ws_needed = ws;
  if (!plan) return ok();
  if (plan_bytes < need) return fail(MTC_E_WORKSPACE, "batch plan of %zu bytes needed, %zu given", need, plan_bytes);
  if (ws && (!workspace || ws_bytes < ws))
    return fail(MTC_E_WORKSPACE, "batch workspace of %zu bytes needed, %zu given", ws, workspace ? ws_bytes : 0);
  if (reinterpret_cast<uintptr_t>(plan) % 64) return fail(MTC_E_WORKSPACE, "batch plan not 64-byte aligned");
  const size_t limit = device_lds_limit();
  if (lds > limit) return fail(MTC_E_SHAPE, "batch needs %zu B of LDS per block (limit %zu)", lds, limit);
  unsigned char* base = reinterpret_cast<unsigned char*>(plan);
  memset(base, 0, need);
  BatchHeader* h = reinterpret_cast<BatchHeader*>(base);
  BatchItem* it = reinterpret_cast<BatchItem*>(base + items_off);
  uint32_t* block_item = reinterpret_cast<uint32_t*>(base + block_off);
  h->magic = kBatchMagic;
  h->abi_version = MTC_ABI_VERSION;
  h->n_items = n;
  h->n_blocks = (int32_t)blocks;
  h->M = M;
  h->mt = mt;
  for (int c = 0; c < kShapeClasses; ++c) h->class_blocks[c] = (int32_t)class_blocks[c];
  h->fs = fs;
  h->lds_bytes = lds;
  h->items_off = items_off;
  h->block_item_off = block_off;
  h->plan_bytes = need;
  h->ws_bytes = ws;
  h->workspace = workspace;
  char* wsp = reinterpret_cast<char*>(workspace);
  unsigned stage_bx = 0;
  int start[kShapeClasses] = {};                      // next block of each shape's launch
  int64_t table_off[kShapeClasses] = {};              // first table entry of each shape's launch
  for (int c = 1; c < kShapeClasses; ++c) table_off[c] = table_off[c - 1] + class_blocks[c - 1];
  for (int i = 0; i < n; ++i) {
    const mtc_stream_desc* d = items[i].desc;
    it[i].d = *d;
    it[i].X = items[i].X;
    it[i].Y = items[i].Y;
    it[i].ldx = items[i].ldx;
    it[i].ldy = items[i].ldy;
    const GemvShape shape = gemv_shape(mt, d);
    const int cls = shape_class(shape);
    it[i].lg = shape.lg;
    size_t cb = 0, xt_off = 0;
    const size_t wsi = gemv_ws_layout(d, M, mt, &cb, &xt_off);
    if (wsi) {
      if (d->n_chunks > 1) {
        it[i].counters = reinterpret_cast<uint32_t*>(wsp);
        it[i].part = reinterpret_cast<float*>(wsp + cb);
      }
      if (mt > 4) it[i].xt = reinterpret_cast<float*>(wsp + xt_off);
      wsp += align_up(wsi, 256);
    }
    stage_bx = std::max(stage_bx, stage_x_blocks(d, mt));
    const int nb = gemv_blocks(d, mt, true);
    uint32_t* table = block_item + table_off[cls];
    it[i].start = start[cls];
    for (int b = 0; b < nb; ++b) table[start[cls] + b] = (uint32_t)i;
    start[cls] += nb;
  }
  h->stage_blocks_x = (int32_t)stage_bx;
  return ok();
}

int launch_gemv_batch(const void* host_plan, const void* device_plan, hipStream_t st) {
  if (!host_plan || !device_plan) return fail(MTC_E_NULL, "host_plan or device_plan is NULL");
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(host_plan);
  if (h->magic != kBatchMagic || h->abi_version != MTC_ABI_VERSION)
    return fail(MTC_E_DESC, "not a batch plan of this library (magic 0x%x, ABI %u)", h->magic, h->abi_version);
  if (reinterpret_cast<uintptr_t>(device_plan) % 64) return fail(MTC_E_DESC, "device plan not 64-byte aligned");
  const unsigned char* dp = reinterpret_cast<const unsigned char*>(device_plan);
  const BatchItem* items = reinterpret_cast<const BatchItem*>(dp + h->items_off);
  const uint32_t* block_item = reinterpret_cast<const uint32_t*>(dp + h->block_item_off);
  int M = h->M;
  const size_t shmem = h->lds_bytes;
  if (h->mt > 4) {                                     // X of every member staged for the matrix core
    const dim3 grid((unsigned)h->stage_blocks_x, (unsigned)((M + h->mt - 1) / h->mt), (unsigned)h->n_items);
    if (h->mt == 8) hipLaunchKernelGGL(k_gemv_stage_x_batch<8>, grid, dim3(kStageThreads), 0, st, items, M);
    else hipLaunchKernelGGL(k_gemv_stage_x_batch<16>, grid, dim3(kStageThreads), 0, st, items, M);
    const int rc = check_launch("k_gemv_stage_x_batch");
    if (rc) return rc;
  }
  int64_t first = 0;
  for (int cls = 0; cls < kShapeClasses; ++cls) {      // one launch per block shape present
    const int nblk = h->class_blocks[cls];
    const uint32_t* table = block_item + first;
    first += nblk;
    if (nblk == 0) continue;
    const int nw = class_waves(cls);
    const void* kern = h->mt == 1   ? gemv_batch_kernel<1>(h->fs, cls)
                     : h->mt == 2   ? gemv_batch_kernel<2>(h->fs, cls)
                     : h->mt == 4   ? gemv_batch_kernel<4>(h->fs, cls)
                     : h->mt == 8   ? gemv_batch_kernel<8>(h->fs, cls)
                                    : gemv_batch_kernel<16>(h->fs, cls);
    if (shmem > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
      if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    }
    dim3 grid(nblk, (M + h->mt - 1) / h->mt);
    const dim3 block(64 * nw);
    void* args[] = {&items, &table, &M};
    const hipError_t e = hipLaunchKernel(kern, grid, block, args, shmem, st);
    if (e != hipSuccess) return fail(MTC_E_LAUNCH, "k_gemv_batch launch: %s", hipGetErrorString(e));
    const int rc = check_launch("k_gemv_batch");
    if (rc) return rc;
  }
  return ok();
}

}  // namespace

MTC_API int mtc_abi_version(void) { return MTC_ABI_VERSION; }

MTC_API int mtc_gemv_batch_plan(const mtc_gemv_batch_item* items, int n, int M, void* workspace,
                                size_t workspace_bytes, void* plan, size_t plan_bytes, size_t* plan_needed,
                                size_t* workspace_needed) {
  return build_batch_plan(items, n, M, workspace, workspace_bytes, plan, plan_bytes, plan_needed, workspace_needed);
}

MTC_API int mtc_gemv_f32_batch(const void* host_plan, const void* device_plan, void* hip_stream) {
  return launch_gemv_batch(host_plan, device_plan, as_stream(hip_stream));
}

MTC_API const char* mtc_last_error(void) { return mtc::host::last_error(); }

MTC_API int mtc_check_desc(const mtc_stream_desc* d) { return check_desc(d); }

MTC_API int mtc_dequant(const mtc_stream_desc* d, float* W_out, void* hip_stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!W_out) return fail(MTC_E_NULL, "W_out is NULL");
  hipStream_t st = as_stream(hip_stream);
  const int64_t n = (int64_t)d->K * d->N;
  const int fill_blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_fill_zero, dim3(fill_blocks), dim3(256), 0, st, W_out, n);
  rc = check_launch("k_fill_zero");
  if (rc) return rc;
  hipLaunchKernelGGL(k_dequant, dim3(d->n_panels * d->n_chunks), dim3(512), 0, st, *d, W_out);
  return check_launch("k_dequant");
}

MTC_API size_t mtc_gemv_lds_bytes(int K, int chunk_rows, int has_row_perm, int M) {
  if (K <= 0 || chunk_rows <= 0 || M <= 0) return 0;
  const size_t v1 = gemv_lds_bytes(K, chunk_rows, has_row_perm != 0, gemv_mt(M, chunk_rows));
  const size_t mx = gemv_mx_lds_bytes(chunk_rows, gemv_waves(1), gemv_lds_gather(1, has_row_perm != 0, K), K);
  return std::max(v1, mx);
}

MTC_API size_t mtc_gemv_workspace_bytes(const mtc_stream_desc* d, int M) {
  if (check_desc(d) || M <= 0) return 0;
  return gemv_ws_layout(d, M, gemv_mt_of(d, M), nullptr);
}

MTC_API int mtc_gemv_f32(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                         void* workspace, size_t workspace_bytes, void* hip_stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!X || !Y) return fail(MTC_E_NULL, "X or Y is NULL");
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  if (ldx < d->K || ldy < d->N) return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy=%lld < N", (long long)ldx, (long long)ldy);
  if ((M - 1) > (INT64_MAX / ldx)) return fail(MTC_E_SHAPE, "M * ldx overflows");
  const int mt = gemv_mt_of(d, M);
  const size_t need = gemv_ws_layout(d, M, mt, nullptr);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MTC_E_WORKSPACE, "GEMV workspace of %zu bytes needed, %zu given", need, workspace ? workspace_bytes : 0);
  hipStream_t st = as_stream(hip_stream);
  switch (mt) {
    case 1: return launch_gemv<1>(d, X, ldx, Y, ldy, M, workspace, st);
    case 2: return launch_gemv<2>(d, X, ldx, Y, ldy, M, workspace, st);
    case 4: return launch_gemv<4>(d, X, ldx, Y, ldy, M, workspace, st);
    case 8: return launch_gemv<8>(d, X, ldx, Y, ldy, M, workspace, st);
    default: return launch_gemv<16>(d, X, ldx, Y, ldy, M, workspace, st);
  }
}

// ---------------------------------------------------------------------------
// decode without a caller workspace: split-K partials and counters in a static per-device array
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = MTC_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
// In host code `scratch` names a host-side stand-in: kernels and copies get the device address
// from scratch_address() instead.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// The address of the current device's `scratch`, looked up once per device (with that device
// current) and kept.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MTC_E_LAUNCH, "device %d beyond the %d this library tracks", dev,
                                                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(MTC_E_LAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return MTC_OK;
}
}  // namespace

MTC_API size_t mtc_gemv_noalloc_scratch_bytes(void) { return kScratchBytes; }

MTC_API int mtc_gemv_f32_noalloc(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                                 void* hip_stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!X || !Y) return fail(MTC_E_NULL, "X or Y is NULL");
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  if (ldx < d->K || ldy < d->N) return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy=%lld < N", (long long)ldx, (long long)ldy);
  if ((M - 1) > (INT64_MAX / ldx)) return fail(MTC_E_SHAPE, "M * ldx overflows");
  size_t counter_bytes = 0;
  const int mt = gemv_mt_of(d, M);
  const size_t need = gemv_ws_layout(d, M, mt, &counter_bytes);
  if (need > kScratchBytes)
    return fail(MTC_E_WORKSPACE, "M=%d over %d row chunks needs %zu bytes of split-K scratch; the static scratch "
                "holds %zu (use mtc_gemv_f32 with a workspace)", M, d->n_chunks, need, kScratchBytes);
  rc = check_gemv_fits(d, mt);                       // fails before any launch
  if (rc) return rc;
  hipStream_t st = as_stream(hip_stream);
  void* ws = nullptr;
  if (need) {
    rc = scratch_address(&ws);
    if (rc) return rc;
  }
  if (d->n_chunks > 1) {
    // the split-K counters start at zero (a fill kernel: no memset node if the caller captures
    // this); single-chunk streams have none (their scratch holds only the staged X, if any)
    const int64_t words = (int64_t)(counter_bytes / sizeof(float));
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<float*>(ws), words);
    rc = check_launch("k_fill_zero");
    if (rc) return rc;
  }
  switch (mt) {
    case 1: return launch_gemv<1>(d, X, ldx, Y, ldy, M, ws, st);
    case 2: return launch_gemv<2>(d, X, ldx, Y, ldy, M, ws, st);
    case 4: return launch_gemv<4>(d, X, ldx, Y, ldy, M, ws, st);
    case 8: return launch_gemv<8>(d, X, ldx, Y, ldy, M, ws, st);
    default: return launch_gemv<16>(d, X, ldx, Y, ldy, M, ws, st);
  }
}

MTC_API int mtc_gemv_f32_group(const mtc_stream_desc* const* descs, int n, const float* X, int64_t ldx,
                               float* const* Y, const int64_t* ldy, int M, void* hip_stream) {
  if (!descs || !Y || !ldy) return fail(MTC_E_NULL, "descs, Y or ldy is NULL");
  if (n < 1 || n > kMaxGroup) return fail(MTC_E_SHAPE, "group of %d matrices (1..%d)", n, kMaxGroup);
  if (!X) return fail(MTC_E_NULL, "X is NULL");
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  for (int i = 0; i < n; ++i) {
    const mtc_stream_desc* d = descs[i];
    int rc = check_desc(d);
    if (rc) return rc;
    if (!Y[i]) return fail(MTC_E_NULL, "Y[%d] is NULL", i);
    if (d->n_chunks != 1)
      return fail(MTC_E_SHAPE, "group member %d has %d row chunks; groups take single-chunk streams", i, d->n_chunks);
    if (d->K != descs[0]->K) return fail(MTC_E_SHAPE, "group member %d has K=%d, member 0 K=%d", i, d->K, descs[0]->K);
    if ((d->leaf_scale != nullptr) != (descs[0]->leaf_scale != nullptr) ||
        (d->row_perm != nullptr) != (descs[0]->row_perm != nullptr) || is_mx(d) != is_mx(descs[0]))
      return fail(MTC_E_SHAPE, "group member %d differs from member 0 in scale format, row permutation or "
                  "payload layout", i);
    if (ldx < d->K || ldy[i] < d->N)
      return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy[%d]=%lld < N", (long long)ldx, i, (long long)ldy[i]);
  }
  if ((M - 1) > (INT64_MAX / ldx)) return fail(MTC_E_SHAPE, "M * ldx overflows");
  hipStream_t st = as_stream(hip_stream);
  int max_rows = 0;
  for (int i = 0; i < n; ++i) max_rows = std::max(max_rows, descs[i]->chunk_rows);
  const int mt = is_mx(descs[0]) ? 1 : gemv_mt(M, max_rows);
  // one launch per block shape among the members (usually one), so that every member's blocks
  // run the code of its own launch
  for (int cls = 0; cls < kShapeClasses; ++cls) {
    GemvGroup g;
    memset(&g, 0, sizeof(g));
    GemvShape shape{};
    int m = 0, blocks = 0;
    for (int i = 0; i < n; ++i) {
      const GemvShape si = gemv_shape(mt, descs[i]);
      if (shape_class(si) != cls) continue;
      shape = si;
      g.d[m] = *descs[i];
      g.Y[m] = Y[i];
      g.ldy[m] = ldy[i];
      g.start[m] = blocks;
      blocks += gemv_blocks(descs[i], mt);
      ++m;
    }
    if (m == 0) continue;
    for (int i = m; i <= kMaxGroup; ++i) g.start[i] = blocks;
    int rc;
    switch (mt) {
      case 1: rc = launch_gemv_group<1>(g, m, shape, X, ldx, M, st); break;
      case 2: rc = launch_gemv_group<2>(g, m, shape, X, ldx, M, st); break;
      case 4: rc = launch_gemv_group<4>(g, m, shape, X, ldx, M, st); break;
      case 8: rc = launch_gemv_group<8>(g, m, shape, X, ldx, M, st); break;
      default: rc = launch_gemv_group<16>(g, m, shape, X, ldx, M, st); break;
    }
    if (rc) return rc;
  }
  return ok();
}

// ---------------------------------------------------------------------------
// shared host state (declared in mtc_host.h)
// ---------------------------------------------------------------------------
namespace mtc {
namespace host {

namespace {
thread_local char g_err[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MTC_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

const char* last_error() { return g_err; }

size_t device_lds_limit() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 64 * 1024;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) return 64 * 1024;
  return (size_t)v;
}

}  // namespace host
}  // namespace mtc
