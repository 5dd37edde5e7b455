// gfx950 prefill kernel: Y = X * W_hat with W_hat decoded from the tile stream
// into bf16 LDS tiles and multiplied on v_mfma_f32_32x32x16_bf16 (fp32 accumulate).
//
//   k_stage_x_rows / k_stage_x : X -> bf16 Xp = X[:, row_perm] (only for fp32 X or a row
//                 permutation, and not for unpermuted fp32 X in the short tiles below);
//                 1-4 rows per block gathered through LDS, or, for rows wider than the LDS
//                 holds, one element per lane from global memory
//   k_gemm_tile : one 256 x 256 output tile per block, K in steps of 64. Warp-specialized:
//                 8 consumer waves (2 x 4 of 128 x 64 outputs) copy X tiles straight
//                 into LDS (buffer loads with the LDS destination, two steps ahead into
//                 three A buffers; unpermuted fp32 X in tiles of 64 or 128 rows goes
//                 through registers instead, rounded to bf16 on the way) and issue the
//                 MFMAs; 4 producer waves (one per SIMD)
//                 decode step k+1's weight cells from registers into the other of two B
//                 buffers and load step k+2's cell payload. Tiles use an XOR swizzle of
//                 16-byte segments; one LDS-only barrier per step (global loads stay in
//                 flight across it). Output columns go through col_perm.
//   k_tile_dequant_bf16 : prefill whose 256-row tiles fill the chip many times over decodes
//                 W_hat once into bf16 and multiplies it with a plain hipBLASLt GEMM instead
//                 (the tile kernel would decode each weight step once per row tile).
//
// Reference behaviour: mtc/kernels/gemm.py:124-210 (block loop: skip P0 blocks,
// unpack, scale, multiply-accumulate) with W_hat as in mtc/core/quadtree.py:157-171.

#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <vector>

#include "mtc_hip.h"
#include "mtc_host.h"

#define MTC_API extern "C" __attribute__((visibility("default")))

using mtc::host::check_launch;
using mtc::host::fail;
using mtc::host::ok;

namespace {

constexpr int kTM = 256;                    // output rows per block
constexpr int kTN = 256;                    // output columns per block (= one column tile)
constexpr int kTK = 64;                     // reduction rows per step
constexpr int kCells = 512;                 // cells per step
constexpr int kConsumerWaves = 8;           // 2 x 4 waves of 128 x 64 outputs
constexpr int kProducerWaves = 4;           // one per SIMD: loads, decode, LDS stores
constexpr int kThreads = 64 * (kConsumerWaves + kProducerWaves);
constexpr int kProducers = 64 * kProducerWaves;
constexpr int kTileBytes = kTM * kTK * 2;   // one bf16 operand tile (A and B are the same size)
constexpr int kABufs = 3;                   // A (X) buffers: copied two steps ahead
constexpr int kBBufs = 2;                   // B (decoded weight) buffers
constexpr int kLdsBytes = (kABufs + kBBufs) * kTileBytes;   // 160 KiB, all of a CU's LDS
constexpr uint32_t kOutOfRange = 0xFFFFFF00u;               // byte offset past any buffer's end
constexpr int kRowGroup = 8;                // row tiles per launch-order group (L2 reuse of B)
constexpr int kXcds = 8;
constexpr int kStageThreads = 256;
// Cell formats of a tile stream (its descriptor flags): bf16 scale pair (2 words), fp32 scales
// (4 words), gathered columns with a bf16 scale pair per column (8 words).
constexpr int kCellBf16 = 0, kCellFp32 = 1, kCellCols = 2;
__host__ __device__ constexpr int cell_words(int cf) { return cf == kCellFp32 ? 4 : cf == kCellCols ? 8 : 2; }
inline int cell_format(const mtc_tile_desc* d) {
  return (d->flags & MTC_FLAG_FP32_SCALES) ? kCellFp32 : (d->flags & MTC_FLAG_COLS_GATHERED) ? kCellCols : kCellBf16;
}
// The kernel of a group or batch whose members have cell formats a and b: bf16-pair and
// gathered-column streams share the kCellCols kernel; fp32-scale streams mix with neither (-1).
inline int joint_cell_format(int a, int b) {
  if (a == b) return a;
  if (a == kCellFp32 || b == kCellFp32) return -1;
  return kCellCols;
}

static_assert(kTN / 4 * (kTK / 8) == kCells, "one cell per (column group, row block)");
static_assert(2 * kProducers == kCells, "two cells per producer thread");

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Byte offset of 16-byte segment `seg` (0..7) of row `row` in a [rows][64] bf16 tile.
// LDS has 64 banks of 4 bytes: a row's 128 bytes fill one half of the banks (by row
// parity), and a 16-lane group of a 128-bit access is conflict-free when its 16
// (row parity, segment) pairs are distinct. The MFMA operand reads take 16 rows at
// one segment, so the segment is XORed with (row & 7) ^ ((row >> 3) & 1): rows r and
// r + 8 share parity and get different segments.
__device__ __forceinline__ uint32_t swz(int row, int seg) {
  return (uint32_t)(row * 128 + ((seg ^ (row & 7) ^ ((row >> 3) & 1)) << 4));
}

// fp32 tiles of the matrix-core fp32 path: [rows][64] floats, 256 bytes (all 64 banks) per row,
// 16-byte segment `seg` (0..15) of row `row` stored at segment seg ^ f(row), f(row) = (row & 15)
// ^ bit 2 of row: the 16 rows that one MFMA operand read takes at one segment land in 16
// different segments (f is a bijection on 0..15), and so do the producers' stores of one column
// of two neighbouring cells (rows n and n + 4, whose f differ in bit 0, at the 8 even or the 8
// odd segments).
constexpr int kTileBytesF32 = kTN * kTK * 4;             // one fp32 B tile (64 KiB)
__device__ __forceinline__ uint32_t swz_f32(int row, int seg) {
  return (uint32_t)(row * 256 + ((seg ^ (row & 15) ^ ((row >> 2) & 1)) << 4));
}

// Hides a value's known bits so byte extraction compiles to v_cvt_f32_ubyteN.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm("" : "+v"(x));
  return x;
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// A buffer resource (base, byte size) for compiler-visible loads: an offset past the end
// reads zeros without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes < 0x7FFFFFFF ? bytes : 0x7FFFFFFF), 0x00020000);
}

// A raw buffer resource (base, byte size) for the DMA copies below.
__device__ __forceinline__ u32x4_t buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  return u32x4_t{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, bytes, 0x00020000u};
}

// Global -> LDS copy of 16 bytes per lane: lane l's bytes land at LDS address lds + 16 l;
// a lane whose offset is past the buffer's end writes zeros. Inline assembly, so the
// compiler neither counts it among its own loads nor makes LDS reads wait for it: the
// consumer waves, which issue no other vector memory loads in their loop, wait for
// these copies with their own counted s_waitcnt.
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rsrc), "s"(lds)
               : "memory");
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS accesses, not for its
// global loads, so the producers' prefetch stays in flight across it (__syncthreads()
// would wait for those loads too and expose their latency every step).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  bf16x2_t p = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, round to nearest even
  return __builtin_bit_cast(uint32_t, p);
}

// Rows 0-3 from the bytes of `top` (scale st, offset term ct), rows 4-7 from `bot`.
__device__ __forceinline__ u32x4_t dec_bytes(uint32_t top, uint32_t bot, float st, float ct, float sb, float cb) {
  u32x4_t r;
  r.x = pk_bf16(__builtin_fmaf((float)(top & 0xFFu), st, ct), __builtin_fmaf((float)((top >> 8) & 0xFFu), st, ct));
  r.y = pk_bf16(__builtin_fmaf((float)((top >> 16) & 0xFFu), st, ct), __builtin_fmaf((float)(top >> 24), st, ct));
  r.z = pk_bf16(__builtin_fmaf((float)(bot & 0xFFu), sb, cb), __builtin_fmaf((float)((bot >> 8) & 0xFFu), sb, cb));
  r.w = pk_bf16(__builtin_fmaf((float)((bot >> 16) & 0xFFu), sb, cb), __builtin_fmaf((float)(bot >> 24), sb, cb));
  return r;
}

__device__ __forceinline__ uint32_t dec_shorts(uint32_t v, float s, float c) {
  return pk_bf16(__builtin_fmaf((float)(v & 0xFFFFu), s, c), __builtin_fmaf((float)(v >> 16), s, c));
}

// The 4 columns (8 rows each, bf16) of one cell from its payload words; column j's top rows
// (0-3) scaled by st[j], its bottom rows by sb[j] (PC: a scale pair per column; otherwise
// st[0], sb[0] for all four). value = (u - offset) * s evaluated as fma(u, s, -offset * s):
// exact in fp32.
template <bool PC>
__device__ __forceinline__ void decode_cell(uint32_t cls, const u32x4_t* pw, const float (&st)[4],
                                            const float (&sb)[4], u32x4_t* out) {
  constexpr int NS = PC ? 4 : 1;
  float ct[NS], cb[NS];
  auto offset_terms = [&](float off) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      ct[j] = -off * st[j];
      cb[j] = -off * sb[j];
    }
  };
  if (cls == 0) {
    offset_terms(8.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = PC ? j : 0;
      const uint32_t x = pw[0][j];
      out[j] = dec_bytes(opaque(x & 0x0F0F0F0Fu), opaque((x >> 4) & 0x0F0F0F0Fu), st[k], ct[k], sb[k], cb[k]);
    }
  } else if (cls == 1) {
    offset_terms(128.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = PC ? j : 0;
      out[j] = dec_bytes(pw[j >> 1][(2 * j) & 3], pw[j >> 1][(2 * j + 1) & 3], st[k], ct[k], sb[k], cb[k]);
    }
  } else if (cls == 2) {
    offset_terms(32768.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = PC ? j : 0;
      out[j].x = dec_shorts(pw[j].x, st[k], ct[k]);
      out[j].y = dec_shorts(pw[j].y, st[k], ct[k]);
      out[j].z = dec_shorts(pw[j].z, sb[k], cb[k]);
      out[j].w = dec_shorts(pw[j].w, sb[k], cb[k]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = u32x4_t{0u, 0u, 0u, 0u};
  }
}

// decode_cell in fp32: out[j][r] = (u - offset) * s for column j, row r (the exact W_hat value,
// fma(u, s, -offset * s), before any bf16 rounding).
template <bool PC>
__device__ __forceinline__ void decode_cell_f32(uint32_t cls, const u32x4_t* pw, const float (&st)[4],
                                                const float (&sb)[4], float (&out)[4][8]) {
  constexpr int NS = PC ? 4 : 1;
  float ct[NS], cb[NS];
  auto offset_terms = [&](float off) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      ct[j] = -off * st[j];
      cb[j] = -off * sb[j];
    }
  };
  // rows 0-3 from the bytes of `top`, rows 4-7 from `bot`
  auto bytes = [&](int j, uint32_t top, uint32_t bot, int k) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      out[j][r] = __builtin_fmaf((float)((top >> (8 * r)) & 0xFFu), st[k], ct[k]);
      out[j][4 + r] = __builtin_fmaf((float)((bot >> (8 * r)) & 0xFFu), sb[k], cb[k]);
    }
  };
  if (cls == 0) {
    offset_terms(8.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = pw[0][j];
      bytes(j, opaque(x & 0x0F0F0F0Fu), opaque((x >> 4) & 0x0F0F0F0Fu), PC ? j : 0);
    }
  } else if (cls == 1) {
    offset_terms(128.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) bytes(j, pw[j >> 1][(2 * j) & 3], pw[j >> 1][(2 * j + 1) & 3], PC ? j : 0);
  } else if (cls == 2) {
    offset_terms(32768.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = PC ? j : 0;
      const uint32_t v[4] = {pw[j].x, pw[j].y, pw[j].z, pw[j].w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float s = h < 2 ? st[k] : sb[k], c = h < 2 ? ct[k] : cb[k];
        out[j][2 * h] = __builtin_fmaf((float)(v[h] & 0xFFFFu), s, c);
        out[j][2 * h + 1] = __builtin_fmaf((float)(v[h] >> 16), s, c);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 8; ++r) out[j][r] = 0.0f;
  }
}

// Output tile (rt, ct) of a launch of one matrix from its block index bx: each XCD (bx % 8)
// takes a contiguous range of tile ids. Without an output column permutation the ids run
// over groups of kRowGroup row tiles, row tile fastest, so the blocks in flight on one XCD
// share column tiles (B) and row tiles (A) in its L2. With one (`row_major`), the ids run
// row-major, so an XCD takes the column tiles of whole row tiles: the scattered 4-byte Y
// writes of an output row then meet in one L2, which merges them into full lines before they
// go to HBM (spread over XCDs they left partial lines: 3.7x the time of plain writes).
// Returns false for a padding block.
__device__ __forceinline__ bool tile_of_block(int bx, int n_row_tiles, int n_ct, int tiles_per_xcd, bool row_major,
                                              int& rt, int& ct) {
  const int tile = (bx % kXcds) * tiles_per_xcd + bx / kXcds;
  if (tile >= n_row_tiles * n_ct) return false;
  if (row_major) {
    rt = tile / n_ct;
    ct = tile - rt * n_ct;
    return true;
  }
  const int per_group = kRowGroup * n_ct;
  const int grp = tile / per_group, in_grp = tile - grp * per_group;
  const int first = grp * kRowGroup;
  const int rows_in = min(n_row_tiles - first, kRowGroup);
  rt = first + in_grp % rows_in;
  ct = in_grp / rows_in;
  return true;
}

// The producer waves of a tile block (pid: 0 .. kProducers-1): load the step's cell descriptors and
// payload, decode the cells of step k+1 into B buffer (k+1) & 1 at bbase (bf16 [256][64] tiles, or
// with F32 fp32 [256][64] tiles in swz_f32 order) while the consumers multiply step k, and
// meet the consumers at one LDS-only barrier per step.
template <int kCF, bool F32>
__device__ __forceinline__ void tile_producers(const mtc_tile_desc& d, const int ct, const int kb0, const int nks,
                                               unsigned char* bbase, const int pid) {
  constexpr int CW = cell_words(kCF);                     // words loaded per cell
  // words per cell of this stream: the kCellCols kernel also runs bf16-pair streams (a group or
  // batch that mixes them with gathered-column ones); their cells are 2 words, and the words a
  // load reads past a cell are not used
  const bool gcols = kCF == kCellCols && (d.flags & MTC_FLAG_COLS_GATHERED) != 0;
  const int cw = kCF == kCellCols && !gcols ? 2 : CW;
  const int p = pid;                                       // 0 .. kProducers-1
  const uint32_t* step_off = d.step_off + (size_t)ct * d.n_ksteps + kb0;
  // cells p and p + kProducers of a step: descriptor words (two sets that swap roles
  // every step, so no register copies wait on loads in flight) and payload words.
  // Every load goes through a buffer resource and every cell issues the same loads
  // (one descriptor load, four 16-byte payload loads; those its class does not need
  // read past the buffer's end and return zeros): with no per-lane branches around
  // loads, the compiler's waits count exactly, so a step waits only for the loads
  // issued a step earlier, never for the ones it has just issued.
  const __amdgpu_buffer_rsrc_t cell_r = buffer_of(d.cells + ((size_t)ct * d.n_ksteps + kb0) * kCells * cw,
                                                  (int64_t)nks * kCells * cw * 4);
  const __amdgpu_buffer_rsrc_t pay_r = buffer_of(d.payload, d.payload_dwords * 4);
  uint32_t sa0[CW], sa1[CW], sb0[CW], sb1[CW];
  uint32_t base_a = 0, base_b = 0;
  u32x4_t q0[4], q1[4];
  auto load_words = [&](uint32_t off, uint32_t (&w)[CW]) __attribute__((always_inline)) {
    if constexpr (CW == 2) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(cell_r, off, 0, 0);
      w[0] = v.x;
      w[1] = v.y;
    } else {
#pragma unroll
      for (int h = 0; h < CW / 4; ++h) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(cell_r, off + 16u * h, 0, 0);
        w[4 * h + 0] = v.x;
        w[4 * h + 1] = v.y;
        w[4 * h + 2] = v.z;
        w[4 * h + 3] = v.w;
      }
    }
  };
  auto load_desc = [&](int ks, uint32_t (&w0)[CW], uint32_t (&w1)[CW], uint32_t& base) {
    load_words((uint32_t)((ks * kCells + p) * cw) * 4u, w0);
    load_words((uint32_t)((ks * kCells + p + kProducers) * cw) * 4u, w1);
    base = step_off[ks];
  };
  auto load_cell = [&](const uint32_t (&w)[CW], uint32_t base, u32x4_t (&q)[4]) {
    const uint32_t cls = (w[0] >> 14) & 3u;
    const uint32_t o = (base + (w[0] & 0x3FFFu)) * 4u;
    const uint32_t n = cls == 0 ? 1u : cls == 1 ? 2u : cls == 2 ? 4u : 0u;
#pragma unroll
    for (uint32_t t = 0; t < 4; ++t)
      q[t] = __builtin_amdgcn_raw_buffer_load_b128(pay_r, t < n ? o + 16u * t : kOutOfRange, 0, 0);
  };
  auto load_payload = [&](const uint32_t (&w0)[CW], const uint32_t (&w1)[CW], uint32_t base) {
    load_cell(w0, base, q0);
    load_cell(w1, base, q1);
  };
  auto stage_cell = [&](unsigned char* bs, const uint32_t (&w)[CW], const u32x4_t (&q)[4]) {
    float st[4], sb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kCF == kCellFp32) {
        st[j] = __uint_as_float(w[1]);
        sb[j] = __uint_as_float(w[2]);
      } else {
        const uint32_t sw = gcols ? w[1 + j] : w[1];          // column j's scales, or the cell's
        st[j] = __uint_as_float(sw << 16);
        sb[j] = __uint_as_float(sw & 0xFFFF0000u);
      }
    }
    const uint32_t pos = w[0] >> 16;
    const int col = (int)(pos >> 3) * 4, seg = (int)(pos & 7u);
    if constexpr (F32) {
      float o[4][8];
      decode_cell_f32<kCF == kCellCols>((w[0] >> 14) & 3u, q, st, sb, o);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = col + j;
        *reinterpret_cast<f32x4_t*>(bs + swz_f32(n, 2 * seg)) = f32x4_t{o[j][0], o[j][1], o[j][2], o[j][3]};
        *reinterpret_cast<f32x4_t*>(bs + swz_f32(n, 2 * seg + 1)) = f32x4_t{o[j][4], o[j][5], o[j][6], o[j][7]};
      }
    } else {
      u32x4_t o[4];
      decode_cell<kCF == kCellCols>((w[0] >> 14) & 3u, q, st, sb, o);
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(bs + swz(col + j, seg)) = o[j];
    }
  };
  auto fill = [&](int buf, const uint32_t (&w0)[CW], const uint32_t (&w1)[CW]) {
    unsigned char* bs = bbase + buf * (F32 ? kTileBytesF32 : kTileBytes);
    stage_cell(bs, w0, q0);
    stage_cell(bs, w1, q1);
  };
  // One step while the consumers multiply step ks: stage step ks+1's B tile (descriptors
  // `cur`, payload already in registers), then load step ks+2's payload (its descriptors
  // `nxt` were loaded a step earlier) and step ks+3's descriptors into `cur`.
  auto step = [&](int ks, uint32_t (&c0)[CW], uint32_t (&c1)[CW], uint32_t& cbase, const uint32_t (&n0)[CW],
                  const uint32_t (&n1)[CW], uint32_t nbase) __attribute__((always_inline)) {
    if (ks + 1 < nks) {
      fill((ks + 1) & 1, c0, c1);
      if (ks + 2 < nks) {
        load_payload(n0, n1, nbase);
        if (ks + 3 < nks) load_desc(ks + 3, c0, c1, cbase);
      }
    }
    lds_barrier();
  };

  // prologue: stage step 0's B tile; hold step 1's payload in registers with its
  // descriptors in set a, and step 2's descriptors in set b
  load_desc(0, sb0, sb1, base_b);
  if (nks > 1) load_desc(1, sa0, sa1, base_a);
  load_payload(sb0, sb1, base_b);
  fill(0, sb0, sb1);
  if (nks > 1) {
    load_payload(sa0, sa1, base_a);
    if (nks > 2) load_desc(2, sb0, sb1, base_b);
  }
  lds_barrier();
  for (int ks = 0; ks < nks; ks += 2) {
    step(ks, sa0, sa1, base_a, sb0, sb1, base_b);
    if (ks + 1 < nks) step(ks + 1, sb0, sb1, base_b, sa0, sa1, base_a);
  }
}

// One output tile block of matrix `d`: output tile (rt, ct), K split by.
// TM: output rows of the block (256, or 128 / 64 for short X, whose full-height tiles are too
// few to fill the chip). The 8 consumer waves are 2 x 4: TM / 2 rows x 64 columns each.
// Xv: bf16 X (copied into LDS as is), or with kXF fp32 X in original row order, which the
// consumers round to bf16 on the way into LDS (tiles of at most 128 rows, whose consumers have
// the registers to hold two steps of X in flight).
template <int kCF, int kYDT, int TM = kTM, bool kXF = false>
__device__ __forceinline__ void gemm_tile_block(const mtc_tile_desc& d, const int rt, const int ct, const int by,
                                                const void* __restrict__ Xv, int64_t ldx, void* __restrict__ Y,
                                                int64_t ldy, int M, int steps_per_split, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  static_assert(TM == 256 || TM == 128 || TM == 64, "row tiles of 256, 128 or 64 rows");
  static_assert(!kXF || TM <= 128, "fp32 X is rounded by the consumers of tiles of at most 128 rows");
  constexpr int DMA = TM / 8 / kConsumerWaves;             // 1 KiB (8-row) A copies per consumer wave
  constexpr int RW = TM / 2, RI = RW / 32;                 // rows per consumer wave, 32-row MFMA blocks

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: keeps per-wave control scalar
  const int m0 = rt * TM, n0 = ct * kTN;
  // split K: this block runs steps kb0 .. kb0 + nks - 1 (split by) and, with `part`,
  // writes its partial tile to part[by] instead of Y
  const int kb0 = by * steps_per_split;
  const int nks = min(steps_per_split, d.n_ksteps - kb0);

  if (wave < kConsumerWaves) {
    // ---------------- consumers: copy X tiles into LDS, bf16 MFMA over the staged tiles ----------------
    // A copies: step s's TM x 64 bf16 X tile is TM / 8 copies of 8 rows; this wave does
    // copies DMA * wave + i. Lane l of a copy fills physical 16-byte slot l of the
    // 8 rows, so it reads the logical segment that swz() maps there. Rows past M and
    // segments past K read zeros (out-of-range offsets).
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
    uint32_t a_off[DMA];                                   // element offset of the lane's segment in the tile
    int a_k[DMA];                                          // first K element of the lane's segment
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
      const int row = 8 * (DMA * wave + i) + (lane >> 3);
      const int lseg = (lane & 7) ^ (row & 7) ^ ((row >> 3) & 1);
      a_k[i] = lseg * 8;
      a_off[i] = m0 + row < M ? (uint32_t)(row * ldx + lseg * 8) : kOutOfRange;
    }
    // K % 8 == 0, so a segment is wholly inside or outside K
    auto a_in = [&](int s, int i) __attribute__((always_inline)) {
      return a_off[i] != kOutOfRange && (kb0 + s) * kTK + a_k[i] < d.K;
    };

    const int wm = wave >> 2, wn = wave & 3;
    f32x16_t acc[RI][2];
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16_t{};
    // the MFMAs of step ks over its staged A and B tiles
    auto mfma_step = [&](int ks) __attribute__((always_inline)) {
      const unsigned char* as = lds + (ks % kABufs) * kTileBytes;
      const unsigned char* bs = lds + (kABufs + (ks & 1)) * kTileBytes;
#pragma unroll
      for (int kk = 0; kk < kTK / 16; ++kk) {
        const int seg = kk * 2 + (lane >> 5);
        bf16x8_t a[RI], b[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          b[j] = *reinterpret_cast<const bf16x8_t*>(bs + swz(wn * 64 + j * 32 + (lane & 31), seg));
#pragma unroll
        for (int i = 0; i < RI; ++i)
          a[i] = *reinterpret_cast<const bf16x8_t*>(as + swz(wm * RW + i * 32 + (lane & 31), seg));
#pragma unroll
        for (int i = 0; i < RI; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    };

    if constexpr (!kXF) {
      const __bf16* X = reinterpret_cast<const __bf16*>(Xv);
      const u32x4_t x_r = buffer_rsrc(X + (int64_t)m0 * ldx, (uint32_t)(TM * ldx * 2));
      auto copy_a = [&](int s) __attribute__((always_inline)) {
        const uint32_t buf = lds0 + (uint32_t)(s % kABufs) * kTileBytes;
        const uint32_t kb = (uint32_t)((kb0 + s) * kTK) * 2;
#pragma unroll
        for (int i = 0; i < DMA; ++i)
          dma16(x_r, a_in(s, i) ? a_off[i] * 2 + kb : kOutOfRange,
                __builtin_amdgcn_readfirstlane(buf + (uint32_t)(DMA * wave + i) * 1024u));
      };
      copy_a(0);
      if (nks > 1) {
        copy_a(1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA) : "memory");   // step 0's copies done
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      lds_barrier();                                       // step 0 staged
      for (int ks = 0; ks < nks; ++ks) {
        const bool ahead = ks + 2 < nks;
        if (ahead) copy_a(ks + 2);                         // into the buffer step ks-1 used
        mfma_step(ks);
        // step ks+1's copies (issued a step ago) must have landed before the barrier
        if (ahead) {
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA) : "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        lds_barrier();                                     // buffers of step ks free, step ks+1 staged
      }
    } else {
      // fp32 X: the lane reads its segment's 8 floats (two 16-byte loads; zeros past M and K),
      // rounds them to bf16 as the staging kernels do (pk_bf16) and stores its slot. Step s + 2's
      // loads go out before step s's MFMAs into the registers step s held; step s + 1's values
      // are stored after them, into the buffer step s - 2 used.
      const float* Xf = reinterpret_cast<const float*>(Xv);
      const __amdgpu_buffer_rsrc_t xf_r = buffer_of(Xf + (int64_t)m0 * ldx, (int64_t)TM * ldx * 4);
      typedef u32x4_t XRegs[DMA][2];
      auto load_x = [&](int s, XRegs& r) __attribute__((always_inline)) {
        const uint32_t kb = (uint32_t)((kb0 + s) * kTK) * 4;
#pragma unroll
        for (int i = 0; i < DMA; ++i) {
          const bool in = a_in(s, i);
          r[i][0] = __builtin_amdgcn_raw_buffer_load_b128(xf_r, in ? a_off[i] * 4 + kb : kOutOfRange, 0, 0);
          r[i][1] = __builtin_amdgcn_raw_buffer_load_b128(xf_r, in ? a_off[i] * 4 + kb + 16 : kOutOfRange, 0, 0);
        }
      };
      auto store_x = [&](int s, const XRegs& r) __attribute__((always_inline)) {
        unsigned char* buf = lds + (s % kABufs) * kTileBytes;
#pragma unroll
        for (int i = 0; i < DMA; ++i) {
          const u32x4_t lo = r[i][0], hi = r[i][1];
          const u32x4_t o{pk_bf16(__uint_as_float(lo.x), __uint_as_float(lo.y)),
                          pk_bf16(__uint_as_float(lo.z), __uint_as_float(lo.w)),
                          pk_bf16(__uint_as_float(hi.x), __uint_as_float(hi.y)),
                          pk_bf16(__uint_as_float(hi.z), __uint_as_float(hi.w))};
          *reinterpret_cast<u32x4_t*>(buf + (DMA * wave + i) * 1024 + 16 * lane) = o;
        }
      };
      XRegs ra, rb;
      load_x(0, ra);
      if (nks > 1) load_x(1, rb);
      store_x(0, ra);
      lds_barrier();                                       // step 0 staged
      // cur: step ks's registers (stored a step ago), nxt: step ks + 1's
      auto body = [&](int ks, XRegs& cur, const XRegs& nxt) __attribute__((always_inline)) {
        if (ks + 2 < nks) load_x(ks + 2, cur);
        mfma_step(ks);
        if (ks + 1 < nks) store_x(ks + 1, nxt);
        lds_barrier();                                     // buffers of step ks free, step ks+1 staged
      };
      for (int ks = 0; ks < nks; ks += 2) {
        body(ks, ra, rb);
        if (ks + 1 < nks) body(ks + 1, rb, ra);
      }
    }

    // epilogue: C element e of lane l is row (e/4)*8 + (l/32)*4 + e%4, column l%32.
    // Split K writes a plain fp32 partial tile to part[by] (no column permutation).
    float* const yf = part ? part + (size_t)by * M * d.N : reinterpret_cast<float*>(Y);
    const int64_t ld = part ? (int64_t)d.N : ldy;
    const bool fp32_out = part || kYDT == MTC_DTYPE_F32;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      const bool cok = col < d.N;
      const int ycol = (d.col_perm && !part) ? d.col_perm[cok ? col : 0] : col;
#pragma unroll
      for (int i = 0; i < RI; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + wm * RW + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          if (cok && row < M) {
            if (fp32_out)
              yf[(int64_t)row * ld + ycol] = acc[i][j][e];
            else
              reinterpret_cast<__bf16*>(Y)[(int64_t)row * ldy + ycol] = (__bf16)acc[i][j][e];
          }
        }
      }
    }
    return;
  }

  tile_producers<kCF, false>(d, ct, kb0, nks, lds + kABufs * kTileBytes, tid - 64 * kConsumerWaves);
}

// One output tile block of matrix `d`: output tile (rt, ct) of TM rows, K split by; X is bf16,
// or fp32 with kXF.
template <int kCF, int kYDT, int TM, bool kXF = false>
__global__ __launch_bounds__(kThreads) void k_gemm_tile(const mtc_tile_desc d, const void* __restrict__ X,
                                                        int64_t ldx, void* __restrict__ Y, int64_t ldy, int M,
                                                        int n_row_tiles, int tiles_per_xcd, int steps_per_split,
                                                        float* __restrict__ part) {
  int rt, ct;
  if (!tile_of_block((int)blockIdx.x, n_row_tiles, d.n_col_tiles, tiles_per_xcd, d.col_perm && !part, rt, ct)) return;
  gemm_tile_block<kCF, kYDT, TM, kXF>(d, rt, ct, (int)blockIdx.y, X, ldx, Y, ldy, M, steps_per_split, part);
}

// ---------------------------------------------------------------------------
// fp32 matrix-core path over the tile stream (mtc_gemm_f32): Y = X * W_hat with fp32 X and
// the exact fp32 W_hat, on v_mfma_f32_16x16x4f32 (fp32 products and sums) - the decode-size
// counterpart of k_gemm_tile for callers that need the fp32 result (M of a few to 16 rows per
// tile). Block = one 16 x 256 output tile, K in steps of 64, the same warp split as k_gemm_tile:
// 4 producer waves decode step k+1's cells into an fp32 B tile ([256][64], swz_f32) while 8
// consumer waves multiply step k; consumer wave w owns output columns 32w .. 32w+31 (two 16 x 16
// MFMA tiles). Waves 0-3 copy the step's X tile ([16][64] fp32, swz_f32; 4 KiB, one 1 KiB copy
// each) straight into LDS two steps ahead. MFMA lane l takes A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16] in register r (checked on the GPU); each
// 16-row group g of a step is 4 MFMAs in which lane quarter q contributes K rows 16g + 4q + s
// (s = 0..3), so one 16-byte LDS read gives a lane its operand for all four.
// ---------------------------------------------------------------------------
constexpr int kFM = 16;                                   // output rows per fp32 tile
constexpr int kABytesF32 = kFM * kTK * 4;                 // one fp32 X tile (4 KiB)
constexpr int kLdsBytesF32 = kABufs * kABytesF32 + kBBufs * kTileBytesF32;   // 140 KiB

template <int kCF>
__device__ __forceinline__ void gemm_f32_block(const mtc_tile_desc& d, const int rt, const int ct, const int by,
                                               const float* __restrict__ X, int64_t ldx, float* __restrict__ Y,
                                               int64_t ldy, int M, int steps_per_split, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = rt * kFM, n0 = ct * kTN;
  const int kb0 = by * steps_per_split;
  const int nks = min(steps_per_split, d.n_ksteps - kb0);
  unsigned char* const bbase = lds + kABufs * kABytesF32;

  if (wave < kConsumerWaves) {
    // X copies: wave w < 4 copies rows 4w .. 4w+3 of each step's tile; lane l fills physical
    // segment l % 16 of row 4w + l / 16, reading the logical segment swz_f32 maps there.
    // Rows past M and segments past K read zeros.
    const bool copies = wave < kFM / 4;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
    const u32x4_t x_r = buffer_rsrc(X + (int64_t)m0 * ldx, (uint32_t)(kFM * ldx * 4));
    const int xrow = 4 * wave + (lane >> 4);
    const int xseg = (lane & 15) ^ (xrow & 15) ^ ((xrow >> 2) & 1);   // logical segment (swz_f32): K 4 xseg .. +3
    const uint32_t x_off = copies && m0 + xrow < M ? (uint32_t)(xrow * ldx + 4 * xseg) * 4 : kOutOfRange;
    auto copy_x = [&](int s) __attribute__((always_inline)) {
      if (!copies) return;
      const bool in = x_off != kOutOfRange && (kb0 + s) * kTK + 4 * xseg < d.K;   // K % 8 == 0
      dma16(x_r, in ? x_off + (uint32_t)((kb0 + s) * kTK) * 4 : kOutOfRange,
            __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(s % kABufs) * kABytesF32 + (uint32_t)wave * 1024u));
    };
    f32x4_t acc[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
    const int r16 = lane & 15, q = lane >> 4;
    copy_x(0);
    if (nks > 1) {
      copy_x(1);
      asm volatile("s_waitcnt vmcnt(1)" ::: "memory");    // step 0's copy done (waves without copies: none)
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    lds_barrier();                                         // step 0 staged
    for (int ks = 0; ks < nks; ++ks) {
      const bool ahead = ks + 2 < nks;
      if (ahead) copy_x(ks + 2);                           // into the buffer step ks-1 used
      const unsigned char* as = lds + (ks % kABufs) * kABytesF32;
      const unsigned char* bs = bbase + (ks & 1) * kTileBytesF32;
      // the step's operands first (12 reads in flight), then its 32 MFMAs
      f32x4_t a[kTK / 16], b[kTK / 16][2];
#pragma unroll
      for (int g = 0; g < kTK / 16; ++g) {
        a[g] = *reinterpret_cast<const f32x4_t*>(as + swz_f32(r16, 4 * g + q));
#pragma unroll
        for (int t = 0; t < 2; ++t)
          b[g][t] = *reinterpret_cast<const f32x4_t*>(bs + swz_f32(32 * wave + 16 * t + r16, 4 * g + q));
      }
#pragma unroll
      for (int g = 0; g < kTK / 16; ++g)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int t = 0; t < 2; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[g][s], b[g][t][s], acc[t], 0, 0, 0);
      if (ahead) {
        asm volatile("s_waitcnt vmcnt(1)" ::: "memory");  // step ks+1's copy (issued a step ago) landed
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      lds_barrier();                                       // buffers of step ks free, step ks+1 staged
    }
    // epilogue: register r of lane l is row 4 (l / 16) + r, column l % 16 of each 16 x 16 tile.
    // Split K writes a plain fp32 partial tile to part[by] (no column permutation).
    float* const yf = part ? part + (size_t)by * M * d.N : Y;
    const int64_t ld = part ? (int64_t)d.N : ldy;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int col = n0 + 32 * wave + 16 * t + r16;
      if (col >= d.N) continue;
      const int ycol = (d.col_perm && !part) ? d.col_perm[col] : col;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 4 * q + r;
        if (row < M) yf[(int64_t)row * ld + ycol] = acc[t][r];
      }
    }
    return;
  }

  tile_producers<kCF, true>(d, ct, kb0, nks, bbase, tid - 64 * kConsumerWaves);
}

template <int kCF>
__global__ __launch_bounds__(kThreads) void k_gemm_f32(const mtc_tile_desc d, const float* __restrict__ X, int64_t ldx,
                                                       float* __restrict__ Y, int64_t ldy, int M, int n_row_tiles,
                                                       int tiles_per_xcd, int steps_per_split,
                                                       float* __restrict__ part) {
  int rt, ct;
  if (!tile_of_block((int)blockIdx.x, n_row_tiles, d.n_col_tiles, tiles_per_xcd, d.col_perm && !part, rt, ct)) return;
  gemm_f32_block<kCF>(d, rt, ct, (int)blockIdx.y, X, ldx, Y, ldy, M, steps_per_split, part);
}

// Xp[m, k] = X[m, row_perm[k]] in fp32 (four outputs per thread), for the fp32 tile path over a
// stream with a row permutation.
__global__ __launch_bounds__(kStageThreads) void k_stage_x_f32(const float* __restrict__ X, int64_t ldx,
                                                               const int32_t* __restrict__ row_perm,
                                                               float* __restrict__ Xp, int K) {
  const int64_t m = blockIdx.y;
  const int k0 = ((int)blockIdx.x * kStageThreads + (int)threadIdx.x) * 4;
  if (k0 >= K) return;
  const int4 src = *reinterpret_cast<const int4*>(row_perm + k0);   // K % 8 == 0, k0 % 4 == 0
  const float* x = X + m * ldx;
  *reinterpret_cast<float4*>(Xp + m * K + k0) = make_float4(x[src.x], x[src.y], x[src.z], x[src.w]);
}

// ---- decode once: W_hat in bf16 (or fp32) for a plain GEMM ----
// One block per (column tile ct, run of `spb` K-steps), grid n_col_tiles x ceil(n_ksteps / spb),
// 256 threads: for each step thread t decodes cells t and t + 256 as the tile kernel's producers
// do (decode_cell: the same bf16 values the MFMAs would read; with F32, decode_cell_f32: the exact
// W_hat) into a swizzled [256][64] LDS tile, then the block writes it out as whole row pieces
// (128 bytes of bf16, 256 of fp32): Wt[n][k] (N rows of ldw elements, ldw = 64 * n_ksteps) holds
// W_hat[k][n] for stream row k (row_perm order, as the staged X) and column n; rows k >= K hold
// the stream's zero padding. While a step is decoded and written, the next step's payload and
// the descriptors of the step after it are in flight. (Stores straight from registers, one cell
// per thread, ran 54 us against 40 us for one step per block at 8192 x 8192 in bf16: a step's
// cells are sorted by class first, so their lines split.)
template <int kCF, bool F32>
__device__ __forceinline__ void tile_dequant_block(const mtc_tile_desc& d, void* __restrict__ Wt, int64_t ldw,
                                                   int spb) {
  __shared__ __attribute__((aligned(16))) unsigned char bs[kTN * kTK * (F32 ? 4 : 2)];
  constexpr int CW = cell_words(kCF);
  const int t = threadIdx.x, ct = blockIdx.x;
  const int ks0 = (int)blockIdx.y * spb, nks = min(spb, d.n_ksteps - ks0);
  const size_t step0 = (size_t)ct * d.n_ksteps + ks0;
  const __amdgpu_buffer_rsrc_t cell_r = buffer_of(d.cells + step0 * kCells * CW, (int64_t)nks * kCells * CW * 4);
  const __amdgpu_buffer_rsrc_t pay_r = buffer_of(d.payload, d.payload_dwords * 4);
  const uint32_t* step_off = d.step_off + step0;
  auto load_desc = [&](int i, uint32_t (&w)[2][CW]) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t off = (uint32_t)((i * kCells + t + 256 * h) * CW) * 4u;
      if constexpr (CW == 2) {
        const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(cell_r, off, 0, 0);
        w[h][0] = v.x;
        w[h][1] = v.y;
      } else {
#pragma unroll
        for (int j = 0; j < CW / 4; ++j) {
          const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(cell_r, off + 16u * j, 0, 0);
          w[h][4 * j + 0] = v.x;
          w[h][4 * j + 1] = v.y;
          w[h][4 * j + 2] = v.z;
          w[h][4 * j + 3] = v.w;
        }
      }
    }
  };
  auto load_payload = [&](uint32_t base, const uint32_t (&w)[2][CW], u32x4_t (&q)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t cls = (w[h][0] >> 14) & 3u;
      const uint32_t o = (base + (w[h][0] & 0x3FFFu)) * 4u;
      const uint32_t n = cls == 0 ? 1u : cls == 1 ? 2u : cls == 2 ? 4u : 0u;
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i)
        q[h][i] = __builtin_amdgcn_raw_buffer_load_b128(pay_r, i < n ? o + 16u * i : kOutOfRange, 0, 0);
    }
  };
  auto decode = [&](const uint32_t (&w)[2][CW], const u32x4_t (&q)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float st[4], sb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (kCF == kCellFp32) {
          st[j] = __uint_as_float(w[h][1]);
          sb[j] = __uint_as_float(w[h][2]);
        } else {
          const uint32_t sw = kCF == kCellCols ? w[h][1 + j] : w[h][1];
          st[j] = __uint_as_float(sw << 16);
          sb[j] = __uint_as_float(sw & 0xFFFF0000u);
        }
      }
      const uint32_t pos = (w[h][0] >> 16) & (kCells - 1);   // (column group, row block) of the cell
      const int col = (int)(pos >> 3) * 4, seg = (int)(pos & 7u);
      if constexpr (F32) {
        float o[4][8];
        decode_cell_f32<kCF == kCellCols>((w[h][0] >> 14) & 3u, q[h], st, sb, o);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          *reinterpret_cast<f32x4_t*>(bs + swz_f32(col + j, 2 * seg)) = f32x4_t{o[j][0], o[j][1], o[j][2], o[j][3]};
          *reinterpret_cast<f32x4_t*>(bs + swz_f32(col + j, 2 * seg + 1)) = f32x4_t{o[j][4], o[j][5], o[j][6], o[j][7]};
        }
      } else {
        u32x4_t o[4];
        decode_cell<kCF == kCellCols>((w[h][0] >> 14) & 3u, q[h], st, sb, o);
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(bs + swz(col + j, seg)) = o[j];
      }
    }
  };
  // 16-byte pieces of the tile's rows: 8 per row in bf16, 16 in fp32
  constexpr int SH = F32 ? 4 : 3, EPP = F32 ? 4 : 8;   // log2 pieces per row, elements per piece
  auto write_out = [&](int ks) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < (kTN << SH) / 256; ++i) {
      const int piece = t + 256 * i, row = piece >> SH, seg = piece & ((1 << SH) - 1);
      const int n = ct * kTN + row;
      if (n < d.N) {
        const int64_t e = (int64_t)n * ldw + (int64_t)ks * kTK + seg * EPP;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(bs + (F32 ? swz_f32(row, seg) : swz(row, seg)));
        *reinterpret_cast<u32x4_t*>(reinterpret_cast<unsigned char*>(Wt) + e * (F32 ? 4 : 2)) = v;
      }
    }
  };
  // step i: descriptors wa, payload qa; step i + 1: descriptors wb, payload qb
  uint32_t wa[2][CW], wb[2][CW];
  u32x4_t qa[2][4], qb[2][4];
  auto body = [&](int i, uint32_t (&wc)[2][CW], u32x4_t (&qc)[2][4], const uint32_t (&wn)[2][CW],
                  u32x4_t (&qn)[2][4]) __attribute__((always_inline)) {
    decode(wc, qc);
    if (i + 1 < nks) load_payload(step_off[i + 1], wn, qn);
    if (i + 2 < nks) load_desc(i + 2, wc);
    lds_barrier();                                     // LDS only: the loads above stay in flight
    write_out(ks0 + i);
    lds_barrier();                                     // the tile is free for the next step
  };
  load_desc(0, wa);
  if (nks > 1) load_desc(1, wb);
  load_payload(step_off[0], wa, qa);
  for (int i = 0; i < nks; i += 2) {
    body(i, wa, qa, wb, qb);
    if (i + 1 < nks) body(i + 1, wb, qb, wa, qa);
  }
}

template <int kCF>
__global__ __launch_bounds__(256) void k_tile_dequant_bf16(const mtc_tile_desc d, __bf16* __restrict__ Wt,
                                                          int64_t ldw, int spb) {
  tile_dequant_block<kCF, false>(d, Wt, ldw, spb);
}

template <int kCF>
__global__ __launch_bounds__(256) void k_tile_dequant_f32(const mtc_tile_desc d, float* __restrict__ Wt,
                                                         int64_t ldw, int spb) {
  tile_dequant_block<kCF, true>(d, Wt, ldw, spb);
}

// Up to kMaxGroup matrices that read the same X, in one launch of each kernel: member i owns
// tile blocks [start[i], start[i + 1]) (whole XCD rounds, so each block runs on the XCD it
// would in a launch of its own) and K splits 0 .. splits[i] - 1 along the grid's y.
constexpr int kMaxGroup = MTC_MAX_GROUP;
struct GemmGroup {
  mtc_tile_desc d[kMaxGroup];
  const __bf16* X[kMaxGroup];
  int64_t ldx[kMaxGroup];
  void* Y[kMaxGroup];
  int64_t ldy[kMaxGroup];
  float* part[kMaxGroup];
  int tiles_per_xcd[kMaxGroup];
  int steps_per_split[kMaxGroup];
  int splits[kMaxGroup];
  int start[kMaxGroup + 1];
};

template <int kCF, int kYDT, int TM>
__global__ __launch_bounds__(kThreads) void k_gemm_tile_group(const GemmGroup g, int M, int n_row_tiles) {
  int i = 0;
#pragma unroll
  for (int k = 1; k < kMaxGroup; ++k) i += (int)blockIdx.x >= g.start[k];
  if ((int)blockIdx.y >= g.splits[i]) return;               // this member has fewer K splits
  int rt, ct;
  if (!tile_of_block((int)blockIdx.x - g.start[i], n_row_tiles, g.d[i].n_col_tiles, g.tiles_per_xcd[i],
                     g.d[i].col_perm && !g.part[i], rt, ct))
    return;
  gemm_tile_block<kCF, kYDT, TM>(g.d[i], rt, ct, (int)blockIdx.y, g.X[i], g.ldx[i], g.Y[i], g.ldy[i], M,
                                 g.steps_per_split[i], g.part[i]);
}

// Xp[m, k] = bf16(X[m, row_perm[k]]) (identity without a permutation); 8 outputs per thread.
__device__ __forceinline__ void stage_x_row(const void* __restrict__ X, int xdt, int64_t ldx,
                                            const int32_t* __restrict__ row_perm, __bf16* __restrict__ Xp, int K) {
  const int64_t m = blockIdx.y;
  const int k0 = ((int)blockIdx.x * kStageThreads + (int)threadIdx.x) * 8;
  if (k0 >= K) return;
  float v[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int src = row_perm ? row_perm[k0 + t] : k0 + t;
    v[t] = xdt == MTC_DTYPE_F32 ? reinterpret_cast<const float*>(X)[m * ldx + src]
                                : (float)reinterpret_cast<const __bf16*>(X)[m * ldx + src];
  }
  u32x4_t o{pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]), pk_bf16(v[4], v[5]), pk_bf16(v[6], v[7])};
  *reinterpret_cast<u32x4_t*>(Xp + m * K + k0) = o;
}

__global__ __launch_bounds__(kStageThreads) void k_stage_x(const void* __restrict__ X, int xdt, int64_t ldx,
                                                           const int32_t* __restrict__ row_perm,
                                                           __bf16* __restrict__ Xp, int K) {
  stage_x_row(X, xdt, ldx, row_perm, Xp, K);
}

// Rows m0 .. m0 + R - 1 of Xp = bf16(X[:, row_perm]) (identity without a permutation),
// R * K bf16 values of LDS: each row is first copied into LDS as bf16 (coalesced reads, the
// same round-to-nearest-even conversion as stage_x_row), then each thread gathers 8 consecutive
// outputs through row_perm from LDS and writes them as one 16-byte store. A gather from global
// memory instead touches a cache line per lane (the permutation scatters a row's columns).
constexpr int kStageLdsMaxBytes = 64 * 1024;
__device__ __forceinline__ void stage_x_rows(const void* __restrict__ X, int xdt, int64_t ldx,
                                             const int32_t* __restrict__ row_perm, __bf16* __restrict__ Xp,
                                             int K, int M, int m0, int R) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];   // [R][K] bf16 bits
  const int tid = threadIdx.x;
  const int rows = min(R, M - m0);
  for (int r = 0; r < rows; ++r) {
    const int64_t base = (int64_t)(m0 + r) * ldx;
    if (xdt == MTC_DTYPE_F32) {
      const float* x = reinterpret_cast<const float*>(X) + base;
      for (int k = tid; k < K; k += kStageThreads) xl[r * K + k] = (uint16_t)pk_bf16(x[k], 0.0f);
    } else {
      const uint16_t* x = reinterpret_cast<const uint16_t*>(X) + base;
      for (int k = tid; k < K; k += kStageThreads) xl[r * K + k] = x[k];
    }
  }
  __syncthreads();
  const int units = K / 8;
  for (int r = 0; r < rows; ++r) {
    const uint16_t* src = xl + r * K;
    __bf16* dst = Xp + (int64_t)(m0 + r) * K;
    for (int u = tid; u < units; u += kStageThreads) {
      const int k0 = 8 * u;
      int4 a = make_int4(k0, k0 + 1, k0 + 2, k0 + 3), b = make_int4(k0 + 4, k0 + 5, k0 + 6, k0 + 7);
      if (row_perm) {
        a = *reinterpret_cast<const int4*>(row_perm + k0);   // 16-byte aligned: k0 % 8 == 0
        b = *reinterpret_cast<const int4*>(row_perm + k0 + 4);
      }
      const u32x4_t o{(uint32_t)src[a.x] | (uint32_t)src[a.y] << 16, (uint32_t)src[a.z] | (uint32_t)src[a.w] << 16,
                      (uint32_t)src[b.x] | (uint32_t)src[b.y] << 16, (uint32_t)src[b.z] | (uint32_t)src[b.w] << 16};
      *reinterpret_cast<u32x4_t*>(dst + k0) = o;
    }
  }
}

// Rows per staging block: up to 4 while R * K bf16 fit kStageLdsMaxBytes and the grid keeps
// at least 1024 blocks; 0 when one row does not fit (the global-gather kernel then stages).
int stage_rows_for(int max_k, int64_t rows_total) {
  if ((int64_t)max_k * 2 > kStageLdsMaxBytes) return 0;
  int r = 1;
  while (r < 4 && (int64_t)2 * r * max_k * 2 <= kStageLdsMaxBytes && rows_total / (2 * r) >= 1024) r *= 2;
  return r;
}

__global__ __launch_bounds__(kStageThreads) void k_stage_x_rows(const void* __restrict__ X, int xdt, int64_t ldx,
                                                                const int32_t* __restrict__ row_perm,
                                                                __bf16* __restrict__ Xp, int K, int M, int R) {
  stage_x_rows(X, xdt, ldx, row_perm, Xp, K, M, (int)blockIdx.x * R, R);
}

// Staging for the members of a group that need it (grid z = entry).
struct StageGroup {
  const int32_t* row_perm[kMaxGroup];
  __bf16* Xp[kMaxGroup];
};

__global__ __launch_bounds__(kStageThreads) void k_stage_x_group(const StageGroup g, const void* __restrict__ X,
                                                                 int xdt, int64_t ldx, int K) {
  stage_x_row(X, xdt, ldx, g.row_perm[blockIdx.z], g.Xp[blockIdx.z], K);
}

// Y[m, col_perm[n]] = sum over splits of part[z][m][n] (fixed order: deterministic), four
// consecutive outputs per thread (N % 4 == 0). Without a column permutation the threads of
// the grid run over the flat M x N range. With one, the writes of a row land all over it, so
// one block takes a whole row: the L2 then merges them into full lines before they leave
// for HBM (blocks that each wrote part of many rows left partly written lines; the c3
// 896 x 4864 gate projection at M = 512 took 5.5 us less with whole rows).
constexpr int kReducePer = 4;
constexpr int kReduceThreads = 256;
__host__ __device__ inline int reduce_blocks(int M, int N, bool col_perm) {
  return col_perm ? M : (int)(((int64_t)M * N / kReducePer + kReduceThreads - 1) / kReduceThreads);
}
template <int kYDT>
__device__ __forceinline__ void splitk_reduce_block(const int b, const float* __restrict__ part, int splits, int M,
                                                    int N, const int32_t* __restrict__ col_perm,
                                                    void* __restrict__ Y, int64_t ldy) {
  if (b >= reduce_blocks(M, N, col_perm != nullptr)) return;
  // whole row b (permuted columns), or the block's slice of the flat range
  const int64_t first = col_perm ? (int64_t)b * N : ((int64_t)b * kReduceThreads + threadIdx.x) * kReducePer;
  const int64_t end = col_perm ? first + N : min(first + kReducePer, (int64_t)M * N);
  const int64_t stride = col_perm ? kReduceThreads * kReducePer : kReducePer;
  for (int64_t i = col_perm ? first + (int64_t)threadIdx.x * kReducePer : first; i < end; i += stride) {
    const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (int z = 0; z < splits; ++z) {
      const float4 p = *reinterpret_cast<const float4*>(part + (size_t)z * M * N + i);
      v.x += p.x;
      v.y += p.y;
      v.z += p.z;
      v.w += p.w;
    }
    const float vs[kReducePer] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int t = 0; t < kReducePer; ++t) {
      const int col = col_perm ? col_perm[n + t] : n + t;
      if (kYDT == MTC_DTYPE_F32)
        reinterpret_cast<float*>(Y)[(int64_t)m * ldy + col] = vs[t];
      else
        reinterpret_cast<__bf16*>(Y)[(int64_t)m * ldy + col] = (__bf16)vs[t];
    }
  }
}

template <int kYDT>
__global__ __launch_bounds__(kReduceThreads) void k_splitk_reduce(const float* __restrict__ part, int splits, int M,
                                                                  int N, const int32_t* __restrict__ col_perm,
                                                                  void* __restrict__ Y, int64_t ldy) {
  splitk_reduce_block<kYDT>((int)blockIdx.x, part, splits, M, N, col_perm, Y, ldy);
}

// The split-K members of a group (grid y = entry).
struct ReduceGroup {
  const float* part[kMaxGroup];
  int splits[kMaxGroup];
  int N[kMaxGroup];
  const int32_t* col_perm[kMaxGroup];
  void* Y[kMaxGroup];
  int64_t ldy[kMaxGroup];
};

template <int kYDT>
__global__ __launch_bounds__(kReduceThreads) void k_splitk_reduce_group(const ReduceGroup g, int M) {
  const int e = blockIdx.y;
  splitk_reduce_block<kYDT>((int)blockIdx.x, g.part[e], g.splits[e], M, g.N[e], g.col_perm[e], g.Y[e], g.ldy[e]);
}

// ---------------------------------------------------------------------------
// Batched prefill: any number of matrices, each with its own X and Y (one M), in one staging
// launch, one tile launch and, for the members whose K is split, one reduction launch. The plan
// (built on the host by mtc_gemm_batch_plan, copied byte for byte to the device by the caller)
// holds one GemmBatchItem per matrix and one entry per grid block: (item, row tile | column
// tile << 12 | K split << 24), or kNoItem where an XCD's list is shorter than the longest.
// ---------------------------------------------------------------------------
struct GemmBatchItem {
  mtc_tile_desc d;
  const void* Xsrc;        // the caller's X
  int64_t ldx_src;
  const __bf16* X;         // what the tile blocks read: the staged bf16 copy, or the caller's bf16 X
  int64_t ldx;
  void* Y;
  int64_t ldy;
  float* part;             // split-K partial tiles (splits > 1)
  int32_t steps_per_split;
  int32_t splits;
  int32_t stage;           // X is staged first (fp32 X, or a row permutation to gather)
  int32_t reserved;
};

constexpr uint32_t kNoItem = 0xFFFFFFFFu;   // a block table entry with no work

template <int kCF, int kYDT, int TM>
__global__ __launch_bounds__(kThreads) void k_gemm_tile_batch(const GemmBatchItem* __restrict__ items,
                                                              const uint2* __restrict__ blocks, int M) {
  const uint2 e = blocks[blockIdx.x];
  if (e.x == kNoItem) return;                               // padding of an XCD's block list
  const GemmBatchItem& it = items[e.x];
  gemm_tile_block<kCF, kYDT, TM>(it.d, (int)(e.y & 0xFFFu), (int)((e.y >> 12) & 0xFFFu), (int)(e.y >> 24), it.X,
                                 it.ldx, it.Y, it.ldy, M, it.steps_per_split, it.splits > 1 ? it.part : nullptr);
}

__global__ __launch_bounds__(kStageThreads) void k_stage_x_batch(const GemmBatchItem* __restrict__ items,
                                                                 const uint32_t* __restrict__ list, int xdt) {
  const GemmBatchItem& it = items[list[blockIdx.z]];
  stage_x_row(it.Xsrc, xdt, it.ldx_src, it.d.row_perm, const_cast<__bf16*>(it.X), it.d.K);
}

// The same through LDS, R rows per block (grid: row groups x members that stage).
__global__ __launch_bounds__(kStageThreads) void k_stage_x_rows_batch(const GemmBatchItem* __restrict__ items,
                                                                      const uint32_t* __restrict__ list, int xdt,
                                                                      int M, int R) {
  const GemmBatchItem& it = items[list[blockIdx.y]];
  stage_x_rows(it.Xsrc, xdt, it.ldx_src, it.d.row_perm, const_cast<__bf16*>(it.X), it.d.K, M, (int)blockIdx.x * R,
               R);
}

template <int kYDT>
__global__ __launch_bounds__(kReduceThreads) void k_splitk_reduce_batch(const GemmBatchItem* __restrict__ items,
                                                                        const uint32_t* __restrict__ list, int M) {
  const GemmBatchItem& it = items[list[blockIdx.y]];
  splitk_reduce_block<kYDT>((int)blockIdx.x, it.part, it.splits, M, it.d.N, it.d.col_perm, it.Y, it.ldy);
}

int check_tile_desc(const mtc_tile_desc* d) {
  if (!d) return fail(MTC_E_NULL, "tile descriptor is NULL");
  if (d->abi_version != MTC_ABI_VERSION)
    return fail(MTC_E_VERSION, "descriptor ABI %u, library ABI %d", d->abi_version, MTC_ABI_VERSION);
  if (d->K <= 0 || d->N <= 0 || d->N % 32 || d->K % 8)
    return fail(MTC_E_DESC, "bad shape K=%d N=%d (N must be a multiple of 32, K of 8)", d->K, d->N);
  if (d->n_ksteps != (d->K + kTK - 1) / kTK || d->n_col_tiles != (d->N + kTN - 1) / kTN)
    return fail(MTC_E_DESC, "n_ksteps=%d n_col_tiles=%d inconsistent with K=%d N=%d", d->n_ksteps, d->n_col_tiles,
                d->K, d->N);
  if (d->flags & ~(MTC_FLAG_FP32_SCALES | MTC_FLAG_COLS_GATHERED)) return fail(MTC_E_DESC, "unknown flags 0x%x", d->flags);
  if ((d->flags & MTC_FLAG_COLS_GATHERED) && ((d->flags & MTC_FLAG_FP32_SCALES) || d->col_perm))
    return fail(MTC_E_DESC, "a gathered-column tile stream has bf16 scales and no col_perm (its columns are in "
                "the original order)");
  if (!d->cells || !d->step_off || !d->payload) return fail(MTC_E_NULL, "tile stream arrays missing");
  if (d->payload_dwords < 4) return fail(MTC_E_DESC, "payload_dwords=%lld", (long long)d->payload_dwords);
  // payload and cells are addressed with 32-bit byte offsets (buffer resources of at most 2 GiB)
  const int64_t cell_bytes = (int64_t)d->n_ksteps * d->n_col_tiles * kCells * 4 * cell_words(cell_format(d));
  if (d->payload_dwords > 0x7FFFFFFF / 4 || cell_bytes > 0x7FFFFFFF)
    return fail(MTC_E_DESC, "tile stream arrays exceed 2 GiB (payload_dwords=%lld, %lld bytes of cells)",
                (long long)d->payload_dwords, (long long)cell_bytes);
  return ok();
}

bool needs_staging(const mtc_tile_desc* d, int x_dtype) { return d->row_perm || x_dtype == MTC_DTYPE_F32; }

constexpr int kFillCUs = 256;             // blocks that fill the chip (one tile block per CU)
constexpr int kMinStepsPerSplit = 2;
constexpr double kReduceBytesPerUs = 4.0e6;   // split-K partials written + read, bytes per microsecond
constexpr double kReduceLaunchUs = 3.0;   // the reduction pass's own launch

// Time of one K-step of a tile block by its row-tile height: 256 rows 1.9-2.4 us. Shorter
// tiles read less X from LDS per step but decode the same 64 x 256 weight cells and keep
// the block's fixed costs; timed at 4096 x 4096, M = 256 with forced plans, relative to 256
// rows: 128 rows 0.79, 64 rows 0.68 (with their fixed costs) of the step time.
inline double step_us(int tm) { return tm == 256 ? 2.0 : tm == 128 ? 1.58 : 1.36; }

struct TilePlan {
  int tm;        // output rows per tile block
  int splits;    // K splits
  int per;       // K-steps per split
};

// Tile height and K split of one call: with M rows in tiles of 256 when those fill the chip;
// otherwise the height (256, or for M <= 256 also 128 or 64) and split count (at most enough
// blocks to fill the chip, at least kMinStepsPerSplit K-steps per split) that minimise the
// estimated time: K-steps per block, rounds of blocks past one per CU, and the split-K
// partial traffic (written by the tile blocks, read by the reduction).
TilePlan tile_plan(const mtc_tile_desc* d, int M) {
  const int64_t full = (int64_t)((M + kTM - 1) / kTM) * d->n_col_tiles;
  if (full >= kFillCUs) return {kTM, 1, d->n_ksteps};
  const double split_bytes = 2.0 * 4.0 * (double)M * d->N;     // one partial, written and read
  TilePlan best{kTM, 1, d->n_ksteps};
  double best_t = 1e300;
  for (int tm : {256, 128, 64}) {
    if (tm < kTM && M > kTM) break;                         // shorter tiles timed for M <= 256 only
    const int64_t n_tiles = (int64_t)((M + tm - 1) / tm) * d->n_col_tiles;
    int max_s = n_tiles >= kFillCUs ? 1 : (int)((kFillCUs + n_tiles - 1) / n_tiles);
    max_s = std::max(1, std::min(max_s, d->n_ksteps / kMinStepsPerSplit));
    for (int s = 1; s <= max_s; ++s) {
      const int per = (d->n_ksteps + s - 1) / s;
      const int s_eff = (d->n_ksteps + per - 1) / per;
      const double rounds = std::ceil((double)(n_tiles * s_eff) / kFillCUs);
      const double t = rounds * per * step_us(tm) +
                       (s_eff > 1 ? s_eff * split_bytes / kReduceBytesPerUs + kReduceLaunchUs : 0.0);
      if (t < best_t) {
        best_t = t;
        best = {tm, s_eff, per};
      }
    }
  }
  return best;
}

// K splits of one call (tile_plan): a group or batch member splits K the same way, so that
// its Y is the single call's bit for bit (the tile height changes no sum). Returns the steps
// per split; `tm`, if given, receives the tile height the single call would use.
int split_steps(const mtc_tile_desc* d, int M, int* splits, int* tm = nullptr) {
  const TilePlan p = tile_plan(d, M);
  *splits = p.splits;
  if (tm) *tm = p.tm;
  return p.per;
}

size_t staging_bytes(const mtc_tile_desc* d, int M, int x_dtype) {
  return needs_staging(d, x_dtype) ? ((size_t)M * d->K * 2 + 255) / 256 * 256 : 0;
}

size_t partial_bytes(const mtc_tile_desc* d, int M) {
  int splits = 1;
  split_steps(d, M, &splits);
  return splits > 1 ? (size_t)splits * M * d->N * 4 : 0;
}

// fp32 X that the tile kernel's consumers round to bf16 themselves, with no staging launch:
// no row permutation, tiles of at most 128 rows, 16-byte aligned rows, and tile offsets within
// 32 bits. The sums are those of the staged call (same bf16 values, same kernel otherwise).
bool fused_x(const mtc_tile_desc* d, const void* X, int x_dtype, int64_t ldx, int M) {
  return x_dtype == MTC_DTYPE_F32 && !d->row_perm && cell_format(d) != kCellCols && tile_plan(d, M).tm <= 128 &&
         ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 && ldx < ((int64_t)1 << 31) / (4 * kTM);
}

template <int kCF, int kYDT>
int launch_tile(const mtc_tile_desc* d, const void* X, int64_t ldx, void* Y, int64_t ldy, int M, float* part,
                hipStream_t st, bool xf = false) {
  if ((size_t)kLdsBytes > mtc::host::device_lds_limit())
    return fail(MTC_E_SHAPE, "prefill kernel needs %d B of LDS per block, device has %zu", kLdsBytes,
                mtc::host::device_lds_limit());
  if (ldx >= ((int64_t)1 << 31) / ((xf ? 4 : 2) * kTM))
    return fail(MTC_E_SHAPE, "ldx=%lld too large for 32-bit X tile offsets", (long long)ldx);
  const TilePlan p = tile_plan(d, M);
  if (xf && p.tm > 128) return fail(MTC_E_SHAPE, "fp32 X is read in place by tiles of at most 128 rows only");
  const void* fn = p.tm == 256 ? reinterpret_cast<const void*>(&k_gemm_tile<kCF, kYDT, 256>)
                   : p.tm == 128 ? reinterpret_cast<const void*>(&k_gemm_tile<kCF, kYDT, 128>)
                                 : reinterpret_cast<const void*>(&k_gemm_tile<kCF, kYDT, 64>);
  if constexpr (kCF != kCellCols) {
    if (xf)
      fn = p.tm == 128 ? reinterpret_cast<const void*>(&k_gemm_tile<kCF, kYDT, 128, true>)
                       : reinterpret_cast<const void*>(&k_gemm_tile<kCF, kYDT, 64, true>);
  } else if (xf) {
    return fail(MTC_E_SHAPE, "fp32 X is not read in place for gathered-column streams");
  }
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  const int n_row_tiles = (M + p.tm - 1) / p.tm;
  const int64_t n_tiles = (int64_t)n_row_tiles * d->n_col_tiles;
  if (n_tiles > (int64_t)1 << 30) return fail(MTC_E_SHAPE, "M=%d gives too many tiles", M);
  const int tiles_per_xcd = (int)((n_tiles + kXcds - 1) / kXcds);
  const int splits = p.splits, per = p.per;
  float* pt = splits > 1 ? part : nullptr;
  int nrt = n_row_tiles, tpx = tiles_per_xcd, spp = per;
  const dim3 grid(tiles_per_xcd * kXcds, splits);
  void* args[] = {const_cast<mtc_tile_desc*>(d), &X, &ldx, &Y, &ldy, &M, &nrt, &tpx, &spp, &pt};
  e = hipLaunchKernel(fn, grid, dim3(kThreads), args, kLdsBytes, st);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "k_gemm_tile launch: %s", hipGetErrorString(e));
  int rc = check_launch("k_gemm_tile");
  if (rc || splits == 1) return rc;
  hipLaunchKernelGGL(k_splitk_reduce<kYDT>, dim3((unsigned)reduce_blocks(M, d->N, d->col_perm != nullptr)),
                     dim3(kReduceThreads), 0, st, part, splits, M, d->N, d->col_perm, Y, ldy);
  return check_launch("k_splitk_reduce");
}

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// X -> bf16 Xp = X[:, row_perm] (M x K, leading dim K) ahead of the tile kernel or the plain GEMM.
int stage_x(const mtc_tile_desc* d, const void* X, int x_dtype, int64_t ldx, int M, __bf16* Xp, hipStream_t st) {
  const int R = stage_rows_for(d->K, M);
  if (R) {
    hipLaunchKernelGGL(k_stage_x_rows, dim3((unsigned)((M + R - 1) / R)), dim3(kStageThreads), (size_t)R * d->K * 2,
                       st, X, x_dtype, ldx, d->row_perm, Xp, d->K, M, R);
  } else {
    dim3 grid((d->K / 8 + kStageThreads - 1) / kStageThreads, M);
    hipLaunchKernelGGL(k_stage_x, grid, dim3(kStageThreads), 0, st, X, x_dtype, ldx, d->row_perm, Xp, d->K);
  }
  return check_launch("k_stage_x");
}

// ---- decode once, then a plain GEMM ----
// A call with at least max(kDecodeOnceMinRows, K / 8) rows of X, at least kDecodeOnceMinMacs
// multiply-adds and no output column permutation: the tile kernel would decode every weight step
// once per row tile (16 times at 4096 rows), so W_hat is decoded once into bf16
// (k_tile_dequant_bf16, the bf16 values the tile kernel's MFMAs read) and multiplied by
// hipBLASLt's bf16 GEMM with fp32 accumulation, X staged as for the tile kernel. (Timed against
// the tile kernel on ten shapes from 896 x 128 to 8192 x 8192: from 512 rows on this path is
// faster where K <= 4864, and with K = 8192 from about 1024 rows; below that the decode, 2 bytes
// written per weight, costs more than it saves, and calls of fewer multiply-adds, such as
// 512 x 896 x 128, are bound by their launches, of which this path has one more.) The
// shape alone makes a call eligible, so workspace sizes never depend on the library; an eligible
// call runs the fused tile kernel when hipBLASLt or an algorithm for its shape is missing, or when
// the path is switched off (mtc_set_prefill_decode_once).
constexpr int kDecodeOnceMinRows = 512;
constexpr int64_t kDecodeOnceMinMacs = (int64_t)1 << 28;   // below: one launch more costs more than it saves
// The GEMM runs without a workspace: the algorithms hipBLASLt picks first for the bf16 shapes timed
// here need none when allowed 32 MiB (and run as fast), and one without a workspace can neither
// leave a memset node in a captured graph nor split K with atomic sums. (Some fp32 shapes' first
// algorithms need one, 896 x 4864 x 1024: 4 MB; with none allowed those calls find no algorithm and
// keep the tile kernel.)
constexpr size_t kBlasWsBytes = 0;
std::atomic<int> g_decode_once{1};

int64_t decode_once_ldw(const mtc_tile_desc* d) { return (int64_t)d->n_ksteps * kTK; }
size_t decode_once_wt_bytes(const mtc_tile_desc* d) { return round256((size_t)d->N * decode_once_ldw(d) * 2); }

bool decode_once_shape(const mtc_tile_desc* d, int M) {
  return !d->col_perm && M >= std::max(kDecodeOnceMinRows, d->K / 8) &&
         (int64_t)M * d->K * d->N >= kDecodeOnceMinMacs;
}

// Workspace of the path: Wt (N x ldw bf16), then the staged X (if any).
size_t decode_once_bytes(const mtc_tile_desc* d, int M, int x_dtype) {
  return decode_once_wt_bytes(d) + round256(staging_bytes(d, M, x_dtype)) + kBlasWsBytes;
}

namespace lt {

struct Api {
  decltype(&hipblasLtCreate) create = nullptr;
  decltype(&hipblasLtMatmulDescCreate) desc_create = nullptr;
  decltype(&hipblasLtMatmulDescSetAttribute) desc_set = nullptr;
  decltype(&hipblasLtMatrixLayoutCreate) layout_create = nullptr;
  decltype(&hipblasLtMatmulPreferenceCreate) pref_create = nullptr;
  decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set = nullptr;
  decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy = nullptr;
  decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic = nullptr;
  decltype(&hipblasLtMatmul) matmul = nullptr;
  bool ok = false;
};

// hipBLASLt, opened on first use: a process that already holds it (a PyTorch process does) shares
// its copy; without it every call takes the fused tile kernel.
const Api& api() {
  static const Api a = [] {
    Api r;
    void* h = nullptr;
    for (const char* name : {"libhipblaslt.so.1", "libhipblaslt.so", "/opt/rocm/lib/libhipblaslt.so.1"})
      if (!h) h = dlopen(name, RTLD_NOW | RTLD_LOCAL);
    if (!h) return r;
    auto sym = [h](auto& f, const char* name) {
      f = reinterpret_cast<std::remove_reference_t<decltype(f)>>(dlsym(h, name));
      return f != nullptr;
    };
    r.ok = sym(r.create, "hipblasLtCreate") && sym(r.desc_create, "hipblasLtMatmulDescCreate") &&
           sym(r.desc_set, "hipblasLtMatmulDescSetAttribute") && sym(r.layout_create, "hipblasLtMatrixLayoutCreate") &&
           sym(r.pref_create, "hipblasLtMatmulPreferenceCreate") &&
           sym(r.pref_set, "hipblasLtMatmulPreferenceSetAttribute") &&
           sym(r.pref_destroy, "hipblasLtMatmulPreferenceDestroy") &&
           sym(r.heuristic, "hipblasLtMatmulAlgoGetHeuristic") && sym(r.matmul, "hipblasLtMatmul");
    return r;
  }();
  return a;
}

// Column-major view of the row-major product: Y^T (N x M, ld ldy) = Wt^T (op T of the K x N,
// ld ldw, array Wt) * Xb^T (K x M, ld ldb, array Xb).
struct Plan {
  hipblasLtHandle_t handle = nullptr;
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;                                   // per device
std::map<std::tuple<int, int, int, int, int, int64_t, int64_t, int64_t, bool>, Plan> g_plans;

// Whether work enqueued on st is being captured into a graph.
bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// The GEMM plan of a shape on the current device, made once (the heuristic's first algorithm
// among those needing at most kBlasWsBytes of workspace, so a shape always runs the same
// algorithm); nullptr when the library or an algorithm is missing. f32: fp32 operands (the
// exact W_hat and fp32 X) instead of bf16 ones. setup: whether the library may be opened and
// the device's handle made here, which allocates; a caller whose stream is being captured passes
// false and gets nullptr (the tile kernel runs) until a call outside a capture has made them.
const Plan* plan_for(int M, int N, int K, int64_t ldw, int64_t ldb, int64_t ldy, int ydt, bool f32, bool setup) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  if (!setup) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto hit = g_handles.find(dev);
    if (hit == g_handles.end() || !hit->second) return nullptr;
  }
  const Api& L = api();
  if (!L.ok) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  const auto key = std::make_tuple(dev, M, N, K, ydt, ldw, ldb, ldy, f32);
  auto it = g_plans.find(key);
  if (it != g_plans.end()) return it->second.ok ? &it->second : nullptr;
  Plan& p = g_plans[key];
  auto hit = g_handles.find(dev);
  if (hit == g_handles.end()) {
    hipblasLtHandle_t h = nullptr;
    if (L.create(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
    hit = g_handles.emplace(dev, h).first;
  }
  if (!hit->second) return nullptr;
  p.handle = hit->second;
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  const hipDataType yt = ydt == MTC_DTYPE_F32 ? HIP_R_32F : HIP_R_16BF;
  if (L.desc_create(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
      L.desc_set(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
      L.desc_set(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS ||
      L.layout_create(&p.a, f32 ? HIP_R_32F : HIP_R_16BF, (uint64_t)K, (uint64_t)N, ldw) != HIPBLAS_STATUS_SUCCESS ||
      L.layout_create(&p.b, f32 ? HIP_R_32F : HIP_R_16BF, (uint64_t)K, (uint64_t)M, ldb) != HIPBLAS_STATUS_SUCCESS ||
      L.layout_create(&p.c, yt, (uint64_t)N, (uint64_t)M, ldy) != HIPBLAS_STATUS_SUCCESS)
    return nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  const uint64_t max_ws = kBlasWsBytes;
  if (L.pref_create(&pref) != HIPBLAS_STATUS_SUCCESS) return nullptr;
  hipblasLtMatmulHeuristicResult_t res[1];
  int got = 0;
  if (L.pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws, sizeof(max_ws)) == HIPBLAS_STATUS_SUCCESS &&
      L.heuristic(p.handle, p.op, p.a, p.b, p.c, p.c, pref, 1, res, &got) == HIPBLAS_STATUS_SUCCESS && got >= 1 &&
      res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= kBlasWsBytes) {
    p.algo = res[0].algo;
    p.ok = true;
  }
  L.pref_destroy(pref);
  return p.ok ? &p : nullptr;
}

int gemm(const Plan* p, const void* Wt, const void* Xb, void* Y, void* ws, hipStream_t st) {
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t s =
      api().matmul(p->handle, p->op, &alpha, Wt, p->a, Xb, p->b, &beta, Y, p->c, Y, p->c, &p->algo, ws, kBlasWsBytes, st);
  if (s != HIPBLAS_STATUS_SUCCESS) return fail(MTC_E_LAUNCH, "hipblasLtMatmul: status %d", (int)s);
  return ok();
}

}  // namespace lt

// The plan of an eligible call, or nullptr for the fused tile kernel (setup: see lt::plan_for).
const lt::Plan* decode_once_plan(const mtc_tile_desc* d, int x_dtype, int64_t ldx, int64_t ldy, int y_dtype, int M,
                                 bool setup) {
  if (!decode_once_shape(d, M) || !g_decode_once.load(std::memory_order_relaxed)) return nullptr;
  return lt::plan_for(M, d->N, d->K, decode_once_ldw(d), needs_staging(d, x_dtype) ? d->K : ldx, ldy, y_dtype, false,
                      setup);
}

// Stage X (if needed), decode W_hat into Wt, run the GEMM; ws holds decode_once_bytes.
int decode_once_call(const mtc_tile_desc* d, const void* X, int x_dtype, int64_t ldx, void* Y, int M, void* ws,
                     const lt::Plan* p, hipStream_t st) {
  char* w = reinterpret_cast<char*>(ws);
  __bf16* const Wt = reinterpret_cast<__bf16*>(w);
  w += decode_once_wt_bytes(d);
  const __bf16* xb = reinterpret_cast<const __bf16*>(X);
  if (needs_staging(d, x_dtype)) {
    const int rc = stage_x(d, X, x_dtype, ldx, M, reinterpret_cast<__bf16*>(w), st);
    if (rc) return rc;
    xb = reinterpret_cast<const __bf16*>(w);
    w += round256(staging_bytes(d, M, x_dtype));
  }
  // K-steps per block: one while there are fewer steps than a wave of resident blocks (five per
  // CU by LDS), up to 8 as the matrix grows (8192 x 8192: 4096 steps, 3 per block)
  const int64_t n_steps = (int64_t)d->n_col_tiles * d->n_ksteps;
  const int spb = (int)std::min<int64_t>(8, std::max<int64_t>(1, n_steps / (5 * kFillCUs)));
  const dim3 grid((unsigned)d->n_col_tiles, (unsigned)((d->n_ksteps + spb - 1) / spb));
  const int64_t ldw = decode_once_ldw(d);
  switch (cell_format(d)) {
    case kCellFp32:
      hipLaunchKernelGGL(k_tile_dequant_bf16<kCellFp32>, grid, dim3(256), 0, st, *d, Wt, ldw, spb);
      break;
    case kCellCols:
      hipLaunchKernelGGL(k_tile_dequant_bf16<kCellCols>, grid, dim3(256), 0, st, *d, Wt, ldw, spb);
      break;
    default:
      hipLaunchKernelGGL(k_tile_dequant_bf16<kCellBf16>, grid, dim3(256), 0, st, *d, Wt, ldw, spb);
  }
  const int rc = check_launch("k_tile_dequant_bf16");
  if (rc) return rc;
  return lt::gemm(p, Wt, xb, Y, w, st);
}

// ---- decode once for fp32 results (mtc_gemm_f32): the exact W_hat in fp32, then hipBLASLt's
// fp32 GEMM (fp32 products and sums, like the tile path), for calls with at least
// kDecodeOnceF32MinRows rows, kDecodeOnceF32MinMacs multiply-adds and no output column
// permutation (an fp32 GEMM of 4096 x 4096 x M took 75 us at M = 256 against 176 us for the fp32
// tile kernel, and 24 against 52 us at M = 64, where writing the 64 MB W_hat costs 20 us more).
constexpr int kDecodeOnceF32MinRows = 256;
constexpr int64_t kDecodeOnceF32MinMacs = (int64_t)1 << 32;

bool decode_once_f32_shape(const mtc_tile_desc* d, int M) {
  return !d->col_perm && M >= kDecodeOnceF32MinRows && (int64_t)M * d->K * d->N >= kDecodeOnceF32MinMacs;
}

// Workspace of the fp32 path: Wt (N x ldw fp32), then X gathered through row_perm (M x K fp32).
size_t decode_once_f32_bytes(const mtc_tile_desc* d, int M) {
  return round256((size_t)d->N * decode_once_ldw(d) * 4) + (d->row_perm ? round256((size_t)M * d->K * 4) : 0);
}

// Workspace of a group: per member, its staged X (if any) then its split-K partials, each on a
// 256-byte boundary; then, when a member is eligible for the decode-once path, one area that the
// eligible members use in turn.
size_t group_ws_bytes(const mtc_tile_desc* const* descs, int n, int M, int x_dtype, size_t* once_off = nullptr) {
  size_t b = 0, once = 0;
  for (int i = 0; i < n; ++i) {
    b += round256(staging_bytes(descs[i], M, x_dtype)) + round256(partial_bytes(descs[i], M));
    if (decode_once_shape(descs[i], M)) once = std::max(once, decode_once_bytes(descs[i], M, x_dtype));
  }
  if (once_off) *once_off = b;
  return b + once;
}

template <int kCF, int kYDT>
int launch_tile_group(GemmGroup& g, int n, int M, int tm, const ReduceGroup& rg, int n_red, hipStream_t st) {
  if ((size_t)kLdsBytes > mtc::host::device_lds_limit())
    return fail(MTC_E_SHAPE, "prefill kernel needs %d B of LDS per block, device has %zu", kLdsBytes,
                mtc::host::device_lds_limit());
  const void* fn = tm == 256 ? reinterpret_cast<const void*>(&k_gemm_tile_group<kCF, kYDT, 256>)
                   : tm == 128 ? reinterpret_cast<const void*>(&k_gemm_tile_group<kCF, kYDT, 128>)
                               : reinterpret_cast<const void*>(&k_gemm_tile_group<kCF, kYDT, 64>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  const int n_row_tiles = (M + tm - 1) / tm;
  int max_splits = 1;
  for (int i = 0; i < n; ++i) max_splits = std::max(max_splits, g.splits[i]);
  const dim3 grid(g.start[n], max_splits);
  if (tm == 256)
    hipLaunchKernelGGL((k_gemm_tile_group<kCF, kYDT, 256>), grid, dim3(kThreads), kLdsBytes, st, g, M, n_row_tiles);
  else if (tm == 128)
    hipLaunchKernelGGL((k_gemm_tile_group<kCF, kYDT, 128>), grid, dim3(kThreads), kLdsBytes, st, g, M, n_row_tiles);
  else
    hipLaunchKernelGGL((k_gemm_tile_group<kCF, kYDT, 64>), grid, dim3(kThreads), kLdsBytes, st, g, M, n_row_tiles);
  int rc = check_launch("k_gemm_tile_group");
  if (rc || n_red == 0) return rc;
  int grid_x = 1;
  for (int i = 0; i < n_red; ++i) grid_x = std::max(grid_x, reduce_blocks(M, rg.N[i], rg.col_perm[i] != nullptr));
  hipLaunchKernelGGL(k_splitk_reduce_group<kYDT>, dim3((unsigned)grid_x, n_red), dim3(kReduceThreads), 0, st, rg, M);
  return check_launch("k_splitk_reduce_group");
}

// ---- batched prefill plan: GemmBatchHeader, GemmBatchItem[n], uint2 blocks[n_blocks], stage list, reduce list ----
struct GemmBatchHeader {
  uint32_t magic;
  uint32_t abi_version;
  int32_t n_items;
  int32_t n_blocks;
  int32_t M;
  int32_t x_dtype;
  int32_t y_dtype;
  int32_t cf;             // cell format of every item (kCellBf16, kCellFp32, kCellCols)
  int32_t n_stage;
  int32_t n_reduce;
  int32_t stage_blocks_x;
  int32_t reduce_blocks_x;
  int32_t stage_rows;     // rows per LDS staging block (0: global gather)
  int32_t stage_max_k;
  int32_t tm;             // output rows per tile block (256, 128 or 64)
  int32_t n_once;         // members on the decode-once path (a batch that does not fill the chip)
  uint64_t once_off;      // their indices (uint32)
  uint64_t once_ws_off;   // their shared workspace area
  uint64_t items_off;
  uint64_t blocks_off;
  uint64_t stage_off;
  uint64_t reduce_off;
  uint64_t plan_bytes;
  uint64_t ws_bytes;
  const void* workspace;
};
constexpr uint32_t kGemmBatchMagic = 0x4D544347u;   // "GCTM"

size_t align64(size_t v) { return (v + 63) / 64 * 64; }

int build_gemm_batch_plan(const mtc_gemm_batch_item* items, int n, int M, int x_dtype, int y_dtype, void* workspace,
                          size_t ws_bytes, void* plan, size_t plan_bytes, size_t* plan_needed, size_t* ws_needed) {
  if (!items) return fail(MTC_E_NULL, "items is NULL");
  if (n < 1 || n > (1 << 16)) return fail(MTC_E_SHAPE, "batch of %d matrices", n);
  if (M <= 0 || M > 65535) return fail(MTC_E_SHAPE, "M=%d must be in [1, 65535]", M);
  if (x_dtype != MTC_DTYPE_F32 && x_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "x_dtype=%d", x_dtype);
  if (y_dtype != MTC_DTYPE_F32 && y_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "y_dtype=%d", y_dtype);
  const int n_row_tiles256 = (M + kTM - 1) / kTM;
  int64_t total_tiles = 0;
  int cf = kCellBf16;
  for (int i = 0; i < n; ++i) {
    const mtc_tile_desc* d = items[i].desc;
    int rc = check_tile_desc(d);
    if (rc) {
      char why[400];
      snprintf(why, sizeof(why), "%s", mtc::host::last_error());
      return fail(rc, "batch item %d: %s", i, why);
    }
    if (!items[i].X || !items[i].Y) return fail(MTC_E_NULL, "batch item %d: X or Y is NULL", i);
    if (items[i].ldx < d->K || items[i].ldy < d->N)
      return fail(MTC_E_SHAPE, "batch item %d: ldx=%lld < K or ldy=%lld < N", i, (long long)items[i].ldx,
                  (long long)items[i].ldy);
    cf = i == 0 ? cell_format(d) : joint_cell_format(cf, cell_format(d));
    if (cf < 0) return fail(MTC_E_SHAPE, "batch item %d differs from the items before it in scale format", i);
    if (!needs_staging(d, x_dtype) && (items[i].ldx % 8 || (reinterpret_cast<uintptr_t>(items[i].X) & 15)))
      return fail(MTC_E_SHAPE, "batch item %d: bf16 X read in place needs 16-byte aligned rows", i);
    const int64_t ldx_used = needs_staging(d, x_dtype) ? d->K : items[i].ldx;
    if (ldx_used >= ((int64_t)1 << 31) / (2 * kTM))
      return fail(MTC_E_SHAPE, "batch item %d: ldx=%lld too large for 32-bit X tile offsets", i, (long long)ldx_used);
    total_tiles += (int64_t)n_row_tiles256 * d->n_col_tiles;
  }
  // the K split of a single call when the batch alone would leave CUs idle; none when it fills them.
  // Tile height: 256 rows when the batch fills the chip, else the shortest any item's single call
  // would use (its split is kept, so its Y stays the single call's bit for bit).
  const bool fill = total_tiles >= kFillCUs;
  // Members that a single call would run on the decode-once path run on it here too, one after
  // another after the tile launches, when the batch does not fill the chip (their Y then stays the
  // single call's); a batch that fills the chip runs every member on the tile kernel.
  std::vector<char> once(n, 0);
  size_t once_ws = 0;
  int n_once = 0;
  if (!fill)
    for (int i = 0; i < n; ++i)
      if (decode_once_plan(items[i].desc, x_dtype, items[i].ldx, items[i].ldy, y_dtype, M, true)) {
        once[i] = 1;
        ++n_once;
        once_ws = std::max(once_ws, decode_once_bytes(items[i].desc, M, x_dtype));
      }
  int tm = kTM;
  if (!fill)
    for (int i = 0; i < n; ++i) {
      if (once[i]) continue;
      int s_i = 1, tm_i = kTM;
      split_steps(items[i].desc, M, &s_i, &tm_i);
      tm = std::min(tm, tm_i);
    }
  const int n_row_tiles = (M + tm - 1) / tm;
  std::vector<int> splits(n), per(n);
  size_t ws = 0;
  int n_stage = 0, n_reduce = 0, stage_bx = 1, reduce_bx = 1;
  // Block placement. Grid block g runs on XCD g % 8, so the table is 8 interleaved lists, one
  // per XCD. Work goes to the lists in groups: the column tiles of one row tile for an unsplit
  // item with an output column permutation (its scattered Y writes of a row then meet in one
  // L2), else the row tiles of one column tile and K split (they share the column tile's
  // weights in L2). Groups go, longest first, to the least loaded list (load = block K-steps);
  // within a list the blocks with the most K-steps come first.
  struct Blk {
    uint32_t item, code;
    int steps;
  };
  struct Group {
    std::vector<Blk> blks;
    int64_t cost;
  };
  std::vector<Group> groups;
  for (int i = 0; i < n; ++i) {
    const mtc_tile_desc* d = items[i].desc;
    if (once[i]) {
      per[i] = splits[i] = 1;
      continue;
    }
    int s = 1;
    per[i] = fill ? d->n_ksteps : split_steps(d, M, &s);
    splits[i] = s;
    if (n_row_tiles >= 4096 || d->n_col_tiles >= 4096 || s > 256)
      return fail(MTC_E_SHAPE, "batch item %d: %d x %d tiles, %d splits exceed the block table fields", i, n_row_tiles,
                  d->n_col_tiles, s);
    const int steps = std::min(per[i], d->n_ksteps);
    auto code = [](int rt, int ct, int by) { return (uint32_t)rt | (uint32_t)ct << 12 | (uint32_t)by << 24; };
    if (d->col_perm && s == 1) {
      for (int rt = 0; rt < n_row_tiles; ++rt) {
        Group g{{}, 0};
        for (int ct = 0; ct < d->n_col_tiles; ++ct) g.blks.push_back({(uint32_t)i, code(rt, ct, 0), steps});
        g.cost = (int64_t)steps * d->n_col_tiles;
        groups.push_back(std::move(g));
      }
    } else {
      for (int by = 0; by < s; ++by)
        for (int ct = 0; ct < d->n_col_tiles; ++ct) {
          Group g{{}, 0};
          const int st = std::min(per[i], d->n_ksteps - by * per[i]);
          for (int rt = 0; rt < n_row_tiles; ++rt) g.blks.push_back({(uint32_t)i, code(rt, ct, by), st});
          g.cost = (int64_t)st * n_row_tiles;
          groups.push_back(std::move(g));
        }
    }
    ws += round256(staging_bytes(d, M, x_dtype)) + round256(s > 1 ? (size_t)s * M * d->N * 4 : 0);
    if (needs_staging(d, x_dtype)) {
      ++n_stage;
      stage_bx = std::max(stage_bx, (d->K / 8 + kStageThreads - 1) / kStageThreads);
    }
    if (s > 1) {
      ++n_reduce;
      reduce_bx = std::max(reduce_bx, reduce_blocks(M, d->N, d->col_perm != nullptr));
    }
  }
  std::stable_sort(groups.begin(), groups.end(), [](const Group& a, const Group& b) { return a.cost > b.cost; });
  std::vector<Blk> lists[kXcds];
  int64_t load[kXcds] = {};
  for (const Group& g : groups) {
    const int x = (int)(std::min_element(load, load + kXcds) - load);
    load[x] += g.cost;
    lists[x].insert(lists[x].end(), g.blks.begin(), g.blks.end());
  }
  size_t longest = 0;
  for (auto& l : lists) {
    std::stable_sort(l.begin(), l.end(), [](const Blk& a, const Blk& b) { return a.steps > b.steps; });
    longest = std::max(longest, l.size());
  }
  const int64_t blocks = (int64_t)longest * kXcds;
  if (blocks > (1 << 30)) return fail(MTC_E_SHAPE, "batch of %lld blocks", (long long)blocks);
  const size_t items_off = align64(sizeof(GemmBatchHeader));
  const size_t blocks_off = align64(items_off + (size_t)n * sizeof(GemmBatchItem));
  const size_t stage_off = align64(blocks_off + (size_t)blocks * sizeof(uint2));
  const size_t reduce_off = align64(stage_off + (size_t)n_stage * sizeof(uint32_t));
  const size_t once_off = align64(reduce_off + (size_t)n_reduce * sizeof(uint32_t));
  const size_t need = once_off + (size_t)n_once * sizeof(uint32_t);
  const size_t once_ws_off = ws;
  ws += once_ws;
  if (plan_needed) *plan_needed = need;
  if (ws_needed) *ws_needed = ws;
  if (!plan) return ok();
  if (plan_bytes < need) return fail(MTC_E_WORKSPACE, "batch plan of %zu bytes needed, %zu given", need, plan_bytes);
  if (reinterpret_cast<uintptr_t>(plan) % 64) return fail(MTC_E_WORKSPACE, "batch plan not 64-byte aligned");
  if (ws && (!workspace || ws_bytes < ws))
    return fail(MTC_E_WORKSPACE, "batch workspace of %zu bytes needed, %zu given", ws, workspace ? ws_bytes : 0);
  if (ws && (reinterpret_cast<uintptr_t>(workspace) & 255)) return fail(MTC_E_WORKSPACE, "workspace not 256-byte aligned");
  unsigned char* base = reinterpret_cast<unsigned char*>(plan);
  memset(base, 0, need);
  GemmBatchHeader* h = reinterpret_cast<GemmBatchHeader*>(base);
  GemmBatchItem* it = reinterpret_cast<GemmBatchItem*>(base + items_off);
  uint2* table = reinterpret_cast<uint2*>(base + blocks_off);
  uint32_t* stage_list = reinterpret_cast<uint32_t*>(base + stage_off);
  uint32_t* reduce_list = reinterpret_cast<uint32_t*>(base + reduce_off);
  uint32_t* once_list = reinterpret_cast<uint32_t*>(base + once_off);
  h->magic = kGemmBatchMagic;
  h->abi_version = MTC_ABI_VERSION;
  h->n_items = n;
  h->n_blocks = (int32_t)blocks;
  h->M = M;
  h->x_dtype = x_dtype;
  h->y_dtype = y_dtype;
  h->cf = cf;
  h->tm = tm;
  h->n_once = n_once;
  h->once_off = once_off;
  h->once_ws_off = once_ws_off;
  h->n_stage = n_stage;
  h->n_reduce = n_reduce;
  h->stage_blocks_x = stage_bx;
  int max_k = 0;
  for (int i = 0; i < n; ++i)
    if (!once[i] && needs_staging(items[i].desc, x_dtype)) max_k = std::max(max_k, items[i].desc->K);
  h->stage_max_k = max_k;
  h->stage_rows = n_stage ? stage_rows_for(max_k, (int64_t)M * n_stage) : 0;
  h->reduce_blocks_x = reduce_bx;
  h->items_off = items_off;
  h->blocks_off = blocks_off;
  h->stage_off = stage_off;
  h->reduce_off = reduce_off;
  h->plan_bytes = need;
  h->ws_bytes = ws;
  h->workspace = workspace;
  char* wsp = reinterpret_cast<char*>(workspace);
  n_stage = n_reduce = n_once = 0;
  for (int i = 0; i < n; ++i) {
    const mtc_tile_desc* d = items[i].desc;
    GemmBatchItem& e = it[i];
    e.d = *d;
    e.Xsrc = items[i].X;
    e.ldx_src = items[i].ldx;
    e.Y = items[i].Y;
    e.ldy = items[i].ldy;
    e.steps_per_split = per[i];
    e.splits = splits[i];
    if (once[i]) {
      e.X = reinterpret_cast<const __bf16*>(items[i].X);
      e.ldx = items[i].ldx;
      once_list[n_once++] = (uint32_t)i;
      continue;
    }
    e.stage = needs_staging(d, x_dtype);
    if (e.stage) {
      e.X = reinterpret_cast<const __bf16*>(wsp);
      e.ldx = d->K;
      wsp += round256(staging_bytes(d, M, x_dtype));
      stage_list[n_stage++] = (uint32_t)i;
    } else {
      e.X = reinterpret_cast<const __bf16*>(items[i].X);
      e.ldx = items[i].ldx;
    }
    if (splits[i] > 1) {
      e.part = reinterpret_cast<float*>(wsp);
      wsp += round256((size_t)splits[i] * M * d->N * 4);
      reduce_list[n_reduce++] = (uint32_t)i;
    }
  }
  for (int x = 0; x < kXcds; ++x)
    for (size_t p = 0; p < longest; ++p)
      table[p * kXcds + x] = p < lists[x].size() ? uint2{lists[x][p].item, lists[x][p].code} : uint2{kNoItem, 0u};
  return ok();
}

template <int kCF, int kYDT>
int launch_tile_batch(const GemmBatchHeader* h, const GemmBatchItem* items, const uint2* blocks,
                      const uint32_t* reduce_list, hipStream_t st) {
  if ((size_t)kLdsBytes > mtc::host::device_lds_limit())
    return fail(MTC_E_SHAPE, "prefill kernel needs %d B of LDS per block, device has %zu", kLdsBytes,
                mtc::host::device_lds_limit());
  const void* fn = h->tm == 256 ? reinterpret_cast<const void*>(&k_gemm_tile_batch<kCF, kYDT, 256>)
                   : h->tm == 128 ? reinterpret_cast<const void*>(&k_gemm_tile_batch<kCF, kYDT, 128>)
                                  : reinterpret_cast<const void*>(&k_gemm_tile_batch<kCF, kYDT, 64>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  const dim3 grid((unsigned)h->n_blocks);
  if (h->tm == 256)
    hipLaunchKernelGGL((k_gemm_tile_batch<kCF, kYDT, 256>), grid, dim3(kThreads), kLdsBytes, st, items, blocks, h->M);
  else if (h->tm == 128)
    hipLaunchKernelGGL((k_gemm_tile_batch<kCF, kYDT, 128>), grid, dim3(kThreads), kLdsBytes, st, items, blocks, h->M);
  else
    hipLaunchKernelGGL((k_gemm_tile_batch<kCF, kYDT, 64>), grid, dim3(kThreads), kLdsBytes, st, items, blocks, h->M);
  int rc = check_launch("k_gemm_tile_batch");
  if (rc || h->n_reduce == 0) return rc;
  hipLaunchKernelGGL(k_splitk_reduce_batch<kYDT>, dim3((unsigned)h->reduce_blocks_x, (unsigned)h->n_reduce),
                     dim3(kReduceThreads), 0, st, items, reduce_list, h->M);
  return check_launch("k_splitk_reduce_batch");
}

int launch_gemm_batch(const void* host_plan, const void* device_plan, hipStream_t st) {
  if (!host_plan || !device_plan) return fail(MTC_E_NULL, "host_plan or device_plan is NULL");
  const GemmBatchHeader* h = reinterpret_cast<const GemmBatchHeader*>(host_plan);
  if (h->magic != kGemmBatchMagic || h->abi_version != MTC_ABI_VERSION)
    return fail(MTC_E_DESC, "not a prefill batch plan of this library (magic 0x%x, ABI %u)", h->magic,
                h->abi_version);
  if (reinterpret_cast<uintptr_t>(device_plan) % 64) return fail(MTC_E_DESC, "device plan not 64-byte aligned");
  const unsigned char* dp = reinterpret_cast<const unsigned char*>(device_plan);
  const GemmBatchItem* items = reinterpret_cast<const GemmBatchItem*>(dp + h->items_off);
  const uint2* blocks = reinterpret_cast<const uint2*>(dp + h->blocks_off);
  const uint32_t* stage_list = reinterpret_cast<const uint32_t*>(dp + h->stage_off);
  const uint32_t* reduce_list = reinterpret_cast<const uint32_t*>(dp + h->reduce_off);
  if (h->n_stage) {
    const int R = h->stage_rows;
    if (R) {
      hipLaunchKernelGGL(k_stage_x_rows_batch, dim3((unsigned)((h->M + R - 1) / R), (unsigned)h->n_stage),
                         dim3(kStageThreads), (size_t)R * h->stage_max_k * 2, st, items, stage_list, h->x_dtype,
                         h->M, R);
    } else {
      hipLaunchKernelGGL(k_stage_x_batch, dim3((unsigned)h->stage_blocks_x, (unsigned)h->M, (unsigned)h->n_stage),
                         dim3(kStageThreads), 0, st, items, stage_list, h->x_dtype);
    }
    const int rc = check_launch("k_stage_x_batch");
    if (rc) return rc;
  }
  const bool f32 = h->y_dtype == MTC_DTYPE_F32;
  int rc = 0;
  if (h->n_blocks) {
    switch (h->cf) {
      case kCellFp32:
        rc = f32 ? launch_tile_batch<kCellFp32, MTC_DTYPE_F32>(h, items, blocks, reduce_list, st)
                 : launch_tile_batch<kCellFp32, MTC_DTYPE_BF16>(h, items, blocks, reduce_list, st);
        break;
      case kCellCols:
        rc = f32 ? launch_tile_batch<kCellCols, MTC_DTYPE_F32>(h, items, blocks, reduce_list, st)
                 : launch_tile_batch<kCellCols, MTC_DTYPE_BF16>(h, items, blocks, reduce_list, st);
        break;
      default:
        rc = f32 ? launch_tile_batch<kCellBf16, MTC_DTYPE_F32>(h, items, blocks, reduce_list, st)
                 : launch_tile_batch<kCellBf16, MTC_DTYPE_BF16>(h, items, blocks, reduce_list, st);
    }
    if (rc) return rc;
  }
  // the decode-once members, from the host copy of the plan
  const unsigned char* hp = reinterpret_cast<const unsigned char*>(host_plan);
  const GemmBatchItem* hitems = reinterpret_cast<const GemmBatchItem*>(hp + h->items_off);
  const uint32_t* once_list = reinterpret_cast<const uint32_t*>(hp + h->once_off);
  for (int j = 0; j < h->n_once && !rc; ++j) {
    // the plan's choice stands (made when it was built; the switch may have changed since)
    const GemmBatchItem& e = hitems[once_list[j]];
    const lt::Plan* p = lt::plan_for(h->M, e.d.N, e.d.K, decode_once_ldw(&e.d),
                                     needs_staging(&e.d, h->x_dtype) ? e.d.K : e.ldx_src, e.ldy, h->y_dtype, false,
                                     !lt::capturing(st));
    if (!p) return fail(MTC_E_LAUNCH, "batch item %u: no GEMM plan for its decode-once path", once_list[j]);
    rc = decode_once_call(&e.d, e.Xsrc, h->x_dtype, e.ldx_src, e.Y, h->M,
                          reinterpret_cast<char*>(const_cast<void*>(h->workspace)) + h->once_ws_off, p, st);
  }
  return rc;
}

}  // namespace

MTC_API int mtc_gemm_batch_plan(const mtc_gemm_batch_item* items, int n, int M, int x_dtype, int y_dtype,
                                void* workspace, size_t workspace_bytes, void* plan, size_t plan_bytes,
                                size_t* plan_needed, size_t* workspace_needed) {
  return build_gemm_batch_plan(items, n, M, x_dtype, y_dtype, workspace, workspace_bytes, plan, plan_bytes,
                               plan_needed, workspace_needed);
}

MTC_API int mtc_gemm_bf16_batch(const void* host_plan, const void* device_plan, void* hip_stream) {
  return launch_gemm_batch(host_plan, device_plan, reinterpret_cast<hipStream_t>(hip_stream));
}

MTC_API int mtc_check_tile_desc(const mtc_tile_desc* d) { return check_tile_desc(d); }

// ---- fp32 tile path (k_gemm_f32) ----
// K splits of an fp32 call: enough (16-row tile, column tile, split) blocks to fill the chip, at
// least kMinStepsPerSplit K-steps each.
struct F32Plan {
  int splits;
  int per;       // K-steps per split
};
F32Plan f32_plan(const mtc_tile_desc* d, int M) {
  const int64_t n_tiles = (int64_t)((M + kFM - 1) / kFM) * d->n_col_tiles;
  int s = n_tiles >= kFillCUs ? 1 : (int)((kFillCUs + n_tiles - 1) / n_tiles);
  s = std::max(1, std::min(s, d->n_ksteps / kMinStepsPerSplit));
  const int per = (d->n_ksteps + s - 1) / s;
  return {(d->n_ksteps + per - 1) / per, per};
}
// Workspace of an fp32 call: X gathered through row_perm (M*K*4, rounded up to 256), then the
// split-K partials (splits*M*N*4).
size_t f32_stage_bytes(const mtc_tile_desc* d, int M) {
  return d->row_perm ? ((size_t)M * d->K * 4 + 255) / 256 * 256 : 0;
}
size_t f32_ws_bytes(const mtc_tile_desc* d, int M) {
  const F32Plan p = f32_plan(d, M);
  return f32_stage_bytes(d, M) + (p.splits > 1 ? (size_t)p.splits * M * d->N * 4 : 0);
}

MTC_API size_t mtc_gemm_f32_workspace_bytes(const mtc_tile_desc* d, int M) {
  if (check_tile_desc(d) || M <= 0) return 0;
  const size_t tiles = f32_ws_bytes(d, M);
  return decode_once_f32_shape(d, M) ? std::max(tiles, decode_once_f32_bytes(d, M)) : tiles;
}

MTC_API int mtc_gemm_f32(const mtc_tile_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                         void* workspace, size_t workspace_bytes, void* hip_stream) {
  int rc = check_tile_desc(d);
  if (rc) return rc;
  if (!X || !Y) return fail(MTC_E_NULL, "X or Y is NULL");
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  if (ldx < d->K || ldy < d->N) return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy=%lld < N", (long long)ldx, (long long)ldy);
  if (!d->row_perm && (ldx % 4 || (reinterpret_cast<uintptr_t>(X) & 15)))
    return fail(MTC_E_SHAPE, "fp32 X read in place needs 16-byte aligned rows (ldx=%lld)", (long long)ldx);
  if (ldx >= ((int64_t)1 << 31) / (4 * kFM))
    return fail(MTC_E_SHAPE, "ldx=%lld too large for 32-bit X tile offsets", (long long)ldx);
  if ((size_t)kLdsBytesF32 > mtc::host::device_lds_limit())
    return fail(MTC_E_SHAPE, "fp32 tile kernel needs %d B of LDS per block, device has %zu", kLdsBytesF32,
                mtc::host::device_lds_limit());
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  const lt::Plan* once = nullptr;
  if (decode_once_f32_shape(d, M) && g_decode_once.load(std::memory_order_relaxed))
    once = lt::plan_for(M, d->N, d->K, decode_once_ldw(d), d->row_perm ? d->K : ldx, ldy, MTC_DTYPE_F32, true,
                        !lt::capturing(st));
  const size_t stage = f32_stage_bytes(d, M), need = once ? decode_once_f32_bytes(d, M) : f32_ws_bytes(d, M);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MTC_E_WORKSPACE, "fp32 tile workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : 0);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MTC_E_WORKSPACE, "workspace not 256-byte aligned");
  const float* xa = X;
  int64_t lda = ldx;
  if (once) {
    // the exact W_hat in fp32, X gathered through row_perm after it, then the fp32 GEMM
    float* const Wt = reinterpret_cast<float*>(workspace);
    const int64_t ldw = decode_once_ldw(d);
    if (d->row_perm) {
      float* xp = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + round256((size_t)d->N * ldw * 4));
      hipLaunchKernelGGL(k_stage_x_f32, dim3((unsigned)((d->K / 4 + kStageThreads - 1) / kStageThreads), (unsigned)M),
                         dim3(kStageThreads), 0, st, X, ldx, d->row_perm, xp, d->K);
      rc = check_launch("k_stage_x_f32");
      if (rc) return rc;
      xa = xp;
      lda = d->K;
    }
    // K-steps per block: two blocks per CU by LDS (a 64 KB fp32 tile)
    const int64_t n_steps = (int64_t)d->n_col_tiles * d->n_ksteps;
    const int spb = (int)std::min<int64_t>(8, std::max<int64_t>(1, n_steps / (2 * kFillCUs)));
    const dim3 grid((unsigned)d->n_col_tiles, (unsigned)((d->n_ksteps + spb - 1) / spb));
    switch (cell_format(d)) {
      case kCellFp32:
        hipLaunchKernelGGL(k_tile_dequant_f32<kCellFp32>, grid, dim3(256), 0, st, *d, Wt, ldw, spb);
        break;
      case kCellCols:
        hipLaunchKernelGGL(k_tile_dequant_f32<kCellCols>, grid, dim3(256), 0, st, *d, Wt, ldw, spb);
        break;
      default:
        hipLaunchKernelGGL(k_tile_dequant_f32<kCellBf16>, grid, dim3(256), 0, st, *d, Wt, ldw, spb);
    }
    rc = check_launch("k_tile_dequant_f32");
    if (rc) return rc;
    return lt::gemm(once, Wt, xa, Y, nullptr, st);
  }
  if (stage) {
    float* xp = reinterpret_cast<float*>(workspace);
    hipLaunchKernelGGL(k_stage_x_f32, dim3((unsigned)((d->K / 4 + kStageThreads - 1) / kStageThreads), (unsigned)M),
                       dim3(kStageThreads), 0, st, X, ldx, d->row_perm, xp, d->K);
    rc = check_launch("k_stage_x_f32");
    if (rc) return rc;
    xa = xp;
    lda = d->K;
  }
  const F32Plan p = f32_plan(d, M);
  float* part = p.splits > 1 ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + stage) : nullptr;
  const int n_row_tiles = (M + kFM - 1) / kFM;
  const int64_t n_tiles = (int64_t)n_row_tiles * d->n_col_tiles;
  if (n_tiles > (int64_t)1 << 30) return fail(MTC_E_SHAPE, "M=%d gives too many tiles", M);
  const int tiles_per_xcd = (int)((n_tiles + kXcds - 1) / kXcds);
  const void* fn = cell_format(d) == kCellFp32   ? reinterpret_cast<const void*>(&k_gemm_f32<kCellFp32>)
                   : cell_format(d) == kCellCols ? reinterpret_cast<const void*>(&k_gemm_f32<kCellCols>)
                                                 : reinterpret_cast<const void*>(&k_gemm_f32<kCellBf16>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytesF32);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  int nrt = n_row_tiles, tpx = tiles_per_xcd, spp = p.per;
  void* args[] = {const_cast<mtc_tile_desc*>(d), &xa, &lda, &Y, &ldy, &M, &nrt, &tpx, &spp, &part};
  e = hipLaunchKernel(fn, dim3(tiles_per_xcd * kXcds, p.splits), dim3(kThreads), args, kLdsBytesF32, st);
  if (e != hipSuccess) return fail(MTC_E_LAUNCH, "k_gemm_f32 launch: %s", hipGetErrorString(e));
  rc = check_launch("k_gemm_f32");
  if (rc || p.splits == 1) return rc;
  hipLaunchKernelGGL(k_splitk_reduce<MTC_DTYPE_F32>, dim3((unsigned)reduce_blocks(M, d->N, d->col_perm != nullptr)),
                     dim3(kReduceThreads), 0, st, part, p.splits, M, d->N, d->col_perm, Y, ldy);
  return check_launch("k_splitk_reduce");
}

MTC_API size_t mtc_gemm_workspace_bytes(const mtc_tile_desc* d, int M, int x_dtype) {
  if (check_tile_desc(d) || M <= 0) return 0;
  const size_t fused = staging_bytes(d, M, x_dtype) + partial_bytes(d, M);
  return decode_once_shape(d, M) ? std::max(fused, decode_once_bytes(d, M, x_dtype)) : fused;
}

MTC_API int mtc_set_prefill_decode_once(int enable) {
  return enable < 0 ? g_decode_once.load() : g_decode_once.exchange(enable ? 1 : 0);
}

MTC_API int mtc_gemm_bf16(const mtc_tile_desc* d, const void* X, int x_dtype, int64_t ldx, void* Y, int y_dtype,
                          int64_t ldy, int M, void* workspace, size_t workspace_bytes, void* hip_stream) {
  int rc = check_tile_desc(d);
  if (rc) return rc;
  if (!X || !Y) return fail(MTC_E_NULL, "X or Y is NULL");
  if (x_dtype != MTC_DTYPE_F32 && x_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "x_dtype=%d", x_dtype);
  if (y_dtype != MTC_DTYPE_F32 && y_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "y_dtype=%d", y_dtype);
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  if (ldx < d->K || ldy < d->N) return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy=%lld < N", (long long)ldx, (long long)ldy);
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  int64_t ldb = ldx;
  const size_t stage = staging_bytes(d, M, x_dtype);
  if (!stage && (ldx % 8 || (reinterpret_cast<uintptr_t>(X) & 15)))
    return fail(MTC_E_SHAPE, "bf16 X read in place needs 16-byte aligned rows (ldx=%lld)", (long long)ldx);
  const lt::Plan* once = decode_once_plan(d, x_dtype, ldx, ldy, y_dtype, M, !lt::capturing(st));
  const size_t need = once ? decode_once_bytes(d, M, x_dtype) : stage + partial_bytes(d, M);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MTC_E_WORKSPACE, "prefill workspace of %zu bytes needed, %zu given", need, workspace ? workspace_bytes : 0);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MTC_E_WORKSPACE, "workspace not 256-byte aligned");
  if (once) return decode_once_call(d, X, x_dtype, ldx, Y, M, workspace, once, st);
  float* part = need > stage ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + stage) : nullptr;
  const void* xa = X;                                  // what the tile kernel reads: X or the staged copy
  const bool xf = fused_x(d, X, x_dtype, ldx, M);      // fp32 X rounded by the tile kernel (staging area unused)
  if (stage && !xf) {
    rc = stage_x(d, X, x_dtype, ldx, M, reinterpret_cast<__bf16*>(workspace), st);
    if (rc) return rc;
    xa = workspace;
    ldb = d->K;
  }
  const bool f32 = y_dtype == MTC_DTYPE_F32;
  switch (cell_format(d)) {
    case kCellFp32:
      return f32 ? launch_tile<kCellFp32, MTC_DTYPE_F32>(d, xa, ldb, Y, ldy, M, part, st, xf)
                 : launch_tile<kCellFp32, MTC_DTYPE_BF16>(d, xa, ldb, Y, ldy, M, part, st, xf);
    case kCellCols:
      return f32 ? launch_tile<kCellCols, MTC_DTYPE_F32>(d, xa, ldb, Y, ldy, M, part, st)
                 : launch_tile<kCellCols, MTC_DTYPE_BF16>(d, xa, ldb, Y, ldy, M, part, st);
    default:
      return f32 ? launch_tile<kCellBf16, MTC_DTYPE_F32>(d, xa, ldb, Y, ldy, M, part, st, xf)
                 : launch_tile<kCellBf16, MTC_DTYPE_BF16>(d, xa, ldb, Y, ldy, M, part, st, xf);
  }
}

MTC_API size_t mtc_gemm_group_workspace_bytes(const mtc_tile_desc* const* descs, int n, int M, int x_dtype) {
  if (!descs || n < 1 || n > kMaxGroup || M <= 0) return 0;
  for (int i = 0; i < n; ++i)
    if (check_tile_desc(descs[i])) return 0;
  return group_ws_bytes(descs, n, M, x_dtype);
}

MTC_API int mtc_gemm_bf16_group(const mtc_tile_desc* const* descs, int n, const void* X, int x_dtype, int64_t ldx,
                                void* const* Y, int y_dtype, const int64_t* ldy, int M, void* workspace,
                                size_t workspace_bytes, void* hip_stream) {
  if (!descs || !Y || !ldy) return fail(MTC_E_NULL, "descs, Y or ldy is NULL");
  if (n < 1 || n > kMaxGroup) return fail(MTC_E_SHAPE, "group of %d matrices (1..%d)", n, kMaxGroup);
  if (!X) return fail(MTC_E_NULL, "X is NULL");
  if (x_dtype != MTC_DTYPE_F32 && x_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "x_dtype=%d", x_dtype);
  if (y_dtype != MTC_DTYPE_F32 && y_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "y_dtype=%d", y_dtype);
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  for (int i = 0; i < n; ++i) {
    const mtc_tile_desc* d = descs[i];
    int rc = check_tile_desc(d);
    if (rc) return rc;
    if (!Y[i]) return fail(MTC_E_NULL, "Y[%d] is NULL", i);
    if (d->K != descs[0]->K) return fail(MTC_E_SHAPE, "group member %d has K=%d, member 0 K=%d", i, d->K, descs[0]->K);
    if ((d->flags & MTC_FLAG_FP32_SCALES) != (descs[0]->flags & MTC_FLAG_FP32_SCALES))
      return fail(MTC_E_SHAPE, "group member %d differs from member 0 in scale format", i);
    if (ldx < d->K || ldy[i] < d->N)
      return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy[%d]=%lld < N", (long long)ldx, i, (long long)ldy[i]);
    if (!needs_staging(d, x_dtype) && (ldx % 8 || (reinterpret_cast<uintptr_t>(X) & 15)))
      return fail(MTC_E_SHAPE, "bf16 X read in place needs 16-byte aligned rows (ldx=%lld)", (long long)ldx);
  }
  size_t once_off = 0;
  const size_t need = group_ws_bytes(descs, n, M, x_dtype, &once_off);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MTC_E_WORKSPACE, "prefill workspace of %zu bytes needed, %zu given", need, workspace ? workspace_bytes : 0);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MTC_E_WORKSPACE, "workspace not 256-byte aligned");
  if (M > (1 << 30)) return fail(MTC_E_SHAPE, "M=%d too large", M);
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  // members that a single call would run on the decode-once path run on it here too, one after
  // another in the area past the fused members' layout; the rest share the fused launches
  const lt::Plan* once[kMaxGroup];
  const bool setup = !lt::capturing(st);
  for (int i = 0; i < n; ++i) once[i] = decode_once_plan(descs[i], x_dtype, ldx, ldy[i], y_dtype, M, setup);
  GemmGroup g;
  StageGroup sg;
  ReduceGroup rg;
  memset(&g, 0, sizeof(g));
  memset(&sg, 0, sizeof(sg));
  memset(&rg, 0, sizeof(rg));
  int n_stage = 0, n_red = 0, blocks = 0, nf = 0, cf = -2;
  char* ws = reinterpret_cast<char*>(workspace);
  // tile height: the shortest any member's single call would use (short X whose 256-row tiles
  // leave CUs idle); every member keeps its own single-call K split
  int tm = kTM;
  for (int i = 0; i < n; ++i) {
    if (once[i]) continue;
    int s_i = 1, tm_i = kTM;
    split_steps(descs[i], M, &s_i, &tm_i);
    tm = std::min(tm, tm_i);
  }
  const int n_row_tiles = (M + tm - 1) / tm;
  for (int i = 0; i < n; ++i) {
    const mtc_tile_desc* d = descs[i];
    const size_t stage = round256(staging_bytes(d, M, x_dtype)), pb = round256(partial_bytes(d, M));
    if (once[i]) {
      ws += stage + pb;
      continue;
    }
    const int j = nf++;
    cf = cf == -2 ? cell_format(d) : joint_cell_format(cf, cell_format(d));
    g.d[j] = *d;
    g.Y[j] = Y[i];
    g.ldy[j] = ldy[i];
    if (stage) {
      sg.row_perm[n_stage] = d->row_perm;
      sg.Xp[n_stage] = reinterpret_cast<__bf16*>(ws);
      ++n_stage;
      g.X[j] = reinterpret_cast<const __bf16*>(ws);
      g.ldx[j] = d->K;
    } else {
      g.X[j] = reinterpret_cast<const __bf16*>(X);
      g.ldx[j] = ldx;
    }
    if (g.ldx[j] >= ((int64_t)1 << 31) / (2 * kTM))
      return fail(MTC_E_SHAPE, "ldx=%lld too large for 32-bit X tile offsets", (long long)g.ldx[j]);
    int splits = 1;
    g.steps_per_split[j] = split_steps(d, M, &splits);
    g.splits[j] = splits;
    g.part[j] = splits > 1 ? reinterpret_cast<float*>(ws + stage) : nullptr;
    if (splits > 1) {
      rg.part[n_red] = g.part[j];
      rg.splits[n_red] = splits;
      rg.N[n_red] = d->N;
      rg.col_perm[n_red] = d->col_perm;
      rg.Y[n_red] = Y[i];
      rg.ldy[n_red] = ldy[i];
      ++n_red;
    }
    ws += stage + pb;
    const int64_t n_tiles = (int64_t)n_row_tiles * d->n_col_tiles;
    g.tiles_per_xcd[j] = (int)((n_tiles + kXcds - 1) / kXcds);
    g.start[j] = blocks;
    blocks += g.tiles_per_xcd[j] * kXcds;
  }
  for (int j = nf; j <= kMaxGroup; ++j) g.start[j] = blocks;
  int rc = 0;
  if (n_stage) {
    dim3 grid((descs[0]->K / 8 + kStageThreads - 1) / kStageThreads, M, n_stage);
    hipLaunchKernelGGL(k_stage_x_group, grid, dim3(kStageThreads), 0, st, sg, X, x_dtype, ldx, descs[0]->K);
    rc = check_launch("k_stage_x_group");
    if (rc) return rc;
  }
  const bool f32 = y_dtype == MTC_DTYPE_F32;
  if (nf) {
    switch (cf) {
      case kCellFp32:
        rc = f32 ? launch_tile_group<kCellFp32, MTC_DTYPE_F32>(g, nf, M, tm, rg, n_red, st)
                 : launch_tile_group<kCellFp32, MTC_DTYPE_BF16>(g, nf, M, tm, rg, n_red, st);
        break;
      case kCellCols:
        rc = f32 ? launch_tile_group<kCellCols, MTC_DTYPE_F32>(g, nf, M, tm, rg, n_red, st)
                 : launch_tile_group<kCellCols, MTC_DTYPE_BF16>(g, nf, M, tm, rg, n_red, st);
        break;
      default:
        rc = f32 ? launch_tile_group<kCellBf16, MTC_DTYPE_F32>(g, nf, M, tm, rg, n_red, st)
                 : launch_tile_group<kCellBf16, MTC_DTYPE_BF16>(g, nf, M, tm, rg, n_red, st);
    }
    if (rc) return rc;
  }
  for (int i = 0; i < n && !rc; ++i)
    if (once[i]) rc = decode_once_call(descs[i], X, x_dtype, ldx, Y[i], M, reinterpret_cast<char*>(workspace) + once_off,
                                       once[i], st);
  return rc;
}
