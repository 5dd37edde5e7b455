// Device-side decoding of the panel stream (layout documented in include/mtc_hip.h).
//
// A lane chunk is 32 offset-binary codes u = q + 2^(P-1) of P bits in P dwords:
// LSB-first for every width but 3; 3-bit codes sit in byte lanes (byte b of the 3
// dwords is a 24-bit string holding codes 8b .. 8b+7, 3 bits each), so one shift
// and mask (two, and an or, where a code crosses a byte) bring a code of every lane
// into its own byte. After full unrolling every bit position is a compile-time
// constant: byte-aligned fields (P = 2, 3, 4 after one mask per 4 or 8 codes, P = 8
// directly) convert with v_cvt_f32_ubyteN, P = 5 and 6 with one v_bfe_u32 (or
// v_alignbit + v_and when a code straddles a dword) and one v_cvt_f32_u32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtc {

constexpr int kPanel = 32;        // output columns per panel (= widest leaf)
constexpr int kCodesPerChunk = 32;
constexpr uint32_t kLeafPad = 1u << 13;   // leaf word flag: padding leaf, contributes nothing
constexpr int kMaxChunkRows = 4096;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t hi16) {
  return __uint_as_float(hi16 << 16);
}

// Round-to-nearest-even float -> bf16 bits (inputs are finite).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// NT = true streams the payload past the caches (read once per call, GEMV);
// NT = false keeps it cacheable (re-read by every M tile, GEMM).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <int P, bool NT>
__device__ __forceinline__ void load_chunk(const uint32_t* __restrict__ src, uint32_t (&w)[P]) {
  if constexpr (P % 4 == 0) {
    const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(src);
#pragma unroll
    for (int i = 0; i < P / 4; ++i) {
      u32x4_t v;
      if constexpr (NT) v = __builtin_nontemporal_load(s4 + i); else v = s4[i];
      w[4 * i + 0] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (P == 2) {
    const u32x2_t* s2 = reinterpret_cast<const u32x2_t*>(src);
    u32x2_t v;
    if constexpr (NT) v = __builtin_nontemporal_load(s2); else v = *s2;
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if constexpr (NT) w[i] = __builtin_nontemporal_load(src + i); else w[i] = src[i];
    }
  }
}

// P dwords of a chunk staged in LDS (16-byte aligned when P % 4 == 0, 8-byte when P == 2).
template <int P>
__device__ __forceinline__ void lds_chunk(const uint32_t* src, uint32_t (&w)[P]) {
  if constexpr (P % 4 == 0) {
#pragma unroll
    for (int i = 0; i < P / 4; ++i) {
      const u32x4_t v = reinterpret_cast<const u32x4_t*>(src)[i];
      w[4 * i + 0] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (P == 2) {
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(src);
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < P; ++i) w[i] = src[i];
  }
}

// Hides a value's known bits so byte extraction compiles to v_cvt_f32_ubyteN.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm("" : "+v"(x));
  return x;
}

__device__ __forceinline__ float ubyte(uint32_t x, int k) { return (float)((x >> (8 * k)) & 0xFFu); }

// Offset-binary code i (0..31) of a chunk (LSB-first widths, P != 3).
template <int P>
__device__ __forceinline__ uint32_t chunk_ucode(const uint32_t (&w)[P], int i) {
  const int b = i * P, j = b >> 5, o = b & 31;
  if (o + P <= 32) return (w[j] >> o) & ((1u << P) - 1u);
  return __builtin_amdgcn_alignbit(w[(j + 1) < P ? (j + 1) : j], w[j], o) & ((1u << P) - 1u);
}

// The 32 offset-binary codes of a chunk as floats (exact), in code order.
template <int P>
__device__ __forceinline__ void decode_chunk_u(const uint32_t (&w)[P], float (&u)[32]) {
  if constexpr (P == 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) u[4 * j + k] = ubyte(w[j], k);
  } else if constexpr (P == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = opaque(w[j] & 0x0F0F0F0Fu), hi = opaque((w[j] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        u[8 * j + 2 * k] = ubyte(lo, k);
        u[8 * j + 2 * k + 1] = ubyte(hi, k);
      }
    }
  } else if constexpr (P == 2) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t f = opaque((w[j] >> (2 * s)) & 0x03030303u);
#pragma unroll
        for (int k = 0; k < 4; ++k) u[16 * j + 4 * k + s] = ubyte(f, k);
      }
  } else if constexpr (P == 3) {
    // byte k of f[a] is code 8k + a (bits 3a .. 3a+2 of byte lane k)
    uint32_t f[8];
    f[0] = w[0] & 0x07070707u;
    f[1] = (w[0] >> 3) & 0x07070707u;
    f[2] = ((w[0] >> 6) & 0x03030303u) | ((w[1] << 2) & 0x04040404u);
    f[3] = (w[1] >> 1) & 0x07070707u;
    f[4] = (w[1] >> 4) & 0x07070707u;
    f[5] = ((w[1] >> 7) & 0x01010101u) | ((w[2] << 1) & 0x06060606u);
    f[6] = (w[2] >> 2) & 0x07070707u;
    f[7] = (w[2] >> 5) & 0x07070707u;
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const uint32_t v = opaque(f[a]);
#pragma unroll
      for (int k = 0; k < 4; ++k) u[8 * k + a] = ubyte(v, k);
    }
  } else if constexpr (P == 16) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      u[2 * j] = (float)(w[j] & 0xFFFFu);
      u[2 * j + 1] = (float)(w[j] >> 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) u[i] = (float)chunk_ucode<P>(w, i);
  }
}

// Signed codes q = u - 2^(P-1) as floats (exact).
template <int P>
__device__ __forceinline__ void decode_chunk(const uint32_t (&w)[P], float (&q)[32]) {
  decode_chunk_u<P>(w, q);
#pragma unroll
  for (int i = 0; i < 32; ++i) q[i] -= (float)(1 << (P - 1));
}

struct LeafInfo {
  int row;    // first row within the unit
  bool pad;
  float scale;
};

__device__ __forceinline__ LeafInfo leaf_info(uint32_t word, const float* __restrict__ fscale, uint32_t leaf) {
  LeafInfo li;
  li.row = static_cast<int>(word & 0x3FFu) * 4;
  li.pad = (word & kLeafPad) != 0;
  li.scale = fscale ? fscale[leaf] : bf16_bits_to_f32(word >> 16);
  return li;
}

// Leaf fields with the fp32 scale (if any) already loaded.
__device__ __forceinline__ LeafInfo leaf_info_v(uint32_t word, bool fp32_scales, float fscale) {
  LeafInfo li;
  li.row = static_cast<int>(word & 0x3FFu) * 4;
  li.pad = (word & kLeafPad) != 0;
  li.scale = fp32_scales ? fscale : bf16_bits_to_f32(word >> 16);
  return li;
}

constexpr int kGroup = 4;             // columns per column group
constexpr int kGroups = kPanel / kGroup;
constexpr int kUnitHdr = 32;          // words per unit header

}  // namespace mtc

// Expands F(S, P) for every supported bucket kind; used to build switch tables.
#define MTC_FOR_EACH_BUCKET(F) \
  F(32, 2) F(32, 3) F(32, 4) F(32, 5) F(32, 6) F(32, 8) F(32, 16) \
  F(16, 2) F(16, 3) F(16, 4) F(16, 5) F(16, 6) F(16, 8) F(16, 16) \
  F(8, 2) F(8, 3) F(8, 4) F(8, 5) F(8, 6) F(8, 8) F(8, 16) \
  F(4, 2) F(4, 3) F(4, 4) F(4, 5) F(4, 6) F(4, 8) F(4, 16)

// Expands F(S, P) for every code width at one leaf size.
#define MTC_FOR_EACH_WIDTH(S, F) F(S, 2) F(S, 3) F(S, 4) F(S, 5) F(S, 6) F(S, 8) F(S, 16)

#define MTC_LOG2_SIZE(S) ((S) == 32 ? 5 : (S) == 16 ? 4 : (S) == 8 ? 3 : 2)
#define MTC_BUCKET_KEY(S, P) (MTC_LOG2_SIZE(S) | ((P) << 8))
