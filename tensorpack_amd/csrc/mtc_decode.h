// Device-side decoding of the panel stream (layout documented in include/mtc_hip.h).
//
// A lane chunk is 32 two's-complement codes of P bits packed LSB-first into P
// dwords. After full unrolling every bit position is a compile-time constant,
// so each code costs one v_bfe_i32 (or v_alignbit + v_bfe_i32 when it
// straddles a dword) and one v_cvt_f32_i32.
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

// Signed code i (0..31) of a chunk.
template <int P>
__device__ __forceinline__ int chunk_code(const uint32_t (&w)[P], int i) {
  const int b = i * P, j = b >> 5, o = b & 31;
  if (o + P <= 32) return static_cast<int>(w[j] << (32 - o - P)) >> (32 - P);
  const uint32_t v = __builtin_amdgcn_alignbit(w[(j + 1) < P ? (j + 1) : j], w[j], o);
  return static_cast<int>(v << (32 - P)) >> (32 - P);
}

template <int P>
__device__ __forceinline__ void decode_chunk(const uint32_t (&w)[P], float (&q)[32]) {
#pragma unroll
  for (int i = 0; i < 32; ++i) q[i] = static_cast<float>(chunk_code<P>(w, i));
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

#define MTC_LOG2_SIZE(S) ((S) == 32 ? 5 : (S) == 16 ? 4 : (S) == 8 ? 3 : 2)
#define MTC_BUCKET_KEY(S, P) (MTC_LOG2_SIZE(S) | ((P) << 8))
