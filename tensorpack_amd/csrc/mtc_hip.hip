// gfx950 kernels and C-ABI for Y = X * W_hat over the panel stream.
//
//   k_fill_zero     : zero an fp32 buffer (used before dequant; no memset nodes)
//   k_dequant       : stream -> dense W_hat (bit-exact q*s, +0.0 for P0)
//   k_gemv<MT>      : fp32 decode path, MT rows of X per block, split-K over
//                     chunks with a deterministic last-block reduction
//   k_gemm_bf16     : prefill path, leaves dequantized to bf16 tiles in LDS,
//                     v_mfma_f32_32x32x16_bf16 with fp32 accumulation
//
// Reference behaviour: mtc/kernels/gemm.py:124-210 (block loop: skip P0
// blocks, unpack codes, scale, fp32 multiply-accumulate) for a dense X and a
// quadtree weight; W_hat as defined by mtc/core/quadtree.py:157-171.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>

#include "mtc_hip.h"
#include "mtc_decode.h"

using namespace mtc;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

#define MTC_API extern "C" __attribute__((visibility("default")))

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
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

// ---------------------------------------------------------------------------
// zero fill
// ---------------------------------------------------------------------------
__global__ void k_fill_zero(float* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// dequant: one block per unit, every lane decodes whole chunks
// ---------------------------------------------------------------------------
template <int S, int P>
__device__ __forceinline__ void dequant_bucket(const mtc_stream_desc& d, const uint32_t* bk, int panel, int kb,
                                               float* __restrict__ W) {
  using Geo = ChunkGeom<S>;
  const uint32_t* payload = d.payload + bk[0];
  const uint32_t l0 = bk[1], n = bk[2];
  for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
    uint32_t w[P];
    load_chunk<P, true>(payload + (size_t)t * P, w);
    float q[32];
    decode_chunk<P>(w, q);
#pragma unroll
    for (int g = 0; g < Geo::G; ++g) {
      uint32_t leaf;
      int cin;
      if constexpr (S == 4) {
        leaf = l0 + 2 * t + (g >> 2);
        cin = g & 3;
      } else {
        leaf = l0 + t / Geo::chunks_per_leaf;
        cin = (int)(t % Geo::chunks_per_leaf) * Geo::G + g;
      }
      const LeafInfo li = leaf_info(d.leaf_word[leaf], d.leaf_scale, leaf);
      if (li.pad) continue;
      int col = panel * kPanel + li.col + cin;
      if (d.col_perm) col = d.col_perm[col];
#pragma unroll
      for (int r = 0; r < Geo::R; ++r) {
        int k = kb + li.row + r;
        if (d.row_perm) k = d.row_perm[k];
        float v = q[g * Geo::R + r] * li.scale;
        // quadtree W_hat is summed into a +0.0 buffer (no -0.0); the uniform-block
        // arena rebuild assigns q*s as is
        if (!d.leaf_scale) v += 0.0f;
        W[(int64_t)k * d.N + col] = v;
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_dequant(const mtc_stream_desc d, float* __restrict__ W) {
  const int u = blockIdx.x;
  const int panel = u / d.n_chunks, chunk = u - panel * d.n_chunks;
  const int kb = chunk * d.chunk_rows;
  const int b0 = d.unit_buckets[u], b1 = d.unit_buckets[u + 1];
  for (int b = b0; b < b1; ++b) {
    const uint32_t* bk = d.buckets + 4 * b;
    switch (bk[3]) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): dequant_bucket<S, P>(d, bk, panel, kb, W); break;
      MTC_FOR_EACH_BUCKET(MTC_CASE)
#undef MTC_CASE
      default: break;
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 GEMV
// ---------------------------------------------------------------------------
template <int R>
__device__ __forceinline__ float dot_rows(const float* __restrict__ x, const float* q) {
  // x is 16-byte aligned (leaf rows start at multiples of 4)
  float s = 0.0f;
  if constexpr (R >= 4) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
#pragma unroll
    for (int i = 0; i < R / 4; ++i) {
      const float4 v = x4[i];
      s += v.x * q[4 * i + 0];
      s += v.y * q[4 * i + 1];
      s += v.z * q[4 * i + 2];
      s += v.w * q[4 * i + 3];
    }
  }
  return s;
}

template <int S, int P, int MT>
__device__ __forceinline__ void gemv_bucket(const mtc_stream_desc& d, const uint32_t* bk, const float* xs, int xs_stride,
                                            float* wacc) {
  using Geo = ChunkGeom<S>;
  const uint32_t* payload = d.payload + bk[0];
  const uint32_t l0 = bk[1], n = bk[2];
  for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
    uint32_t w[P];
    load_chunk<P, true>(payload + (size_t)t * P, w);
    float q[32];
    decode_chunk<P>(w, q);
    if constexpr (S == 4) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t leaf = l0 + 2 * t + h;
        const LeafInfo li = leaf_info(d.leaf_word[leaf], d.leaf_scale, leaf);
        if (li.pad) continue;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float* xr = xs + m * xs_stride + li.row;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float part = dot_rows<4>(xr, q + (4 * h + g) * 4);
            atomicAdd(&wacc[m * kPanel + li.col + g], part * li.scale);
          }
        }
      }
    } else {
      const uint32_t leaf = l0 + t / Geo::chunks_per_leaf;
      const int cbase = (int)(t % Geo::chunks_per_leaf) * Geo::G;
      const LeafInfo li = leaf_info(d.leaf_word[leaf], d.leaf_scale, leaf);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float* xr = xs + m * xs_stride + li.row;
#pragma unroll
        for (int g = 0; g < Geo::G; ++g) {
          const float part = dot_rows<Geo::R>(xr, q + g * Geo::R);
          atomicAdd(&wacc[m * kPanel + li.col + cbase + g], part * li.scale);
        }
      }
    }
  }
}

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;

template <int MT>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(const mtc_stream_desc d, const float* __restrict__ X, int64_t ldx,
                                                      float* __restrict__ Y, int64_t ldy, int M,
                                                      float* __restrict__ part, uint32_t* __restrict__ counters) {
  extern __shared__ float smem[];
  const int kc = d.chunk_rows;
  float* xs = smem;                       // [MT][kc]
  float* acc = smem + MT * kc;            // [waves][MT][32]
  const int tid = threadIdx.x;
  const int u = blockIdx.x, mt = blockIdx.y;
  const int n_units = d.n_panels * d.n_chunks;
  const int panel = u / d.n_chunks, chunk = u - panel * d.n_chunks;
  const int m0 = mt * MT;
  const int kb = chunk * kc;
  const int rows = min(kc, d.K - kb);

  for (int m = 0; m < MT; ++m) {
    const bool live = m0 + m < M;
    const float* xrow = X + (int64_t)(m0 + m) * ldx;
    for (int r = tid; r < kc; r += kGemvThreads) {
      float v = 0.0f;
      if (live && r < rows) {
        int k = kb + r;
        if (d.row_perm) k = d.row_perm[k];
        v = xrow[k];
      }
      xs[m * kc + r] = v;
    }
  }
  for (int i = tid; i < kGemvWaves * MT * kPanel; i += kGemvThreads) acc[i] = 0.0f;
  __syncthreads();

  float* wacc = acc + (tid >> 6) * MT * kPanel;
  const int b0 = d.unit_buckets[u], b1 = d.unit_buckets[u + 1];
  for (int b = b0; b < b1; ++b) {
    const uint32_t* bk = d.buckets + 4 * b;
    switch (bk[3]) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): gemv_bucket<S, P, MT>(d, bk, xs, kc, wacc); break;
      MTC_FOR_EACH_BUCKET(MTC_CASE)
#undef MTC_CASE
      default: break;
    }
  }
  __syncthreads();

  constexpr int n_out = MT * kPanel;
  if (d.n_chunks == 1) {
    for (int i = tid; i < n_out; i += kGemvThreads) {
      float v = acc[i];
#pragma unroll
      for (int wv = 1; wv < kGemvWaves; ++wv) v += acc[wv * n_out + i];
      const int m = i / kPanel, c = i % kPanel;
      if (m0 + m < M) {
        int col = panel * kPanel + c;
        if (d.col_perm) col = d.col_perm[col];
        Y[(int64_t)(m0 + m) * ldy + col] = v;
      }
    }
    return;
  }

  float* mine = part + ((size_t)mt * n_units + u) * n_out;
  for (int i = tid; i < n_out; i += kGemvThreads) {
    float v = acc[i];
#pragma unroll
    for (int wv = 1; wv < kGemvWaves; ++wv) v += acc[wv * n_out + i];
    __hip_atomic_store(mine + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __threadfence();
  __syncthreads();
  __shared__ int last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[mt * d.n_panels + panel], 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last = (prev == (uint32_t)(d.n_chunks - 1));
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  const float* pp = part + ((size_t)mt * n_units + (size_t)panel * d.n_chunks) * n_out;
  for (int i = tid; i < n_out; i += kGemvThreads) {
    float v = 0.0f;
    for (int c = 0; c < d.n_chunks; ++c)
      v += __hip_atomic_load(pp + (size_t)c * n_out + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int m = i / kPanel, cc = i % kPanel;
    if (m0 + m < M) {
      int col = panel * kPanel + cc;
      if (d.col_perm) col = d.col_perm[col];
      Y[(int64_t)(m0 + m) * ldy + col] = v;
    }
  }
  if (tid == 0)
    __hip_atomic_store(&counters[mt * d.n_panels + panel], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// bf16 MFMA GEMM (prefill)
// ---------------------------------------------------------------------------
constexpr int kGBM = 128;              // rows of X per block
constexpr int kGBN = 128;              // output columns per block (4 panels)
constexpr int kGBK = 64;               // reduction rows per step (= stream chunk_rows)
constexpr int kGLds = kGBK + 8;        // bf16 elements per LDS row (padded)

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// Write R consecutive-k bf16 values q[0..R) * scale at LDS row `dst` (k-contiguous).
template <int R>
__device__ __forceinline__ void store_bf16_run(uint16_t* dst, const float* q, float scale) {
  if constexpr (R >= 8) {
#pragma unroll
    for (int i = 0; i < R / 8; ++i) {
      uint4 v;
      v.x = pack_bf16x2(q[8 * i + 0] * scale, q[8 * i + 1] * scale);
      v.y = pack_bf16x2(q[8 * i + 2] * scale, q[8 * i + 3] * scale);
      v.z = pack_bf16x2(q[8 * i + 4] * scale, q[8 * i + 5] * scale);
      v.w = pack_bf16x2(q[8 * i + 6] * scale, q[8 * i + 7] * scale);
      reinterpret_cast<uint4*>(dst)[i] = v;
    }
  } else {
    uint2 v;
    v.x = pack_bf16x2(q[0] * scale, q[1] * scale);
    v.y = pack_bf16x2(q[2] * scale, q[3] * scale);
    *reinterpret_cast<uint2*>(dst) = v;
  }
}

template <int S, int P>
__device__ __forceinline__ void gemm_bucket(const mtc_stream_desc& d, const uint32_t* bk, uint16_t* bs /* panel base */) {
  using Geo = ChunkGeom<S>;
  const uint32_t* payload = d.payload + bk[0];
  const uint32_t l0 = bk[1], n = bk[2];
  for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
    uint32_t w[P];
    load_chunk<P, false>(payload + (size_t)t * P, w);
    float q[32];
    decode_chunk<P>(w, q);
    if constexpr (S == 4) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t leaf = l0 + 2 * t + h;
        const LeafInfo li = leaf_info(d.leaf_word[leaf], d.leaf_scale, leaf);
        if (li.pad) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) store_bf16_run<4>(bs + (li.col + g) * kGLds + li.row, q + (4 * h + g) * 4, li.scale);
      }
    } else {
      const uint32_t leaf = l0 + t / Geo::chunks_per_leaf;
      const int cbase = (int)(t % Geo::chunks_per_leaf) * Geo::G;
      const LeafInfo li = leaf_info(d.leaf_word[leaf], d.leaf_scale, leaf);
#pragma unroll
      for (int g = 0; g < Geo::G; ++g)
        store_bf16_run<Geo::R>(bs + (li.col + cbase + g) * kGLds + li.row, q + g * Geo::R, li.scale);
    }
  }
}

__device__ __forceinline__ uint16_t load_x_bf16(const void* X, int xdt, int64_t idx) {
  if (xdt == MTC_DTYPE_BF16) return reinterpret_cast<const uint16_t*>(X)[idx];
  return (uint16_t)f32_to_bf16_bits(reinterpret_cast<const float*>(X)[idx]);
}

__global__ __launch_bounds__(256) void k_gemm_bf16(const mtc_stream_desc d, const void* __restrict__ X, int xdt, int64_t ldx,
                                                  void* __restrict__ Y, int ydt, int64_t ldy, int M, int x_vec) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kGBM * kGLds];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kGBN * kGLds];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int p0 = blockIdx.x * (kGBN / kPanel);
  const int m0 = blockIdx.y * kGBM;
  const int wm = wave >> 1, wn = wave & 1;
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  for (int chunk = 0; chunk < d.n_chunks; ++chunk) {
    const int kb = chunk * kGBK;
    const int rows = min(kGBK, d.K - kb);
    __syncthreads();
    // zero the weight tile (P0 leaves leave zeros behind)
    for (int i = tid; i < kGBN * kGLds / 8; i += 256) reinterpret_cast<uint4*>(Bs)[i] = make_uint4(0, 0, 0, 0);
    // activation tile: 128 rows x 64 k, 8 k per item
    for (int it = tid; it < kGBM * (kGBK / 8); it += 256) {
      const int r = it >> 3, k8 = (it & 7) * 8;
      const int m = m0 + r;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m < M) {
        if (x_vec && k8 + 8 <= rows) {
          v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(X) + (int64_t)m * ldx + kb + k8);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            e[j] = 0;
            if (k8 + j < rows) {
              int k = kb + k8 + j;
              if (d.row_perm) k = d.row_perm[k];
              e[j] = load_x_bf16(X, xdt, (int64_t)m * ldx + k);
            }
          }
          v.x = e[0] | ((uint32_t)e[1] << 16);
          v.y = e[2] | ((uint32_t)e[3] << 16);
          v.z = e[4] | ((uint32_t)e[5] << 16);
          v.w = e[6] | ((uint32_t)e[7] << 16);
        }
      }
      *reinterpret_cast<uint4*>(As + r * kGLds + k8) = v;
    }
    __syncthreads();
    // weight tile: dequantize the leaves of up to 4 panel units into LDS
    for (int pi = 0; pi < kGBN / kPanel; ++pi) {
      const int p = p0 + pi;
      if (p >= d.n_panels) break;
      const int u = p * d.n_chunks + chunk;
      uint16_t* bs = Bs + pi * kPanel * kGLds;
      const int b0 = d.unit_buckets[u], b1 = d.unit_buckets[u + 1];
      for (int b = b0; b < b1; ++b) {
        const uint32_t* bk = d.buckets + 4 * b;
        switch (bk[3]) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): gemm_bucket<S, P>(d, bk, bs); break;
          MTC_FOR_EACH_BUCKET(MTC_CASE)
#undef MTC_CASE
          default: break;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kGBK / 16; ++ks) {
      bf16x8_t a[2], b[2];
      const int koff = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t*>(As + (wm * 64 + i * 32 + (lane & 31)) * kGLds + koff);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t*>(Bs + (wn * 64 + j * 32 + (lane & 31)) * kGLds + koff);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: accumulator element e of lane l is row (e/4)*8 + (l/32)*4 + e%4, column l%32
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = p0 * kPanel + wn * 64 + j * 32 + (lane & 31);
      if (n >= d.N) continue;
      const int col = d.col_perm ? d.col_perm[n] : n;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (m < M) {
          if (ydt == MTC_DTYPE_BF16)
            reinterpret_cast<uint16_t*>(Y)[(int64_t)m * ldy + col] = (uint16_t)f32_to_bf16_bits(acc[i][j][e]);
          else
            reinterpret_cast<float*>(Y)[(int64_t)m * ldy + col] = acc[i][j][e];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
int check_desc(const mtc_stream_desc* d) {
  if (!d) return fail(MTC_E_NULL, "descriptor is NULL");
  if (d->abi_version != MTC_ABI_VERSION)
    return fail(MTC_E_VERSION, "descriptor ABI %u, library ABI %d", d->abi_version, MTC_ABI_VERSION);
  if (d->K <= 0 || d->N <= 0 || d->N % kPanel)
    return fail(MTC_E_DESC, "bad shape K=%d N=%d (N must be a positive multiple of %d)", d->K, d->N, kPanel);
  if (d->chunk_rows <= 0 || d->chunk_rows % 32 || d->chunk_rows > 1024)
    return fail(MTC_E_DESC, "chunk_rows=%d must be a multiple of 32 in [32, 1024]", d->chunk_rows);
  if (d->n_panels != d->N / kPanel) return fail(MTC_E_DESC, "n_panels=%d != N/32=%d", d->n_panels, d->N / kPanel);
  if (d->n_chunks != (d->K + d->chunk_rows - 1) / d->chunk_rows)
    return fail(MTC_E_DESC, "n_chunks=%d inconsistent with K=%d chunk_rows=%d", d->n_chunks, d->K, d->chunk_rows);
  if (!d->unit_buckets) return fail(MTC_E_NULL, "unit_buckets is NULL");
  if (d->n_buckets > 0 && (!d->buckets || !d->payload || !d->leaf_word))
    return fail(MTC_E_NULL, "stream arrays missing for %d buckets", d->n_buckets);
  if ((d->flags & MTC_FLAG_FP32_SCALES) && !d->leaf_scale && d->n_leaves > 0)
    return fail(MTC_E_NULL, "fp32-scale stream without leaf_scale");
  if (!(d->flags & MTC_FLAG_FP32_SCALES) && d->leaf_scale)
    return fail(MTC_E_DESC, "leaf_scale given but MTC_FLAG_FP32_SCALES not set");
  return ok();
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int gemv_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

size_t gemv_ws_layout(const mtc_stream_desc* d, int M, size_t* counters_bytes) {
  const int mt = gemv_mt(M);
  const size_t n_mt = (size_t)((M + mt - 1) / mt);
  const size_t cb = ((n_mt * d->n_panels * sizeof(uint32_t)) + 255) & ~(size_t)255;
  if (counters_bytes) *counters_bytes = cb;
  if (d->n_chunks == 1) return 0;
  return cb + n_mt * (size_t)d->n_panels * d->n_chunks * mt * kPanel * sizeof(float);
}

template <int MT>
int launch_gemv(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M, void* ws,
                hipStream_t st) {
  size_t cb = 0;
  gemv_ws_layout(d, M, &cb);
  uint32_t* counters = reinterpret_cast<uint32_t*>(ws);
  float* part = ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + cb) : nullptr;
  const size_t shmem = (size_t)(MT * d->chunk_rows + kGemvWaves * MT * kPanel) * sizeof(float);
  if (shmem > 64 * 1024)
    return fail(MTC_E_SHAPE, "fp32 path: %d rows x chunk_rows=%d needs %zu B of LDS (max 65536); use a stream "
                "with smaller chunk_rows", MT, d->chunk_rows, shmem);
  dim3 grid(d->n_panels * d->n_chunks, (M + MT - 1) / MT);
  hipLaunchKernelGGL(k_gemv<MT>, grid, dim3(kGemvThreads), shmem, st, *d, X, ldx, Y, ldy, M, part, counters);
  return check_launch("k_gemv");
}

}  // namespace

MTC_API int mtc_abi_version(void) { return MTC_ABI_VERSION; }

MTC_API const char* mtc_last_error(void) { return g_err; }

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
  hipLaunchKernelGGL(k_dequant, dim3(d->n_panels * d->n_chunks), dim3(256), 0, st, *d, W_out);
  return check_launch("k_dequant");
}

MTC_API size_t mtc_gemv_workspace_bytes(const mtc_stream_desc* d, int M) {
  if (check_desc(d) || M <= 0) return 0;
  return gemv_ws_layout(d, M, nullptr);
}

MTC_API int mtc_gemv_f32(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M,
                         void* workspace, size_t workspace_bytes, void* hip_stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!X || !Y) return fail(MTC_E_NULL, "X or Y is NULL");
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  if (ldx < d->K || ldy < d->N) return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy=%lld < N", (long long)ldx, (long long)ldy);
  if ((M - 1) > (INT64_MAX / ldx)) return fail(MTC_E_SHAPE, "M * ldx overflows");
  const size_t need = gemv_ws_layout(d, M, nullptr);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MTC_E_WORKSPACE, "GEMV workspace of %zu bytes needed, %zu given", need, workspace ? workspace_bytes : 0);
  hipStream_t st = as_stream(hip_stream);
  switch (gemv_mt(M)) {
    case 1: return launch_gemv<1>(d, X, ldx, Y, ldy, M, workspace, st);
    case 2: return launch_gemv<2>(d, X, ldx, Y, ldy, M, workspace, st);
    case 4: return launch_gemv<4>(d, X, ldx, Y, ldy, M, workspace, st);
    case 8: return launch_gemv<8>(d, X, ldx, Y, ldy, M, workspace, st);
    default: return launch_gemv<16>(d, X, ldx, Y, ldy, M, workspace, st);
  }
}

MTC_API int mtc_gemm_bf16(const mtc_stream_desc* d, const void* X, int x_dtype, int64_t ldx, void* Y, int y_dtype,
                          int64_t ldy, int M, void* hip_stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!X || !Y) return fail(MTC_E_NULL, "X or Y is NULL");
  if (d->chunk_rows != kGBK) return fail(MTC_E_SHAPE, "bf16 GEMM needs a stream with chunk_rows=%d (got %d)", kGBK, d->chunk_rows);
  if (x_dtype != MTC_DTYPE_F32 && x_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "x_dtype=%d", x_dtype);
  if (y_dtype != MTC_DTYPE_F32 && y_dtype != MTC_DTYPE_BF16) return fail(MTC_E_DTYPE, "y_dtype=%d", y_dtype);
  if (M <= 0) return fail(MTC_E_SHAPE, "M=%d must be positive", M);
  if (ldx < d->K || ldy < d->N) return fail(MTC_E_SHAPE, "ldx=%lld < K or ldy=%lld < N", (long long)ldx, (long long)ldy);
  // 16-byte activation loads: bf16, unpermuted, row starts aligned
  const int x_vec = (x_dtype == MTC_DTYPE_BF16 && !d->row_perm && ldx % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(X) & 15) == 0) ? 1 : 0;
  dim3 grid((d->n_panels * kPanel + kGBN - 1) / kGBN, (M + kGBM - 1) / kGBM);
  hipLaunchKernelGGL(k_gemm_bf16, grid, dim3(256), 0, as_stream(hip_stream), *d, X, x_dtype, ldx, Y, y_dtype, ldy, M, x_vec);
  return check_launch("k_gemm_bf16");
}
