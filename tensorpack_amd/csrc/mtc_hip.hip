// gfx950 decode kernels and C-ABI for Y = X * W_hat over the panel stream,
// plus the host error state shared with mtc_gemm.hip.
//
//   k_fill_zero  : zero an fp32 buffer (used before dequant; no memset nodes)
//   k_dequant    : stream -> dense W_hat (bit-exact q*s, +0.0 for P0)
//   k_gemv<MT>   : fp32 decode path. One block per (unit, column-group range);
//                  the unit's payload is staged in LDS, each wave owns one
//                  column group and accumulates its 4 columns in registers
//                  (no atomics), then reduces across lanes once.
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
template <int S, int P>
__device__ __forceinline__ void dequant_chunk(const mtc_stream_desc& d, const uint32_t* src, const uint32_t* lw,
                                              uint32_t lg0, uint32_t t, int kb, int col0, float* __restrict__ W) {
  uint32_t w[P];
  load_chunk<P, true>(src, w);
  float q[32];
  decode_chunk<P>(w, q);
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
  for (int b = 0; b < nb; ++b) {
    const Bucket e = read_bucket(bk + 4 * b);
    const uint32_t* lw = d.leaf_word + hdr[2] + e.leaf;
    const uint32_t lg0 = hdr[2] + e.leaf;
    for (uint32_t t = lane; t < e.n; t += 64) {
      switch (e.key) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): dequant_chunk<S, P>(d, pay + e.pay + t * P, lw, lg0, t, kb, col0, W); break;
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
// Block = (unit, G adjacent column groups), two waves per column group. The
// block copies its column groups' payload and bucket entries and the unit's
// leaf words into LDS with every load of a round in flight at once, and
// gathers X rows (row_perm) into LDS alongside. A column group's work is a
// list of 64-chunk steps, each inside ONE bucket (a bucket of n chunks gives
// ceil(n/64) steps), so the bucket kind of a step is wave-uniform and
// dispatches on a scalar register; the group's two waves split the steps.
// Lanes accumulate their 4 columns in registers (no atomics). Blocks of one
// unit are mapped to the same XCD so its leaf words stay in one L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dot4(const float4 x, const float* q) {
  return x.x * q[0] + x.y * q[1] + x.z * q[2] + x.w * q[3];
}

// One lane chunk from LDS into the lane's 4-column accumulators.
template <int S, int P, int MT>
__device__ __forceinline__ void gemv_chunk(const uint32_t* src, const uint32_t* lw, uint32_t t, const float* fscale,
                                           uint32_t lg0, const float* xs, int kc, float (&acc)[MT][kGroup]) {
  uint32_t w[P];
  lds_chunk<P>(src, w);
  float q[32];
  decode_chunk<P>(w, q);
  if constexpr (S == 4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t leaf = 2 * t + h;
      const LeafInfo li = leaf_info(lw[leaf], fscale, lg0 + leaf);
      if (li.pad) continue;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 x = *reinterpret_cast<const float4*>(xs + m * kc + li.row);
#pragma unroll
        for (int c = 0; c < kGroup; ++c) acc[m][c] += li.scale * dot4(x, q + 16 * h + 4 * c);
      }
    }
  } else {
    constexpr int NRB = S / 8;
    const uint32_t leaf = t / NRB;
    const LeafInfo li = leaf_info(lw[leaf], fscale, lg0 + leaf);
    const int row = li.row + 8 * (int)(t % NRB);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float4 x0 = *reinterpret_cast<const float4*>(xs + m * kc + row);
      const float4 x1 = *reinterpret_cast<const float4*>(xs + m * kc + row + 4);
#pragma unroll
      for (int c = 0; c < kGroup; ++c) acc[m][c] += li.scale * (dot4(x0, q + 8 * c) + dot4(x1, q + 8 * c + 4));
    }
  }
}

constexpr int kGemvWavesPerGroup = 2;
constexpr int kStageU4 = 8;     // uint4 payload loads in flight per thread per staging round
constexpr int kStageW = 8;      // leaf-word loads per thread per round
constexpr int kXcds = 8;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// M-tile rows -> column groups per block (more X rows on chip, fewer blocks per CU)
__host__ __device__ constexpr int gemv_groups(int MT) { return MT <= 2 ? 2 : 4; }

template <int MT>
__global__ __launch_bounds__(64 * kGemvWavesPerGroup * gemv_groups(MT)) void k_gemv(
    const mtc_stream_desc d, const float* __restrict__ X, int64_t ldx, float* __restrict__ Y, int64_t ldy, int M,
    float* __restrict__ part, uint32_t* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int G = gemv_groups(MT), V = kGemvWavesPerGroup, W = G * V, T = 64 * W;
  constexpr int BPU = kGroups / G;                    // blocks per unit
  const int kc = d.chunk_rows;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_units = d.n_panels * d.n_chunks;
  // block -> (unit, column-group block) with all blocks of a unit on one XCD
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
  const int u = (slot / BPU) * kXcds + xcd;
  if (u >= n_units) return;                           // padding block of the XCD mapping
  const int cg_lo = (slot % BPU) * G;
  const int mt = blockIdx.y;
  const int panel = u / d.n_chunks, chunk = u - panel * d.n_chunks;
  const int m0 = mt * MT;
  const int kb = chunk * kc;
  const int rows = min(kc, d.K - kb);

  float* xs = smem;                                   // [MT][kc]
  float* red = xs + MT * kc;                          // [waves][MT][4]
  uint32_t* s_pay = reinterpret_cast<uint32_t*>(red + W * MT * kGroup);   // 16-byte aligned

  const int32_t* hdr = d.unit_hdr + kUnitHdr * u;
  const int pay_lo = hdr[17 + cg_lo], npay = hdr[17 + cg_lo + G] - pay_lo;
  const int lf0 = hdr[2], nlf = hdr[3] - hdr[2];
  const int bk_lo = hdr[8 + cg_lo], nbk = hdr[8 + cg_lo + G] - bk_lo;
  uint32_t* s_lw = s_pay + npay;
  uint32_t* s_bk = s_lw + nlf;

  // ---- stage: every global load of a round (branch-free, clamped index) goes
  // out before any LDS store; X indices and bucket entries ride along ----
  {
    const u32x4_t* gpay = reinterpret_cast<const u32x4_t*>(d.payload + hdr[0] + pay_lo);
    const uint32_t* glw = d.leaf_word + lf0;
    const int npay4 = npay >> 2;
    constexpr int XR = kMaxChunkRows / T;
    int kk[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      const int k = kb + min(i * T + tid, rows - 1);
      kk[i] = d.row_perm ? d.row_perm[k] : k;
    }
    for (int i = tid; i < 4 * nbk; i += T) s_bk[i] = d.buckets[4 * (hdr[4] + bk_lo) + i];
    const int rounds = max((npay4 + T * kStageU4 - 1) / (T * kStageU4), (nlf + T * kStageW - 1) / (T * kStageW));
    for (int r = 0; r < rounds; ++r) {
      u32x4_t pv[kStageU4];
      uint32_t lv[kStageW];
      if (npay4 > 0) {
#pragma unroll
        for (int i = 0; i < kStageU4; ++i) pv[i] = __builtin_nontemporal_load(gpay + min((r * kStageU4 + i) * T + tid, npay4 - 1));
      }
      if (nlf > 0) {
#pragma unroll
        for (int i = 0; i < kStageW; ++i) lv[i] = glw[min((r * kStageW + i) * T + tid, nlf - 1)];
      }
#pragma unroll
      for (int i = 0; i < kStageU4; ++i) {
        const int idx = (r * kStageU4 + i) * T + tid;
        if (idx < npay4) reinterpret_cast<u32x4_t*>(s_pay)[idx] = pv[i];
      }
#pragma unroll
      for (int i = 0; i < kStageW; ++i) {
        const int idx = (r * kStageW + i) * T + tid;
        if (idx < nlf) s_lw[idx] = lv[i];
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float* xrow = X + (int64_t)min(m0 + m, M - 1) * ldx;
      float xv[XR];
#pragma unroll
      for (int i = 0; i < XR; ++i) xv[i] = (i * T < kc) ? xrow[kk[i]] : 0.0f;
#pragma unroll
      for (int i = 0; i < XR; ++i) {
        const int rr = i * T + tid;
        if (rr < kc) xs[m * kc + rr] = (rr < rows && m0 + m < M) ? xv[i] : 0.0f;
      }
    }
  }
  __syncthreads();

  // ---- decode: the column group's steps, split between its V waves ----
  float acc[MT][kGroup];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < kGroup; ++c) acc[m][c] = 0.0f;
  {
    const int gl = wave / V, sub = wave % V;
    const int b0 = hdr[8 + cg_lo + gl] - bk_lo, b1 = hdr[8 + cg_lo + gl + 1] - bk_lo;
    int nsteps = 0;
    for (int b = b0; b < b1; ++b) nsteps += (int)(((s_bk[4 * b + 2] & 0xFFFFu) + 63) >> 6);
    const int per = (nsteps + V - 1) / V;
    const int s_beg = sub * per, s_end = min(s_beg + per, nsteps);
    // advance to the bucket holding step s_beg (uniform)
    int b = b0, bsteps = 0, s = 0;
    if (s_beg < s_end) {
      while (true) {
        bsteps = (int)(((s_bk[4 * b + 2] & 0xFFFFu) + 63) >> 6);
        if (s + bsteps > s_beg) break;
        s += bsteps;
        ++b;
      }
    }
    int k = s_beg - s;                                // step within bucket b
    for (int st = s_beg; st < s_end; ++st) {
      const Bucket e = read_bucket(s_bk + 4 * b);
      const uint32_t t = (uint32_t)(64 * k + lane);
      if (t < e.n) {
        const uint32_t* src = s_pay + (e.pay - pay_lo);
        const uint32_t* lw = s_lw + e.leaf;
        const uint32_t lg0 = lf0 + e.leaf;
        // e.key is the same for every lane (one bucket per step): scalar dispatch
        switch (__builtin_amdgcn_readfirstlane(e.key)) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): gemv_chunk<S, P, MT>(src + t * P, lw, t, d.leaf_scale, lg0, xs, kc, acc); break;
          MTC_FOR_EACH_BUCKET(MTC_CASE)
#undef MTC_CASE
          default: break;
        }
      }
      if (++k == bsteps && st + 1 < s_end) {
        ++b;
        k = 0;
        bsteps = (int)(((s_bk[4 * b + 2] & 0xFFFFu) + 63) >> 6);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < kGroup; ++c) acc[m][c] = wave_sum(acc[m][c]);
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < kGroup; ++c) red[(wave * MT + m) * kGroup + c] = acc[m][c];
  }
  __syncthreads();

  // ---- combine the waves of each column group; write Y or this block's partial ----
  constexpr int nout = MT * G * kGroup;
  if (d.n_chunks == 1) {
    for (int i = tid; i < nout; i += T) {
      const int m = i / (G * kGroup), gc = i - m * (G * kGroup);
      const int gl = gc / kGroup, c = gc - gl * kGroup;
      float v = 0.0f;
#pragma unroll
      for (int s2 = 0; s2 < V; ++s2) v += red[((gl * V + s2) * MT + m) * kGroup + c];
      if (m0 + m < M) {
        int col = panel * kPanel + (cg_lo + gl) * kGroup + c;
        if (d.col_perm) col = d.col_perm[col];
        Y[(int64_t)(m0 + m) * ldy + col] = v;
      }
    }
    return;
  }

  // split-K over chunks: deterministic last-block reduction per (M tile, panel)
  constexpr int n_part = MT * kPanel;
  float* mine = part + ((size_t)mt * n_units + u) * n_part;
  for (int i = tid; i < nout; i += T) {
    const int m = i / (G * kGroup), gc = i - m * (G * kGroup);
    const int gl = gc / kGroup, c = gc - gl * kGroup;
    float v = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < V; ++s2) v += red[((gl * V + s2) * MT + m) * kGroup + c];
    __hip_atomic_store(mine + m * kPanel + (cg_lo + gl) * kGroup + c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __threadfence();
  __syncthreads();
  __shared__ int last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[mt * d.n_panels + panel], 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last = (prev == (uint32_t)(d.n_chunks * BPU - 1));
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
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
  if ((d->flags & MTC_FLAG_FP32_SCALES) && !d->leaf_scale && d->n_leaves > 0)
    return fail(MTC_E_NULL, "fp32-scale stream without leaf_scale");
  if (!(d->flags & MTC_FLAG_FP32_SCALES) && d->leaf_scale)
    return fail(MTC_E_DESC, "leaf_scale given but MTC_FLAG_FP32_SCALES not set");
  return ok();
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

using mtc::host::device_lds_limit;

int gemv_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }

size_t gemv_ws_layout(const mtc_stream_desc* d, int M, size_t* counters_bytes) {
  const int mt = gemv_mt(M);
  const size_t n_mt = (size_t)((M + mt - 1) / mt);
  const size_t cb = ((n_mt * d->n_panels * sizeof(uint32_t)) + 255) & ~(size_t)255;
  if (counters_bytes) *counters_bytes = cb;
  if (d->n_chunks == 1) return 0;
  return cb + n_mt * (size_t)d->n_panels * d->n_chunks * mt * kPanel * sizeof(float);
}

size_t gemv_lds_bytes(const mtc_stream_desc* d, int MT) {
  const int waves = kGemvWavesPerGroup * gemv_groups(MT);
  const int staged = gemv_groups(MT) == 2 ? d->max_unit_words : d->max_unit_words4;
  return ((size_t)MT * d->chunk_rows + (size_t)waves * MT * kGroup + (size_t)staged) * 4;
}

template <int MT>
int launch_gemv(const mtc_stream_desc* d, const float* X, int64_t ldx, float* Y, int64_t ldy, int M, void* ws,
                hipStream_t st) {
  size_t cb = 0;
  gemv_ws_layout(d, M, &cb);
  uint32_t* counters = reinterpret_cast<uint32_t*>(ws);
  float* part = ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + cb) : nullptr;
  const size_t shmem = gemv_lds_bytes(d, MT);
  const size_t limit = device_lds_limit();
  if (shmem > limit)
    return fail(MTC_E_SHAPE, "fp32 path: %d rows x chunk_rows=%d with %d staged words needs %zu B of LDS (limit %zu); "
                "use a stream with smaller chunk_rows", MT, d->chunk_rows, d->max_unit_words, shmem, limit);
  if (shmem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<MT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
    if (e != hipSuccess) return fail(MTC_E_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  }
  constexpr int G = gemv_groups(MT);
  const int n_units = d->n_panels * d->n_chunks;
  const int units_padded = (n_units + kXcds - 1) / kXcds * kXcds;
  dim3 grid(units_padded * (kGroups / G), (M + MT - 1) / MT);
  hipLaunchKernelGGL(k_gemv<MT>, grid, dim3(64 * kGemvWavesPerGroup * G), shmem, st, *d, X, ldx, Y, ldy, M, part,
                     counters);
  return check_launch("k_gemv");
}

}  // namespace

MTC_API int mtc_abi_version(void) { return MTC_ABI_VERSION; }

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
    default: return launch_gemv<4>(d, X, ldx, Y, ldy, M, workspace, st);
  }
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
