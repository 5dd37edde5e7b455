/*
 * CPU oracle / CPU baseline -- TEST INFRASTRUCTURE ONLY (tests/, smoke(), and
 * bench.py's cpu_baseline leg). Never linked into the product.
 *
 * Port of the loop structure of the reference's numba kernel
 * mtc_gemm_core_kernel (mtc/kernels/gemm.py:124-210), generalized from
 * uniform A/B blocks to a dense X and quadtree leaves of any size:
 *   - skip P0 leaves (they are not listed),
 *   - unpack each leaf's codes to f32 with the reference codecs
 *     (gemm.py:29-117: P2 4/byte, P4 2/byte, P8 int8, P16 LE int16,
 *     P3/P5/P6 little-endian bitstream), row-major within the leaf,
 *   - c_acc[m][c] += (x[m][k] * scale) * b[k][c]   (gemm.py:200-205),
 *   - parallel over 32-column output panels (the reference's prange over
 *     row blocks degenerates at M = 1).
 */
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static void unpack_leaf(const uint8_t* a, int64_t off, int s, int mode, float* out) {
  const int n = s * s;
  if (mode == 2) {
    for (int i = 0; i < n; ++i) {
      int v = (a[off + (i >> 2)] >> (2 * (i & 3))) & 3;
      out[i] = (float)(v >= 2 ? v - 4 : v);
    }
  } else if (mode == 4) {
    for (int i = 0; i < n; ++i) {
      int v = (a[off + (i >> 1)] >> (4 * (i & 1))) & 15;
      out[i] = (float)(v >= 8 ? v - 16 : v);
    }
  } else if (mode == 8) {
    for (int i = 0; i < n; ++i) out[i] = (float)(int8_t)a[off + i];
  } else if (mode == 16) {
    for (int i = 0; i < n; ++i) out[i] = (float)(int16_t)(a[off + 2 * i] | (a[off + 2 * i + 1] << 8));
  } else {
    const int mask = (1 << mode) - 1, sign = 1 << (mode - 1);
    for (int i = 0; i < n; ++i) {
      const int64_t bit = (int64_t)i * mode;
      const int64_t byte = off + (bit >> 3);
      const int sh = (int)(bit & 7);
      int word = a[byte];
      if (sh + mode > 8) word |= a[byte + 1] << 8;
      int v = (word >> sh) & mask;
      if (v >= sign) v -= 1 << mode;
      out[i] = (float)v;
    }
  }
}

int oracle_threads(void) { return omp_get_max_threads(); }

/* X: M x K row-major. Leaves sorted by panel; panel_begin has n_panels+1 entries.
 * Y: M x N row-major (written). row_perm/col_perm may be NULL. */
int oracle_qt_gemm(const float* X, int M, int K, int N, const uint8_t* arena, const int64_t* off, const int32_t* k0,
                   const int32_t* n0, const int32_t* size, const int32_t* mode, const float* scale,
                   const int64_t* panel_begin, const int32_t* row_perm, const int32_t* col_perm, float* Y,
                   void* reserved, int n_threads) {
  (void)reserved;
  if (!X || !arena || !Y || N % 32) return -1;
  if (n_threads > 0) omp_set_num_threads(n_threads);
  const int n_panels = N / 32;
  int err = 0;
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)M * 32);
    float* buf = (float*)malloc(sizeof(float) * 32 * 32);
    if (!acc || !buf) {
#pragma omp atomic write
      err = -2;
    }
#pragma omp for schedule(dynamic, 1)
    for (int p = 0; p < n_panels; ++p) {
      if (!acc || !buf) continue;
      memset(acc, 0, sizeof(float) * (size_t)M * 32);
      for (int64_t l = panel_begin[p]; l < panel_begin[p + 1]; ++l) {
        const int s = size[l];
        const int c0 = n0[l] - p * 32;
        const float sc = scale[l];
        unpack_leaf(arena, off[l], s, mode[l], buf);
        for (int m = 0; m < M; ++m) {
          float* am = acc + (size_t)m * 32 + c0;
          for (int r = 0; r < s; ++r) {
            int k = k0[l] + r;
            if (row_perm) k = row_perm[k];
            const float v = X[(size_t)m * K + k] * sc;
            const float* br = buf + r * s;
            for (int c = 0; c < s; ++c) am[c] += v * br[c];
          }
        }
      }
      for (int m = 0; m < M; ++m)
        for (int c = 0; c < 32; ++c) {
          int n = p * 32 + c;
          if (col_perm) n = col_perm[n];
          Y[(size_t)m * N + n] = acc[(size_t)m * 32 + c];
        }
    }
    free(acc);
    free(buf);
  }
  return err;
}
