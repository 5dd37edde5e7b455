// CPU half of the offline rate-distortion allocator: the exhaustive per-block
// scale search. Host-only code (g++, OpenMP); it never touches the GPU.
//
// Semantics follow mtc/core/allocation.py:106-136 (_search_kernel) and
// allocation.py:97-103 (_round_bf16) operation for operation, because the
// allocator's leaf/mode/scale decisions hinge on exact fp32 rounding:
//   s   = f32( f64( f32(sign*alpha) * amax ) / qmag )      [f32 mul, f64 div]
//   s   = round-to-8-significant-bits(s), ties to even      [if bf16 scales]
//   inv = f32(1) / s                                         [f32 div]
//   q   = clamp(rint_even(x * inv), lo, hi)                  [f32]
//   e   = x - q * s ;  acc_r += e * e                        [f32, column order]
//   d   = sum_r h_r * acc_r                                  [f64, row order]
// and the first candidate with the strictly smallest d wins (alpha ascending,
// then sign +, -). The file must be compiled with -ffp-contract=off so that no
// multiply-add is fused.
//
// The only liberty taken is evaluation order across independent chains: the
// Bs row accumulators are advanced together (vectorised over r), each one still
// summing its columns c = 0..Bs-1 in order, so every acc_r is bit-identical to
// the scalar loop.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <omp.h>

namespace {

inline double round_sig8(double x) {
  if (x == 0.0) return x;
  int e = 0;
  double m = std::frexp(x, &e);             // |m| in [0.5, 1)
  double r = std::nearbyint(m * 256.0);     // default mode: ties to even
  return std::ldexp(r / 256.0, e);
}

template <int BS>
void search_block(const float* __restrict blk, const double* __restrict hrow, float amax,
                  float lo, float hi, double qmag, const float* alphas, int n_alpha,
                  const float* signs, int n_sign, bool bf16, double* out_d, float* out_s) {
  // column-major copy: xt[c*BS + r] = blk[r*BS + c]
  alignas(64) float xt[BS * BS];
  for (int r = 0; r < BS; ++r)
    for (int c = 0; c < BS; ++c) xt[c * BS + r] = blk[r * BS + c];

  double bd = std::numeric_limits<double>::infinity();
  float bs = 0.0f;
  for (int ai = 0; ai < n_alpha; ++ai) {
    for (int si = 0; si < n_sign; ++si) {
      float t = signs[si] * alphas[ai];
      t = t * amax;
      float s = static_cast<float>(static_cast<double>(t) / qmag);
      if (bf16) s = static_cast<float>(round_sig8(static_cast<double>(s)));
      const float inv = 1.0f / s;
      alignas(64) float acc[BS];
      for (int r = 0; r < BS; ++r) acc[r] = 0.0f;
      for (int c = 0; c < BS; ++c) {
        const float* col = xt + c * BS;
#pragma GCC ivdep
        for (int r = 0; r < BS; ++r) {
          const float x = col[r];
          float q = std::nearbyint(x * inv);
          q = q < lo ? lo : q;
          q = q > hi ? hi : q;
          const float e = x - q * s;
          acc[r] = acc[r] + e * e;
        }
      }
      double d = 0.0;
      for (int r = 0; r < BS; ++r) d += hrow[r] * static_cast<double>(acc[r]);
      if (d < bd) {
        bd = d;
        bs = s;
      }
    }
  }
  *out_d = bd;
  *out_s = bs;
}

template <int BS>
void search_all(const float* blocks, const double* h, const float* amax, int64_t nb, float lo,
                float hi, double qmag, const float* alphas, int n_alpha, const float* signs,
                int n_sign, bool bf16, double* best_d, float* best_s) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t b = 0; b < nb; ++b) {
    search_block<BS>(blocks + b * BS * BS, h + b * BS, amax[b], lo, hi, qmag, alphas, n_alpha,
                     signs, n_sign, bf16, best_d + b, best_s + b);
  }
}

}  // namespace

extern "C" {

// Returns 0 on success, -1 on an unsupported block size, -2 on a null pointer.
//   blocks : (nb, bs, bs) float32, row-major within each block
//   h      : (nb, bs) float64 row importance
//   amax   : (nb,) float32 block abs-max (already floored to 1 where tiny)
int mtc_rd_search(const float* blocks, const double* h, const float* amax, int64_t nb, int bs,
                  double lo, double hi, double qmag, const float* alphas, int n_alpha,
                  const float* signs, int n_sign, int round_bf16, int n_threads, double* best_d,
                  float* best_s) {
  if (nb == 0) return 0;
  if (!blocks || !h || !amax || !alphas || !signs || !best_d || !best_s) return -2;
  if (n_threads > 0) omp_set_num_threads(n_threads);
  const float flo = static_cast<float>(lo), fhi = static_cast<float>(hi);
  const bool bf = round_bf16 != 0;
  switch (bs) {
    case 4: search_all<4>(blocks, h, amax, nb, flo, fhi, qmag, alphas, n_alpha, signs, n_sign, bf, best_d, best_s); break;
    case 8: search_all<8>(blocks, h, amax, nb, flo, fhi, qmag, alphas, n_alpha, signs, n_sign, bf, best_d, best_s); break;
    case 16: search_all<16>(blocks, h, amax, nb, flo, fhi, qmag, alphas, n_alpha, signs, n_sign, bf, best_d, best_s); break;
    case 32: search_all<32>(blocks, h, amax, nb, flo, fhi, qmag, alphas, n_alpha, signs, n_sign, bf, best_d, best_s); break;
    case 64: search_all<64>(blocks, h, amax, nb, flo, fhi, qmag, alphas, n_alpha, signs, n_sign, bf, best_d, best_s); break;
    default: return -1;
  }
  return 0;
}

// Round each value to 8 significant bits, ties to even (allocation.py:97-103).
void mtc_round_sig8(const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = static_cast<float>(round_sig8(static_cast<double>(in[i])));
}

int mtc_rd_abi_version(void) { return 1; }

}  // extern "C"
