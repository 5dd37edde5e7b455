/*
 * C-ABI of libmtc_rd.so: the host-side (CPU, OpenMP) exhaustive scale search
 * of the offline rate-distortion allocator. Stays on the CPU by design.
 *
 * Reference interfaces replaced (Sharexi/TensorPack):
 *   mtc_rd_search  <- _search_kernel, mtc/core/allocation.py:106-136 (numba, parallel)
 *   mtc_round_sig8 <- _round_bf16,    mtc/core/allocation.py:97-103
 */
#ifndef MTC_RD_H
#define MTC_RD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* For each of nb blocks (bs x bs float32, row-major) with row importance h
 * (nb x bs float64) and abs-max amax (nb float32), search scale candidates
 * s = f32(f32(sign*alpha)*amax / qmag) over alphas x signs (alpha-major), with
 * 8-significant-bit rounding when round_bf16 != 0, and keep the first with the
 * strictly smallest importance-weighted squared error. n_threads <= 0 keeps
 * the OpenMP default. Returns 0, -1 (unsupported bs) or -2 (NULL pointer). */
int mtc_rd_search(const float* blocks, const double* h, const float* amax, int64_t nb, int bs, double lo,
                  double hi, double qmag, const float* alphas, int n_alpha, const float* signs, int n_sign,
                  int round_bf16, int n_threads, double* best_d, float* best_s);

/* out[i] = in[i] rounded to 8 significant bits, ties to even. */
void mtc_round_sig8(const float* in, float* out, int64_t n);

int mtc_rd_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MTC_RD_H */
