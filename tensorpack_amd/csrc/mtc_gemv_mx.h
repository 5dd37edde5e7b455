// Decode of one X row on the matrix core, over the "mx" payload layout (MTC_FLAG_MX_LAYOUT,
// include/mtc_hip.h). Included by mtc_hip.hip inside its anonymous namespace, after the step
// record, buffer and reduction helpers it uses.
//
// A decode block is the same (unit, 4 column groups) block as the vector path's; lane
// (slot g, quad b, column j) = lane 16 g + 4 b + j of a wave takes column j of chunks
// 4 b .. 4 b + 3 of slot g's step, whose 32 codes are its P payload dwords. Its work per chunk is
// one block of v_mfma_f32_4x4x4_16b_f16 (16 independent 4x4x4 products per wave; block b on
// lanes 4b .. 4b + 3: A row i from lane 4b + i, B column j from lane 4b + j, D[i][j] in lane
// 4b + j register i):
//   B = four rows of the chunk in column j, as f16 values 2^W + u (u the offset-binary code of
//       plane width W; one shift and one masked OR per two codes, no convert);
//   A = the same four rows of X, split exactly enough in two f16 parts x' = hi + lo (rows 0
//       and 1 of A; rows 2 and 3 repeat them and are not used), after a power-of-two prescale
//       2^e per block that keeps |x'| < 2^13;
// so D[0][j] + D[1][j] = sum_r x'_r (2^W + u_r). A third MFMA with A = the two 4-row sums of x'
// (also split) and B = -(2^W + 2^(P-1)) in every entry subtracts the code bias, leaving
// sum_r x'_r q_r; the lane adds scale * (D[0] + D[1]) to its column's accumulator. Products of
// two f16 values are exact in fp32 and every sum is an fp32 sum, so the result is within the
// fp32 path's error (the 2^W term keeps the partial sums within a few times the signed ones).
// P = 16 is two planes of W = 8 (low and high bytes of u), combined as 256 D_hi + D_lo.
//
// X is staged per block in LDS as two f16 row arrays (hi, lo; kc rows each, the second starting
// mx_rows_stride(kc) bytes after the first) and two arrays of the 4-row sums of x' split the same
// way (kc / 4 each, mx_sums_stride(kc) bytes apart); the 64-byte pads put the two halves of a
// pair of reads on different LDS banks. A block's column accumulators are unscaled by 2^-e
// before the reduction, so split-K units combine in the original scale.

typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

// (x & m) | c, one v_and_or_b32 when m and c are register values: a VOP3 instruction, which on
// this target takes no 32-bit literal, so the masks and exponent words are kept in registers
// (MxK). Plain code, not inline assembly, so that the compiler sees the instruction and keeps the
// wait states the matrix core needs between writing an operand and reading it.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }

// The constants of plane width W in registers: the code mask at mantissa bits [10 - W, 10) of
// both halves, the exponent word of 2^W in both halves, and the two masks a code split over two
// dwords needs (its first n1 bits, its other W - n1 bits; n1 = 16 - s of the code at bit s).
template <int W>
struct MxK {
  uint32_t m, cc;
  __device__ __forceinline__ MxK() {
    constexpr int p = 10 - W;
    constexpr uint32_t mm = ((1u << W) - 1u) << p, C = (uint32_t)(15 + W) << 10;
    m = mm | (mm << 16);
    cc = C | (C << 16);
    asm volatile("" : "+v"(m), "+v"(cc));           // held in VGPRs, not rematerialized per use
  }
};

// Operand dword O (0..15) of a lane's codes of plane width W whose dwords start at w[BASE]:
// two f16 values 2^W + u for chunk O / 4, chunk rows 2 (O % 4) (low half) and 2 (O % 4) + 1
// (high half). Code O of each half-string sits at bits [O W, O W + W) of the string formed by
// the dwords' low (or high) 16-bit halves; it lands in mantissa bits [10 - W, 10) under the
// exponent of 2^W.
template <int W, int O, int BASE>
__device__ __forceinline__ uint32_t mx_op(const u32x16_t w, const MxK<W>& k) {
  constexpr int p = 10 - W;
  constexpr int b = O * W, d = BASE + (b >> 4), s = b & 15;
  if constexpr (s + W <= 16) {
    const uint32_t x = w[d];
    const uint32_t y = s == p ? x : s > p ? (x >> (s - p)) : (x << (p - s));
    return and_or(y, k.m, k.cc);
  } else {                                            // the code spans two dwords' halves
    constexpr int n1 = 16 - s;                        // its low bits in dword d (s > p here)
    constexpr uint32_t m1 = ((1u << n1) - 1u) << p, M1 = m1 | (m1 << 16);
    constexpr uint32_t m2 = ((1u << (W - n1)) - 1u) << (p + n1), M2 = m2 | (m2 << 16);
    const uint32_t lo = ((w[d] >> (s - p)) & M1) | k.cc;
    return lo | ((w[d + 1] << (p + n1)) & M2);
  }
}

// The B operand of chunk T, rows 4H .. 4H + 3, plane at dword BASE.
template <int W, int T, int H, int BASE>
__device__ __forceinline__ f16x4_t mx_b(const u32x16_t w, const MxK<W>& k) {
  const u32x2_t v = {mx_op<W, 4 * T + 2 * H, BASE>(w, k), mx_op<W, 4 * T + 2 * H + 1, BASE>(w, k)};
  return __builtin_bit_cast(f16x4_t, v);
}

// -(2^W + off) in the first `n` k slots of a B operand, 0 in the others.
template <int W, int OFF, int n>
__device__ __forceinline__ f16x4_t mx_bias() {
  constexpr _Float16 c = (_Float16)(-(float)((1 << W) + OFF));
  u32x2_t v = __builtin_bit_cast(u32x2_t, f16x4_t{c, n > 1 ? c : (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f});
  asm volatile("" : "+v"(v));                         // built once per step
  return __builtin_bit_cast(f16x4_t, v);
}

__device__ __forceinline__ f32x4_t mx_mfma(f16x4_t a, f16x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

// One lane's loads of a step, like the vector path's chunk li: its P payload dwords (dword
// pay + li P, the lane's column of its quad) and the leaf word(s) of chunk li (word li >>
// (log2 S - 3), or words 2 li, 2 li + 1 for S = 4; the second load reads past the buffer's end,
// zeros, for S >= 8), plus the fp32 scales at the same places for FS streams. The lanes of a
// quad hold the words of its four chunks between them; a chunk's word reaches the quad's other
// lanes by a DPP broadcast when it is needed, so a prefetched record costs 2 + P registers.
struct MxRegs {
  u32x16_t w;
  uint32_t lw0, lw1;
  float fs0, fs1;
  uint32_t ob, key, nv;
  bool live;             // the record has chunks (wave-uniform)
};

template <bool FS>
__device__ __forceinline__ void mx_load(__amdgpu_buffer_rsrc_t pay_r, __amdgpu_buffer_rsrc_t lw_r,
                                        __amdgpu_buffer_rsrc_t fs_r, uint32_t key, uint32_t pay, uint32_t leaf,
                                        uint32_t li, MxRegs& r) {
  gemv_load<FS>(pay_r, lw_r, fs_r, key, pay, leaf, li, r.w, r.ob, r.lw0, r.lw1, r.fs0, r.fs1);
  if constexpr (!FS) r.fs0 = r.fs1 = 0.0f;
}

// Quad lane T's value (DPP quad_perm broadcast within each group of 4 lanes).
template <int T>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, T * 0x55, 0xF, 0xF, false);
}

// The staged X of a block: per split (hi, lo) the f16 rows (2 bytes per row) and the f16 4-row
// sums (2 bytes per 4 rows); split 1's arrays start 64 bytes past a multiple of 128, so that the
// two splits of one group of rows sit in different halves of the 32 LDS banks. A lane reads
// split lane & 1.
constexpr int kMxSplitPad = 64;
__host__ __device__ constexpr int mx_rows_stride(int kc) { return 2 * kc + kMxSplitPad; }
__host__ __device__ constexpr int mx_sums_stride(int kc) { return kc / 2 + kMxSplitPad; }

// Chunk T's leaf word (word 1: a 4x4 chunk's second leaf), 0 (row 0, scale 0) for a chunk past
// the slot's count, whose word may be another bucket's, of any leaf size. Pad leaves' words hold
// no scale and no row.
template <int T, int H>
__device__ __forceinline__ uint32_t mx_word(const MxRegs& r, bool on) {
  const uint32_t w = quad_bcast<T>(H ? r.lw1 : r.lw0);
  return on ? w : 0u;
}

// A leaf's scale from its (masked) word: the bf16 in its high half, or the fp32 scale (0 for pad
// leaves).
template <bool FS, int T, int H>
__device__ __forceinline__ float mx_scale(const MxRegs& r, bool on, uint32_t lw) {
  if constexpr (FS) {
    const float f = __uint_as_float(quad_bcast<T>(__float_as_uint(H ? r.fs1 : r.fs0)));
    return on ? f : 0.0f;
  } else {
    return __uint_as_float(lw & 0xFFFF0000u);
  }
}

struct MxX {
  const char* xr;        // this lane's split of the rows
  const char* xs;        // and of the 4-row sums
};

// Chunk T of a lane's step for leaf sizes of 8 or more: rows 8 (T & RBM) of its leaf.
template <int S, int P, bool FS, int T>
__device__ __forceinline__ void mx_chunk8(const MxRegs& r, const MxX& x, const MxK<P == 16 ? 8 : P>& k,
                                          f16x4_t bias, float& acc) {
  constexpr int W = P == 16 ? 8 : P;
  constexpr int LS = S == 32 ? 5 : S == 16 ? 4 : 3;
  constexpr int RBM = (1 << (LS - 3)) - 1;
  const bool on = (uint32_t)T < r.nv;
  const uint32_t lw = mx_word<T, 0>(r, on);
  const uint32_t row4 = lw & 0x3FFu;
  const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(x.xr + row4 * 8 + 16 * (T & RBM));   // rows 0-7
  const uint32_t sv = *reinterpret_cast<const uint32_t*>(x.xs + row4 * 2 + 4 * (T & RBM));  // two 4-row sums
  const float s = mx_scale<FS, T, 0>(r, on, lw);
  const f16x4_t a0 = __builtin_bit_cast(f16x4_t, u32x2_t{xv.x, xv.y});
  const f16x4_t a1 = __builtin_bit_cast(f16x4_t, u32x2_t{xv.z, xv.w});
  const f16x4_t as = __builtin_bit_cast(f16x4_t, u32x2_t{sv, 0u});
  const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t d = mx_mfma(a0, mx_b<W, T, 0, 0>(r.w, k), z);
  d = mx_mfma(a1, mx_b<W, T, 1, 0>(r.w, k), d);
  if constexpr (P == 16) {
    // sum x' u = 256 sum x' (v_hi - 256) + sum x' (v_lo - 256), q = u - 2^15: all of the bias
    // goes with the high bytes
    f32x4_t e = mx_mfma(a0, mx_b<8, T, 0, 8>(r.w, k), z);
    e = mx_mfma(a1, mx_b<8, T, 1, 8>(r.w, k), e);
    e = mx_mfma(as, bias, e);
    acc = __builtin_fmaf(s, __builtin_fmaf(256.0f, e[0] + e[1], d[0] + d[1]), acc);
  } else {
    d = mx_mfma(as, bias, d);
    acc = __builtin_fmaf(s, d[0] + d[1], acc);
  }
}

// Chunk T of a lane's step for 4x4 leaves: its leaves (rows 0-3 and 4-7) at any rows of the unit.
template <int P, bool FS, int T>
__device__ __forceinline__ void mx_chunk4(const MxRegs& r, const MxX& x, const MxK<P == 16 ? 8 : P>& k,
                                          f16x4_t bias, float& acc) {
  constexpr int W = P == 16 ? 8 : P;
  const bool on = (uint32_t)T < r.nv;
  const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t lw = h ? mx_word<T, 1>(r, on) : mx_word<T, 0>(r, on);
    const uint32_t row4 = lw & 0x3FFu;
    const f16x4_t a = __builtin_bit_cast(f16x4_t, *reinterpret_cast<const u32x2_t*>(x.xr + row4 * 8));
    const uint32_t sv = *reinterpret_cast<const uint16_t*>(x.xs + row4 * 2);
    const f16x4_t as = __builtin_bit_cast(f16x4_t, u32x2_t{sv, 0u});
    const float s = h ? mx_scale<FS, T, 1>(r, on, lw) : mx_scale<FS, T, 0>(r, on, lw);
    f32x4_t d = mx_mfma(a, h ? mx_b<W, T, 1, 0>(r.w, k) : mx_b<W, T, 0, 0>(r.w, k), z);
    if constexpr (P == 16) {
      f32x4_t e = mx_mfma(a, h ? mx_b<8, T, 1, 8>(r.w, k) : mx_b<8, T, 0, 8>(r.w, k), z);
      e = mx_mfma(as, bias, e);
      acc = __builtin_fmaf(s, __builtin_fmaf(256.0f, e[0] + e[1], d[0] + d[1]), acc);
    } else {
      d = mx_mfma(as, bias, d);
      acc = __builtin_fmaf(s, d[0] + d[1], acc);
    }
  }
}

// A lane's whole step of kind (S, P): its quad's four chunks.
template <int S, int P, bool FS>
__device__ __forceinline__ void mx_step(const MxRegs& r, const MxX& x, float& acc) {
  constexpr int W = P == 16 ? 8 : P;
  const MxK<W> k;
  if constexpr (S == 4) {
    const f16x4_t bias = P == 16 ? mx_bias<8, 129, 1>() : mx_bias<W, (1 << (P - 1)), 1>();
    mx_chunk4<P, FS, 0>(r, x, k, bias, acc);
    mx_chunk4<P, FS, 1>(r, x, k, bias, acc);
    mx_chunk4<P, FS, 2>(r, x, k, bias, acc);
    mx_chunk4<P, FS, 3>(r, x, k, bias, acc);
  } else {
    const f16x4_t bias = P == 16 ? mx_bias<8, 129, 2>() : mx_bias<W, (1 << (P - 1)), 2>();
    mx_chunk8<S, P, FS, 0>(r, x, k, bias, acc);
    mx_chunk8<S, P, FS, 1>(r, x, k, bias, acc);
    mx_chunk8<S, P, FS, 2>(r, x, k, bias, acc);
    mx_chunk8<S, P, FS, 3>(r, x, k, bias, acc);
  }
}

// LDS of a block (bytes): the split X rows and 4-row sums, the cross-wave reduction, the wave
// maxima of |x| and, with the LDS gather, one whole X row.
__host__ __device__ constexpr size_t gemv_mx_lds_bytes(int kc, int nw, bool gather, int K) {
  return (size_t)2 * mx_rows_stride(kc) + (size_t)2 * mx_sums_stride(kc) + (size_t)nw * kStepGroups * kGroup * 4 +
         (size_t)nw * 4 + (gather ? (size_t)4 * K : 0);
}

// Codes of chunk t (0..3) of a quad whose four lanes' dwords start at q (P dwords each), as
// floats q = u - 2^(P-1) in the panel stream's chunk code order (the dequantizer's input).
template <int S, int P, int T>
__device__ __forceinline__ void mx_codes_t(const uint32_t* q, float (&out)[32]) {
  constexpr int W = P == 16 ? 8 : P;
  constexpr float off = (float)(1 << (P - 1)), beta = (float)(1 << W);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x16_t w = {};
#pragma unroll
    for (int k = 0; k < P; ++k) w[k] = q[j * P + k];
    const MxK<W> kw;
    const uint32_t ops[4] = {mx_op<W, 4 * T, 0>(w, kw), mx_op<W, 4 * T + 1, 0>(w, kw), mx_op<W, 4 * T + 2, 0>(w, kw),
                             mx_op<W, 4 * T + 3, 0>(w, kw)};
    uint32_t ops_hi[4] = {0u, 0u, 0u, 0u};
    if constexpr (P == 16) {
      ops_hi[0] = mx_op<8, 4 * T, 8>(w, kw);
      ops_hi[1] = mx_op<8, 4 * T + 1, 8>(w, kw);
      ops_hi[2] = mx_op<8, 4 * T + 2, 8>(w, kw);
      ops_hi[3] = mx_op<8, 4 * T + 3, 8>(w, kw);
    }
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      const uint32_t lo = ops[o], hi = ops_hi[o];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int r = 2 * o + half;                   // chunk row
        const int ci = S == 4 ? 16 * (r / 4) + 4 * j + r % 4 : 8 * j + r;
        float u = (float)__builtin_bit_cast(_Float16, (uint16_t)(lo >> (16 * half))) - beta;
        if constexpr (P == 16) u += 256.0f * ((float)__builtin_bit_cast(_Float16, (uint16_t)(hi >> (16 * half))) - beta);
        out[ci] = u - off;
      }
    }
  }
}

template <int S, int P>
__device__ __forceinline__ void mx_codes(const uint32_t* q, uint32_t t, float (&out)[32]) {
  switch (t) {
    case 0: mx_codes_t<S, P, 0>(q, out); break;
    case 1: mx_codes_t<S, P, 1>(q, out); break;
    case 2: mx_codes_t<S, P, 2>(q, out); break;
    default: mx_codes_t<S, P, 3>(q, out); break;
  }
}

// One decode block over an mx stream (one X row: blockIdx.y). Block id, unit mapping, waves,
// record order and the X gather are those of gemv_block; see the comment at the top of this file
// for the arithmetic.
template <bool FS, bool LG, int NW, int KC>
__device__ __forceinline__ void gemv_block_mx(const mtc_stream_desc& d, const int bid, const float* __restrict__ X,
                                              int64_t ldx, float* __restrict__ Y, int64_t ldy, int M,
                                              float* __restrict__ part, uint32_t* __restrict__ counters,
                                              const bool lg = true) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int W = NW, T = 64 * W, BPU = kGemvBlocksPerUnit;
  const int kc = d.chunk_rows;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_units = d.n_panels * d.n_chunks;
  const int xcd = bid % kXcds, slot = bid / kXcds;
  const int u = (slot / BPU) * kXcds + xcd;
  if (u >= n_units) return;                           // padding block of the XCD mapping
  const int cb = slot % BPU;
  const int m = blockIdx.y;                           // the X row
  const int panel = u / d.n_chunks, chunk = u - panel * d.n_chunks;
  const int kb = chunk * kc;
  const int rows = min(kc, d.K - kb);

  char* lds = reinterpret_cast<char*>(smem);
  const int rs = mx_rows_stride(kc), ss = mx_sums_stride(kc);
  char* xr_l = lds;                                   // rows, split 0 at 0, split 1 at rs
  char* xs_l = xr_l + 2 * rs;                         // 4-row sums, split 0 at 0, split 1 at ss
  float* red = reinterpret_cast<float*>(xs_l + 2 * ss);   // [waves][4 slots][1][4]
  float* wmax = red + W * kStepGroups * kGroup;       // [waves] max |x|
  float* xraw = wmax + W;                             // [K] one whole X row (LDS gather only)

  const ci32p hdr = (ci32p)(d.unit_hdr + kUnitHdr * u);
  static_assert(KC % T == 0, "the X staging loops cover KC rows");
  constexpr int XG = (KC + 4 * T - 1) / (4 * T);
  constexpr int XR = KC / T;
  constexpr int PF = gemv_prefetch(NW);
  const bool perm = d.row_perm != nullptr;
  const bool lds_gather = LG && lg;
  const float* xrow = X + (int64_t)min(m, M - 1) * ldx;
  const bool mv = m < M;
  int4 kk[XG];
#pragma unroll
  for (int i = 0; i < XG; ++i) {
    const int r = 4 * (i * T + tid);
    if (perm && r < rows) {
      kk[i] = *reinterpret_cast<const int4*>(d.row_perm + kb + r);
    } else {
      kk[i] = make_int4(kb + r, kb + r + 1, kb + r + 2, kb + r + 3);
    }
  }
  float xw[XR];
  if (lds_gather) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      const int k = i * T + tid;
      xw[i] = (k < d.K && mv) ? xrow[k] : 0.0f;
    }
  }

  const int F = d.fixed_steps;
  const int blk = u * BPU + cb;
  const uint32_t null_rec = (uint32_t)(d.n_panels * d.n_chunks * BPU) * (uint32_t)F;
  const int g = lane / kStepLanes, li = lane % kStepLanes;
  const __amdgpu_buffer_rsrc_t rec_r = buffer_of(d.steps, d.n_steps * kStepWords * 4);
  const __amdgpu_buffer_rsrc_t pay_r = buffer_of(d.payload, d.payload_dwords * 4);
  const __amdgpu_buffer_rsrc_t lw_r = buffer_of(d.leaf_word, d.n_leaves * 4);
  const __amdgpu_buffer_rsrc_t fs_r =
      buffer_of(FS ? static_cast<const void*>(d.leaf_scale) : static_cast<const void*>(d.leaf_word), d.n_leaves * 4);
  const uint32_t pay0 = (uint32_t)hdr[0], leaf0 = (uint32_t)hdr[2];
  auto slot_of = [&](uint32_t r) __attribute__((always_inline)) { return record_slot(rec_r, r, g); };
  auto fetch = [&](const u32x2_t f, MxRegs& r) __attribute__((always_inline)) {
    r.key = record_key(f.y);
    r.live = (__builtin_amdgcn_readfirstlane(f.y) >> 8) != 0u;
    const uint32_t cnt = record_count(f.y, g), q0 = 4u * (uint32_t)(li >> 2);
    r.nv = cnt > q0 ? cnt - q0 : 0u;                  // chunks of this lane's quad in the step
    mx_load<FS>(pay_r, lw_r, fs_r, r.key, pay0 + ((f.x & 0xFFFFu) << 2), leaf0 + (f.x >> 16), (uint32_t)li, r);
  };

  MxRegs r0, r1, r2;
  {
    auto fixed = [&](int k) __attribute__((always_inline)) {
      const int i = wave + k * W;
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
    asm volatile("" ::"s"(pay0), "s"(leaf0));
#pragma unroll
    for (int i = 0; i < XG; ++i) asm volatile("" ::"v"(kk[i].x));
    if (lds_gather) {
#pragma unroll
      for (int i = 0; i < XR; ++i) asm volatile("" ::"v"(xw[i]));
    }
    fetch(f0, r0);
    if constexpr (PF >= 2) fetch(f1, r1);
    if constexpr (PF >= 3) fetch(f2, r2);
  }

  // ---- X: the unit's rows (gathered), max |x| over the block for the prescale, then the
  //      split rows and 4-row sums. With the LDS gather the maximum is the whole row's. ----
  float xmax = 0.0f;
  float4 xv[XG];
  if (lds_gather) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      const int k = i * T + tid;
      if (k < d.K) xraw[k] = xw[i];
      xmax = fmaxf(xmax, fabsf(xw[i]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < XG; ++i) {
      const int r = 4 * (i * T + tid);
      xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (r < rows && mv) xv[i] = make_float4(xrow[kk[i].x], xrow[kk[i].y], xrow[kk[i].z], xrow[kk[i].w]);
      xmax = fmaxf(xmax, fmaxf(fmaxf(fabsf(xv[i].x), fabsf(xv[i].y)), fmaxf(fabsf(xv[i].z), fabsf(xv[i].w))));
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) xmax = fmaxf(xmax, __shfl_xor(xmax, o, 64));
  if (lane == 0) wmax[wave] = xmax;
  lds_barrier();
  float bmax = 0.0f;
#pragma unroll
  for (int w2 = 0; w2 < W; ++w2) bmax = fmaxf(bmax, wmax[w2]);
  int ex = 0;
  (void)frexpf(bmax, &ex);                            // bmax < 2^ex
  const float xscale = ldexpf(1.0f, 13 - ex);         // |x'| < 2^13, 4-row sums < 2^15
  if (lds_gather) {
#pragma unroll
    for (int i = 0; i < XG; ++i) {
      const int r = 4 * (i * T + tid);
      xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (r < rows && mv) xv[i] = make_float4(xraw[kk[i].x], xraw[kk[i].y], xraw[kk[i].z], xraw[kk[i].w]);
    }
  }
#pragma unroll
  for (int i = 0; i < XG; ++i) {
    const int r = 4 * (i * T + tid);
    if (i * 4 * T < kc && r < kc) {
      const float a[4] = {xv[i].x * xscale, xv[i].y * xscale, xv[i].z * xscale, xv[i].w * xscale};
      _Float16 hi[4], lo[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        hi[k] = (_Float16)a[k];
        lo[k] = (_Float16)(a[k] - (float)hi[k]);
      }
      const float s4 = (a[0] + a[1]) + (a[2] + a[3]);
      const _Float16 sh = (_Float16)s4, sl = (_Float16)(s4 - (float)sh);
      *reinterpret_cast<f16x4_t*>(xr_l + 2 * r) = f16x4_t{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<f16x4_t*>(xr_l + rs + 2 * r) = f16x4_t{lo[0], lo[1], lo[2], lo[3]};
      *reinterpret_cast<_Float16*>(xs_l + (r >> 1)) = sh;
      *reinterpret_cast<_Float16*>(xs_l + ss + (r >> 1)) = sl;
    }
  }
  lds_barrier();                                      // payload loads stay in flight
  const int sp = lane & 1;                            // this lane's split (A rows 0, 1; 2, 3 repeat)
  const MxX xx{xr_l + rs * sp, xs_l + ss * sp};

  float acc = 0.0f;
  // A record runs on every lane (the MFMA blocks of idle quads add scale 0 times their sums),
  // so the matrix-core instructions never sit under a divergent branch.
  auto compute = [&](const MxRegs& cur) __attribute__((always_inline)) {
    if (cur.live) {
      const uint32_t key = cur.key;
      switch (key) {
#define MTC_CASE(S, P) \
  case MTC_BUCKET_KEY(S, P): \
    if constexpr (P == 16) { \
      MxRegs t16 = cur; \
      t16.w = gemv_load_p16_tail(pay_r, cur.w, cur.ob); \
      mx_step<S, P, FS>(t16, xx, acc); \
    } else { \
      mx_step<S, P, FS>(cur, xx, acc); \
    } \
    break;
        MTC_FOR_EACH_BUCKET(MTC_CASE)
#undef MTC_CASE
        default: break;
      }
    }
  };
  const int nrec = hdr[28 + 2 * cb];
  const uint32_t ovf = (uint32_t)hdr[27 + 2 * cb];
  auto rec = [&](int i) __attribute__((always_inline)) {
    return i < F ? (uint32_t)(blk * F + i) : ovf + (uint32_t)(i - F);
  };
  int i = wave + PF * W;
  compute(r0);
  u32x2_t nxt = {};
  if (i < nrec) nxt = slot_of(rec(i));
  if constexpr (PF >= 2) compute(r1);
  if constexpr (PF >= 3) compute(r2);
  for (; i < nrec; i += W) {
    fetch(nxt, r0);
    if (i + W < nrec) nxt = slot_of(rec(i + W));
    compute(r0);
  }

  // ---- reduce: undo the prescale, the quads of each slot (lanes j, j + 4, j + 8, j + 12),
  //      then the block's waves ----
  acc *= ldexpf(1.0f, ex - 13);
  acc += row_shr<4>(acc);
  acc += row_shr<8>(acc);
  if (li >= kStepLanes - 4) red[(wave * kStepGroups + g) * kGroup + (li & 3)] = acc;
  __syncthreads();
  gemv_store<1, W, 1>(d, red, u, cb, Y, ldy, M, part, counters);
}
