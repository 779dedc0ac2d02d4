// Device-side building blocks shared by the BCJR / Viterbi kernels (gfx950).
//
// Trellis geometry (the reference's bitshift trellis, src/bcjr/forward_backward.py:62-86):
//   S  = 2^L states, R = 2^kV branches per state, NT = 2^(L-kV) reduced states,
//   NB = NT / R butterflies.
//   Butterfly u (0 <= u < NB) owns the R*R states  s(p, r) = p*NT + R*u + r.
//   Forward (alpha) direction: inputs  m_{t-1}(p*NB + u)  (p = 0..R-1),
//                              outputs m_t(R*u + r)       (r = 0..R-1),
//     because alpha_t(s) = ll_t(s) + m_{t-1}(s >> kV) and
//     m_t(j) = LSE_p alpha_t(p*NT + j).
//   Backward (beta) direction is the transpose: inputs n_t(R*u + c), outputs
//     n_{t-1}(p*NB + u), because beta_t(s) = n_t(s mod NT) and
//     n_{t-1}(j) = LSE_c [ll_t(R*j + c) + beta_t(R*j + c)].
//   A thread keeps the same butterflies for every step ("constant geometry"),
//   so state codewords can stay in registers; the reduced state vector moves
//   between threads through LDS once per step.
//
// Log-domain values are kept in base 2 (v_exp_f32 / v_log_f32 are exp2 / log2):
//   ll2_t(s) = -(c(s) - w_t)^2 * log2(e) / T = -d^2, d = (c - w) * sqrt(log2(e)/T).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>
#include <climits>

namespace bcjr {

// CODE_HYB_COL is HYB with its LUT staged for the column walk (hyb_col_base);
// the soft kernels take it at L = 16, kV = 4, 3 <= Q <= 9.  It never crosses the
// C ABI.
enum { CODE_TABLE = 0, CODE_1MAD = 1, CODE_3INST = 2, CODE_HYB = 3, CODE_HYB_COL = 4 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr double kLn2 = 0.6931471805599453;
constexpr int kMaxWaves = 16;

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---------------------------------------------------------------------------
// Codeword generators.  The "exact" forms are bit-identical to the reference
// (src/codes/ref.py:33-41 for 1MAD, :76-91 for 3INST, src/qat/ste.py:376-392 for
// HYB); they are used wherever a codeword is computed once and cached, and by
// the Viterbi path.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int mad1_bytesum_centered(uint32_t s) {
  const uint32_t x = 34038481u * s + 76625530u;
  // v_sad_u8 with a zero operand sums the four bytes.
  return (int)__builtin_amdgcn_sad_u8(x, 0u, 0u) - 510;
}

__device__ __forceinline__ float code_1mad_exact(uint32_t s) {
  return __fdiv_rn((float)mad1_bytesum_centered(s), 147.8f);
}

__device__ __forceinline__ float code_3inst(uint32_t s) {
  const uint32_t x = 89226354u * s + 64248484u;
  const uint32_t y = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;  // fp16(0.922) = 0x3B60 per half
  const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(y & 0xFFFFu));
  const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(y >> 16));
  // Both halves have exponents in [2^-3, 2^1): their float32 sum is exact.
  const float h = (float)lo + (float)hi;
  return h * (float)(1.0 / 1.2447);
}

__device__ __forceinline__ void code_hyb(uint32_t s, const float* lut, int Q, float& c0, float& c1) {
  // s < 2^16 (L <= 16): the 24-bit multiply-add is exact (v_mad_u32_u24, full rate)
  const uint32_t x = __umul24(s, s) + s;
  const uint32_t idx = (x >> (15 - Q)) & ((1u << Q) - 1u);
  c0 = lut[2 * idx];
  const float b = lut[2 * idx + 1];
  c1 = (x & 0x8000u) ? -b : b;
}

// The same codeword from a signed LUT: 2^(Q+1) float2 entries, entry i holding
// (lut[i mod 2^Q].x, +-lut[i mod 2^Q].y) with the minus sign where bit Q of i is
// set.  Bits [15-Q, 16) of x are the index and the sign bit together, so one
// bit-field extract replaces the index mask and the sign select.
__device__ __forceinline__ void code_hyb_signed(uint32_t s, const float2* lut2s, int Q, float& c0, float& c1) {
  const uint32_t x = __umul24(s, s) + s;
  const float2 v = lut2s[(x >> (15 - Q)) & ((2u << Q) - 1u)];
  c0 = v.x;
  c1 = v.y;
}

// Fills a signed LUT (code_hyb_signed) from the (2^Q, 2) table, threads tid of nthr.
__device__ __forceinline__ void stage_hyb_signed(float2* dst, const float* table, int Q, int tid, int nthr) {
  const int n = 2 << Q, mask = (1 << Q) - 1;
  for (int i = tid; i < n; i += nthr) {
    const int e = i & mask;
    const float y = table[2 * e + 1];
    dst[i] = make_float2(table[2 * e], (i >> Q) ? -y : y);
  }
}

// Column walk of the HYB LUT (L = 16, kV = 4, 3 <= Q <= 9).  State
// s = p * 4096 + r (p < 16, r < 4096) has x = s^2 + s = x(r) + 2^12 * p * (2r + 1)
// (mod 2^16): p moves only bits [12, 16) of x.  The LUT index, bits [15-Q, 16) of
// x, splits into a column, bits [15-Q, 12), fixed by r, and a row, bits [12, 16)
// (its top bit the sign bit), which steps by 2r + 1 (odd, so every row once) per
// unit of p.  The signed LUT is staged as 32 rows of 64 float2 (512 bytes a row),
// rows 16..31 repeating rows 0..15, so state s is the float2 at byte
//   hyb_col_base(r) + hyb_col_step(p, r mod 8)
// without a wrap: a per-lane base per butterfly output and a uniform step per p,
// in place of the multiply, field extract and address arithmetic of each state.

__device__ __forceinline__ uint32_t hyb_col_base(uint32_t r, int Q) {
  const uint32_t x = __umul24(r, r) + r;
  return (((x >> (15 - Q)) & ((1u << (Q - 3)) - 1u)) << 3) | (((x >> 12) & 15u) << 9);
}

// 2r + 1 mod 16 depends on r mod 8 only, so the step is uniform when r is a
// butterfly's output index (state R*u + r, R = 16).
__device__ __forceinline__ uint32_t hyb_col_step(int p, int r) {
  return ((uint32_t)(p * (2 * r + 1)) & 15u) << 9;
}

__device__ __forceinline__ float2 hyb_col_read(const unsigned char* lutb, uint32_t off) {
  return *reinterpret_cast<const float2*>(lutb + off);
}

// Butterfly of thread tid in the column-walk soft kernels (256 threads, one
// 16-state butterfly each).  The LUT column of state 16u + c is bits [6, 12) of
// x = s^2 + s for Q = 9 (the reference's LUT).  Over each coset of span(bits
// 2..7 of u) those columns are all 64 distinct, for every c, so a wave owns one
// coset: u takes tid's bits 0..5 as its bits 2..7 and the wave index as its bits
// 0, 1.  Then a half-wave's 8-byte LUT reads hit 32 distinct banks and a wave's
// 4-byte reads of a per-step table in the LUT's layout 64 distinct banks
// (checked in tests/test_capi_cpu.py).  (A smaller Q has fewer columns.)
__host__ __device__ constexpr uint32_t col_walk_unit(uint32_t tid) {
  return ((tid >> 6) & 3u) | ((tid & 63u) << 2);
}

// LDS layout of the column-walk forward's one state vector: with the rotation of
// step t applied, x = rotr(j, rho_t), reduced state j sits at element
// col_walk_state_el(x).  Under col_walk_unit, every 32-bit read (64 lanes, banks
// mod 64) and write (32 lanes, mod 32) of x = rotr(k*256 + u, rho) is
// conflict-free, for k < 16 and rho = 0, 4, 8.  Linear, so the element of
// k*256 + u is that of u XOR that of k*256.
__host__ __device__ constexpr uint32_t col_walk_state_el(uint32_t x) {
  return x ^ ((x >> 4) & 3u) ^ ((x >> 6) & 63u) ^ ((x >> 7) & 31u);
}

// Any state from the column-walk LUT (rows 0..15).
__device__ __forceinline__ void code_hyb_col(uint32_t s, const float2* lut2c, int Q, float& c0, float& c1) {
  const uint32_t x = __umul24(s, s) + s;
  const float2 v = lut2c[(((x >> 12) & 15u) << 6) | ((x >> (15 - Q)) & ((1u << (Q - 3)) - 1u))];
  c0 = v.x;
  c1 = v.y;
}

// Fills the column-walk LUT from the (2^Q, 2) table: entry (row, col) is signed
// entry col + 2^(Q-3) * (row mod 16); columns past 2^(Q-3) are never read.
__device__ __forceinline__ void stage_hyb_col(float2* dst, const float* table, int Q, int tid, int nthr) {
  const int ncol = 1 << (Q - 3), mask = (1 << Q) - 1;
  for (int k = tid; k < 32 * 64; k += nthr) {
    const int col = k & 63, i = col + ncol * ((k >> 6) & 15);
    float2 v = make_float2(0.0f, 0.0f);
    if (col < ncol) {
      const int e = i & mask;
      const float y = table[2 * e + 1];
      v = make_float2(table[2 * e], (i >> Q) ? -y : y);
    }
    dst[k] = v;
  }
}

// code_hyb_signed from 2^rep interleaved copies of the signed LUT in LDS: entry
// i of copy k is the float2 at i * 2^rep + k, so the lanes reading one copy
// spread over the LDS banks instead of all 64 lanes gathering from one 4 KiB
// table (about 5-way bank conflicts for random 8-byte reads).
__device__ __forceinline__ void code_hyb_signed_rep(uint32_t s, const float2* lut2s, int Q, int rep,
                                                    uint32_t copy, float& c0, float& c1) {
  const uint32_t x = __umul24(s, s) + s;
  const float2 v = lut2s[(((x >> (15 - Q)) & ((2u << Q) - 1u)) << rep) | copy];
  c0 = v.x;
  c1 = v.y;
}

// c(s) for the soft kernels.  `table` is the global (S, V) codebook for
// CODE_TABLE; `lut` the LDS copy of the HYB LUT.
template <int CODE, int V>
__device__ __forceinline__ void codeword(uint32_t s, const float* __restrict__ table,
                                         const float* lut, int Q, float (&c)[V]) {
  if constexpr (CODE == CODE_TABLE) {
    if constexpr (V == 1) {
      c[0] = table[s];
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) c[v] = table[(size_t)s * V + v];
    }
  } else if constexpr (CODE == CODE_1MAD) {
    static_assert(V == 1, "1MAD is a scalar code");
    c[0] = code_1mad_exact(s);
  } else if constexpr (CODE == CODE_3INST) {
    static_assert(V == 1, "3INST is a scalar code");
    c[0] = code_3inst(s);
  } else {
    static_assert(V == 2, "HYB is a 2-D code");
    code_hyb(s, lut, Q, c[0], c[1]);
  }
}

// ---------------------------------------------------------------------------
// Raw codewords for the soft kernels: c(s) = kSigma * h(s) with h cheap to form.
// The LCG codes hash x(s) = A*s + B; for the butterfly states
// s = p*NT + R*u + c this is x = (A*R*u + B) + A*(p*NT + c): one integer add per
// state on top of a per-butterfly base.  h is exact:
//   1MAD : h = (byte sum of x) - 510   (v_sad_u8 with the -510 in its accumulator)
//   3INST: h = f16(lo) + f16(hi)       (one v_fma_mix_f32; the sum is exact)
// Tables and HYB have kSigma = 1 and h = c.
// ---------------------------------------------------------------------------
template <int CODE> struct CodeTraits {
  static constexpr uint32_t A = 0, B = 0;
  static constexpr float kSigma = 1.0f;
};
template <> struct CodeTraits<CODE_1MAD> {
  static constexpr uint32_t A = 34038481u, B = 76625530u;
  static constexpr float kSigma = 1.0f / 147.8f;
};
template <> struct CodeTraits<CODE_3INST> {
  static constexpr uint32_t A = 89226354u, B = 64248484u;
  static constexpr float kSigma = (float)(1.0 / 1.2447);
};

template <int CODE>
__device__ __forceinline__ float raw_from_hash(uint32_t x) {
  if constexpr (CODE == CODE_1MAD) {
    return (float)(int)__builtin_amdgcn_sad_u8(x, 0u, (uint32_t)-510);
  } else {
    // lo * 1 + hi with f16 sources is one v_fma_mix_f32 (exact: both halves lie
    // in [2^-3, 2) in magnitude).  The 1.0 sits in an SGPR the optimiser cannot
    // see through; a literal 1.0 folds to an add of two converts (three
    // instructions), and v_dot2c needs a zeroed accumulator (two).
    const uint32_t y = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    float one = 1.0f;
    asm("" : "+s"(one));
    const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(y & 0xFFFFu));
    const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(y >> 16));
    return fmaf((float)lo, one, (float)hi);
  }
}

// d = h * ssk + nw for the 3INST code straight from the hash: h is the sum of
// the two f16 halves of y, so d = fma(lo, ssk, fma(hi, ssk, nw)) with f16
// sources, which the compiler forms as two v_fma_mix_f32 (no f32 h is needed).
// Two roundings instead of one: |error| <= 2 ulp(d).
__device__ __forceinline__ float d_3inst(uint32_t x, float ssk, float nw) {
  const uint32_t y = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
  const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(y & 0xFFFFu));
  const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(y >> 16));
  return fmaf((float)lo, ssk, fmaf((float)hi, ssk, nw));
}

// h(s) for state s = p*NT + R*u + c given the per-butterfly hash base
// xu = A*(R*u) + B (LCG codes) or the state index s (tables).
template <int CODE, int V>
__device__ __forceinline__ void raw_codeword(uint32_t xu, uint32_t off, uint32_t s,
                                             const float* __restrict__ table, const float* lut, int Q,
                                             float (&h)[V]) {
  if constexpr (CODE == CODE_1MAD || CODE == CODE_3INST) {
    h[0] = raw_from_hash<CODE>(xu + off);
  } else if constexpr (CODE == CODE_TABLE) {
#pragma unroll
    for (int v = 0; v < V; ++v) h[v] = table[(size_t)s * V + v];
  } else if constexpr (CODE == CODE_HYB_COL) {
    code_hyb_col(s, reinterpret_cast<const float2*>(lut), Q, h[0], h[1]);
  } else {
    code_hyb_signed(s, reinterpret_cast<const float2*>(lut), Q, h[0], h[1]);
  }
}

// Group log-sum-exp.  The R inputs of a butterfly are normalised by their
// maximum, so every term 2^a of a group is <= 1 and, at moderate temperature,
// the group sum needs no per-group maximum: one exp2 per term, no compare or
// subtract.  v_exp_f32 flushes results below 2^-126 to zero, so a group whose
// sum is s loses at most (R - 1) 2^-126 / s of it; a butterfly with a group sum
// below kUnderflow = 2^-100 (loss then under 2^-22 relative) is recomputed
// against the group maxima (exec-masked, rare for T >= kExactBelowT).  Below
// kExactBelowT that fallback would fire in most waves, so sequences with a
// lower temperature use the group maxima throughout.
constexpr float kUnderflow = 0x1p-100f;
constexpr float kExactBelowT = 0.08f;
// The 1024-thread forward's switch point.  Its exact variant hashes every
// codeword (the cache does not fit beside that variant's working set in 128
// VGPRs), so its group-sum variant, recomputes included, stays the faster one
// down to T = 0.045 on Gaussian weights at L = 16 (at 0.05: 45 against 51 ms
// per 4,096 sequences; at 0.04 they are even).
constexpr float kExactBelowTFwd4 = 0.045f;

// Load / store n consecutive floats (16-byte aligned when n % 4 == 0, 8-byte
// aligned when n == 2).
template <int n>
__device__ __forceinline__ void load_vec(const float* src, float* dst) {
  if constexpr (n % 4 == 0) {
#pragma unroll
    for (int i = 0; i < n; i += 4) {
      const float4 v = *reinterpret_cast<const float4*>(src + i);
      dst[i] = v.x;
      dst[i + 1] = v.y;
      dst[i + 2] = v.z;
      dst[i + 3] = v.w;
    }
  } else if constexpr (n == 2) {
    const float2 v = *reinterpret_cast<const float2*>(src);
    dst[0] = v.x;
    dst[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < n; ++i) dst[i] = src[i];
  }
}

template <int n>
__device__ __forceinline__ void store_vec(float* dst, const float* src) {
  if constexpr (n % 4 == 0) {
#pragma unroll
    for (int i = 0; i < n; i += 4)
      *reinterpret_cast<float4*>(dst + i) = make_float4(src[i], src[i + 1], src[i + 2], src[i + 3]);
  } else if constexpr (n == 2) {
    *reinterpret_cast<float2*>(dst) = make_float2(src[0], src[1]);
  } else {
#pragma unroll
    for (int i = 0; i < n; ++i) dst[i] = src[i];
  }
}

// Maximum of a butterfly's R inputs as read from LDS.  fmaxf on a loaded value
// first quiets a possible signalling NaN (one v_max_f32 x, x per operand the
// compiler cannot prove canonical); these values all come out of arithmetic, so
// they never are one, and v_max3_f32 / v_max_f32 take them directly.  A quiet
// NaN operand is skipped, as by fmaxf.
__device__ __forceinline__ float vmax3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float vmax_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// max(m, v[0], ..., v[n-1]) in v_max3_f32 steps, on the raw operands like
// max_of_inputs (none is NaN): the running maximum of a step's outputs.
template <int n>
__device__ __forceinline__ float max_with(float m, const float (&v)[n]) {
  int i = 0;
#pragma unroll
  for (; i + 1 < n; i += 2) m = vmax3_raw(m, v[i], v[i + 1]);
  if (i < n) m = vmax_raw(m, v[i]);
  return m;
}
template <int n>
__device__ __forceinline__ float max_of_inputs(const float (&v)[n]) {
  static_assert(n >= 2, "at least two inputs");
  if constexpr (n == 2) {
    return vmax_raw(v[0], v[1]);
  } else if constexpr (n == 4) {
    return vmax_raw(vmax3_raw(v[0], v[1], v[2]), v[3]);
  } else {
    float m = vmax3_raw(v[0], v[1], v[2]);
#pragma unroll
    for (int i = 3; i + 1 < n; i += 2) m = vmax3_raw(m, v[i], v[i + 1]);
    if constexpr ((n - 3) % 2 == 1) m = vmax_raw(m, v[n - 1]);
    return m;
  }
}

// Returns x unchanged but opaque to the optimiser.  Kernels that recompute
// codewords every step pass their butterfly index through this inside the step
// loop; otherwise loop-invariant code motion hoists all R*R codewords per unit
// out of the N-step loop and the kernel spills.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The same for a float kept in a VGPR.  The rare underflow recompute of a
// butterfly derives its exponents from such a copy of -w_t*sk, so they are
// recomputed there instead of kept live from the fast path across the test.
__device__ __forceinline__ float opaque_f(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The fast path's results exist at this point: nothing of it is sunk past the
// underflow test, so its per-state exponentials are dead at the branch.
__device__ __forceinline__ void materialise_one(float x) { asm volatile("" ::"v"(x)); }
template <typename... Ts>
__device__ __forceinline__ void materialise(Ts... x) {
  (materialise_one(x), ...);
}

// Wave-uniform variant.  The LCG kernels keep A*NT behind it so that
// base + A*(p*NT + c) cannot be refolded into one multiply A*s + B per state.
__device__ __forceinline__ uint32_t opaque_uniform(uint32_t x) {
  asm volatile("" : "+s"(x));
  return x;
}

// ---------------------------------------------------------------------------
// Wave (64-lane) and block reductions.  Blocks are always a whole number of
// waves; threads without work contribute the neutral element.
// ---------------------------------------------------------------------------
// DPP move of v (rows of 16 lanes: quad_perm, row mirrors; or row broadcasts
// under a row mask); rows the mask leaves out read `old`.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_i(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL, ROWS>(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v)));
}

constexpr int kDppSwap1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppSwap2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror
constexpr int kDppBcast15 = 0x142;    // lane 15 of each row to the next row (rows 1, 3: mask 0xA)
constexpr int kDppBcast31 = 0x143;    // lane 31 to rows 2 and 3 (mask 0xC)

// Order-preserving integer key of a float that is not NaN (-inf included):
// signed comparison of keys orders the floats, so maxima reduce with
// v_max_i32, whose DPP forms take the move for free (the float max would
// quiet each DPP operand first).
__device__ __forceinline__ int fkey(float v) {
  const int b = __builtin_bit_cast(int, v);
  return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float fkey_inv(int k) { return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7fffffff)); }

// The 16 lanes of each row end with the row's maximum key.
__device__ __forceinline__ int row_max_key(int k) {
  k = max(k, dpp_i<kDppSwap1>(INT_MIN, k));
  k = max(k, dpp_i<kDppSwap2>(INT_MIN, k));
  k = max(k, dpp_i<kDppHalfMirror>(INT_MIN, k));
  return max(k, dpp_i<kDppMirror>(INT_MIN, k));
}

// Maximum over the wave (v not NaN; -inf for lanes without work), uniform:
// the row maxima, then two row broadcasts leave the wave's in lane 63.
__device__ __forceinline__ float wave_max(float v) {
  int k = row_max_key(fkey(v));
  k = max(k, dpp_i<kDppBcast15, 0xA>(INT_MIN, k));
  k = max(k, dpp_i<kDppBcast31, 0xC>(INT_MIN, k));
  return fkey_inv(__builtin_amdgcn_readlane(k, 63));
}

// Maximum over the kMaxWaves = 16 per-wave entries at w (entries of waves
// that do not exist hold -inf), uniform: every row of a wave reads the 16
// entries and reduces them.
__device__ __forceinline__ float block_max(const float* w) {
  static_assert(kMaxWaves == 16, "one entry per lane of a row");
  const int k = row_max_key(fkey(w[threadIdx.x & 15]));
  return fkey_inv(__builtin_amdgcn_readfirstlane(k));
}

// Sum over the wave, uniform: the row sums (four DPP steps), then row 1 +=
// row 0 and row 3 += row 2, then row 3 += row 1, i.e. (r3 + r2) + (r1 + r0).
// -0 is the identity the rows a broadcast leaves out read.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppSwap1>(0.0f, v);
  v += dpp_f<kDppSwap2>(0.0f, v);
  v += dpp_f<kDppHalfMirror>(0.0f, v);
  v += dpp_f<kDppMirror>(0.0f, v);
  v += dpp_f<kDppBcast15, 0xA>(-0.0f, v);
  v += dpp_f<kDppBcast31, 0xC>(-0.0f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum of the n <= 16 per-wave entries w[0], w[stride], ..., w[(n - 1) stride],
// uniform over the calling wave: every row of 16 lanes reads them (lanes past n
// read 0) and adds them pairwise in four DPP steps.
__device__ __forceinline__ float sum_of_waves(const float* w, int n, int stride) {
  const int l = (int)(threadIdx.x & 15);
  float v = l < n ? w[l * stride] : 0.0f;
  v += dpp_f<kDppSwap1>(0.0f, v);
  v += dpp_f<kDppSwap2>(0.0f, v);
  v += dpp_f<kDppHalfMirror>(0.0f, v);
  v += dpp_f<kDppMirror>(0.0f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// ---------------------------------------------------------------------------
// Kernel parameter blocks (passed by value).
// ---------------------------------------------------------------------------
struct FwdParams {
  const float* seq;    // (B, N, V)
  const float* T;      // (B,) or (1,)
  const float* table;  // (S, V) codebook or (2^Q, 2) LUT
  float* soft;         // (B, N, V)
  float* logZ;         // (B,) or null
  float* ws;           // slots x (N * NT) floats
  float* P_out;        // (B, N, S) marginals, or null (diagnostics)
  float* la_out;       // (B, N, S) log alpha (natural log), or null
  float* lb_out;       // (B, N, S) log beta (natural log), or null
  float* H_out;        // (B, N) marginal entropy in nats, or null (diagnostics)
  long long B;
  int N, L, Q, t_per_seq;
};

// In-place layout of a reduced-state vector in LDS.  Reduced state j of the
// vector after step t sits at element S(rotr(j, rho_t)), rotr over nb = L - kV
// bits and rho_t = kV * (t - 1) mod nb.  Because rotr(R*u + r, kV) = r*NB + u,
// the R inputs of butterfly u at step t and its R outputs occupy the same R
// elements, so each thread updates its butterflies in place with one barrier
// per step.  S XORs up to four higher bit fields (x >> a[i]) & m[i] into the low
// bits (a shift of 31 drops a field); the host picks the fields that keep every
// rotation free of LDS bank conflicts.  S is linear: S(x ^ y) = S(x) ^ S(y).
struct Swizzle {
  int a[4];
  uint32_t m[4];
};

__device__ __forceinline__ uint32_t swizzle(uint32_t x, const Swizzle& s) {
  return x ^ ((x >> s.a[0]) & s.m[0]) ^ ((x >> s.a[1]) & s.m[1]) ^ ((x >> s.a[2]) & s.m[2]) ^
         ((x >> s.a[3]) & s.m[3]);
}

// rotr of an nb-bit value (nb <= 16).
__device__ __forceinline__ uint32_t rotr_bits(uint32_t x, int rho, int nb) {
  return ((x | (x << nb)) >> rho) & ((1u << nb) - 1u);
}

struct BwdParams {
  const float* seq;
  const float* T;
  const float* table;
  const float* g_soft;  // (B, N, V)
  const float* g_logZ;  // (B,) or null
  float* g_seq;         // (B, N, V)
  float* ws;            // slots x (N * 2 * NT) floats
  long long B;
  int N, L, Q, t_per_seq;
  Swizzle swz;          // LDS layout of (m~, mu) and (n~, nu)
};

struct VitParams {
  const float* seq;
  const float* table;
  int32_t* walk;      // (B, N) or null
  int32_t* bits;      // (B, N) or null
  int32_t* start;     // (B,) or null
  float* recon;       // (B, N, V) or null
  float* mse;         // (B,) or null
  uint8_t* packed;    // (B, ceil(N*kV/8)) or null
  uint8_t* ws;        // slots x (N * NT) bytes of backpointers
  // Tail-biting constraint (src/viterbi/encode.py:105-172), when overlap is
  // non-null: s_0 >> (L - ob) == overlap[b] and s_{N-1} mod 2^ob == overlap[b]
  // (ob = overlap_bits, overlap[b] < 2^ob); start[b] = -1 when no walk meets it.
  const int32_t* overlap;  // (B,) or null
  long long B;
  int N, L, Q;
  int overlap_bits;
};

struct DecParams {
  const int32_t* bits;    // (B, N) or null when packed is given
  const uint8_t* packed;  // (B, ceil(N*kV/8)) or null
  const int32_t* start;   // (B,)
  const float* table;     // codebook or HYB LUT (global)
  int32_t* walk;          // (B, N) or null
  float* recon;           // (B, N, V) or null
  long long B;
  int N, L, Q;
};

struct TraceParams {
  const float* seq;    // (B, N, V)
  const float* table;  // codebook or HYB LUT (global)
  float* trace;        // (B, N, 2^L) cumulative costs
  int32_t* backptr;    // (B, N, 2^L) chosen predecessor states
  long long B;
  int N, L, Q;
};

// Bitstream layouts (the values of BCJR_BITS_* in the C ABI).
enum { BITS_FMT_U8 = 0, BITS_FMT_I32 = 1, BITS_FMT_PACKED = 2 };

struct DqParams {
  const int32_t* bits32;  // (B, N) one step per int32, or null
  const uint8_t* bits8;   // (B, N) one step per byte (the reference's payload), or null
  const uint8_t* packed;  // (B, ceil(N*kV/8)) kV bits per step, LSB-first, or null
  const int32_t* start;   // (B,)
  const float* table;     // codebook or HYB LUT (global)
  float* out;             // (m, n) row-major
  long long m, n;
  int N, L, Q, Tx, Ty;
  int tx_shift, ty_shift; // log2 of Tx / Ty when they are powers of two, else -1
  int scale_is_f32;       // scale is a float32 value: c * scale is exact in double, so a
                          // float32 multiply rounds it identically
  double scale;           // the product is rounded once to float32, as numpy does
};

struct CbParams {
  const float* lut;  // HYB LUT or null
  float* out;        // (S, V)
  long long S;
  int Q;
};

}  // namespace bcjr
