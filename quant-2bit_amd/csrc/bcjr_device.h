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
#include <stdint.h>

namespace bcjr {

enum { CODE_TABLE = 0, CODE_1MAD = 1, CODE_3INST = 2, CODE_HYB = 3 };

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
// the Viterbi path.  code_1mad_fast trades the correctly-rounded division for a
// multiply by the reciprocal (<= 1 ulp), for per-cell use in the soft kernels.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int mad1_bytesum_centered(uint32_t s) {
  const uint32_t x = 34038481u * s + 76625530u;
  // v_sad_u8 with a zero operand sums the four bytes.
  return (int)__builtin_amdgcn_sad_u8(x, 0u, 0u) - 510;
}

__device__ __forceinline__ float code_1mad_exact(uint32_t s) {
  return __fdiv_rn((float)mad1_bytesum_centered(s), 147.8f);
}

__device__ __forceinline__ float code_1mad_fast(uint32_t s) {
  return (float)mad1_bytesum_centered(s) * (1.0f / 147.8f);
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
  const uint32_t x = s * s + s;
  const uint32_t idx = (x >> (15 - Q)) & ((1u << Q) - 1u);
  c0 = lut[2 * idx];
  const float b = lut[2 * idx + 1];
  c1 = (x & 0x8000u) ? -b : b;
}

// c(s) for the soft kernels.  `table` is the global (S, V) codebook for
// CODE_TABLE; `lut` the LDS copy of the HYB LUT.
template <int CODE, int V, bool EXACT>
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
    c[0] = EXACT ? code_1mad_exact(s) : code_1mad_fast(s);
  } else if constexpr (CODE == CODE_3INST) {
    static_assert(V == 1, "3INST is a scalar code");
    c[0] = code_3inst(s);
  } else {
    static_assert(V == 2, "HYB is a 2-D code");
    code_hyb(s, lut, Q, c[0], c[1]);
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

// ---------------------------------------------------------------------------
// Wave (64-lane) reductions.  Blocks are always a whole number of waves;
// threads without work contribute the neutral element.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
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
  long long B;
  int N, L, Q, t_per_seq;
};

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
  long long B;
  int N, L, Q;
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

struct CbParams {
  const float* lut;  // HYB LUT or null
  float* out;        // (S, V)
  long long S;
  int Q;
};

}  // namespace bcjr
