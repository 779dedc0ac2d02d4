// Soft forward pass for two-bit steps (kV = 2, V = 1) at L = 14..16, shaped for
// four waves per SIMD.
//
// Same recursions, offsets, underflow handling and outputs as bcjr_fwd_kernel
// (bcjr_fwd.hip; replaces the compute of src/bcjr/forward_backward.py:190-232).
// What differs is the launch shape.  On gfx950 one wave issues VALU work at a
// fraction of the SIMD's rate (an FMA stream of independent chains reaches 33%
// of peak with one wave per SIMD, 62% with two, 79% with four), and the
// 512-thread forward holds two waves per SIMD.  This kernel runs 1024 threads
// (sixteen waves, four per SIMD) with UPT = 2^(L-14) butterflies per thread and
// keeps all 16*UPT of a thread's codewords in VGPRs for the launch, within the
// 128 VGPRs four waves per SIMD allow:
//   * one butterfly at a time (a scheduling barrier between butterflies keeps
//     the working set to one butterfly plus what is in flight);
//   * block-uniform per-step values (offsets, -w_t*sk, K_t) read into SGPRs;
//   * the next butterfly's LDS inputs and the next two butterflies' slot
//     inputs in flight while the current one computes.
//
// A butterfly u owns states p*NT + 4u + r (p, r < 4).  Alpha sweep: inputs
// m~_{t-1}(p*NB + u) (LDS, strided reads), outputs m~_t(4u + r) (one 16-byte LDS
// write); the raw inputs go to the sequence's HBM slot at [t][u].  Beta sweep:
// inputs n~_t(4u + c) (one 16-byte read), outputs n~_{t-1}(p*NB + u); marginal
// P = e * 2^(m~_{t-1}(p*NB+u) + K_t + ...) with the raw alpha inputs read back
// from the slot.  All logs are base 2.
#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace bcjr {

namespace {

__device__ __forceinline__ float uniform_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

// Block-uniform doubles (the running offsets) live in SGPR pairs, not VGPRs.
__device__ __forceinline__ double uniform_d(double x) {
  const uint64_t v = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// f(0) ... f(UPT - 1): unrolled, or as a loop (one unit's registers reused).
template <bool ROLLED, int UPT, typename F>
__device__ __forceinline__ void for_units(F&& f) {
  if constexpr (ROLLED) {
#pragma unroll 1
    for (int i = 0; i < UPT; ++i) f(i);
  } else {
#pragma unroll
    for (int i = 0; i < UPT; ++i) f(i);
  }
}

}  // namespace

template <int CODE, int UPT>
__global__ __launch_bounds__(1024) void bcjr_fwd4_kernel(FwdParams P) {
  constexpr int KV = 2, R = 4, NTHR = 1024;
  constexpr int NB = NTHR * UPT, NT = NB * R;
  static_assert(CODE == CODE_TABLE || CODE == CODE_1MAD || CODE == CODE_3INST, "scalar codes only");
  using CT = CodeTraits<CODE>;

  extern __shared__ __align__(16) unsigned char smem[];
  const int N = P.N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  double* cvec = reinterpret_cast<double*>(smem);                 // N     C_{t-1}
  float* mbuf = reinterpret_cast<float*>(cvec + ((N + 1) & ~1));   // 2*NT  reduced state, double-buffered
  float* wmax = mbuf + 2 * NT;                                     // 2*16  per-wave maxima
  float* wsum = wmax + 2 * kMaxWaves;                              // 16    per-wave sums (log Z)
  int* bflag = reinterpret_cast<int*>(wsum + kMaxWaves);           // 4     input-check flag (one word)
  float* wbuf = wsum + kMaxWaves + 4;                              // N     the sequence
  float* spart = wbuf + N;                                         // 2*16  per-wave soft partials

  // Raw codeword h(s) of state p*NT + 4u + r, u = utid + i*NTHR (utid = tid).
  auto h_of = [&](int utid, int i, int p, int r) -> float {
    const uint32_t s = (uint32_t)(p * NT) + R * (uint32_t)(utid + i * NTHR) + (uint32_t)r;
    if constexpr (CODE == CODE_TABLE) {
      return P.table[s];
    } else {
      return raw_from_hash<CODE>(CT::A * s + CT::B);
    }
  };

  if (tid == 0) *bflag = 0;
  __syncthreads();

  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    float* slot = P.ws + (size_t)blockIdx.x * (size_t)N * NT;
    const float Tb = P.T[P.t_per_seq ? b : 0];
    const float sk = sqrtf(kLog2e / Tb);
    const float ssk = CT::kSigma * sk;
    const float* seqb = P.seq + (size_t)b * N;
    float* softb = P.soft + (size_t)b * N;

    // T must be finite and > 0 and the weights finite, else the outputs are NaN.
    int bad = !(Tb > 0.0f && Tb < INFINITY);
    for (int i = tid; i < N; i += NTHR) {
      const float w = seqb[i];
      wbuf[i] = w;
      bad |= !__builtin_isfinite(w);
    }
    for (int j = tid; j < NT; j += NTHR) mbuf[NT + j] = (float)KV;  // m~_{-1} = log2(R)
    if (tid < 2 * kMaxWaves) wmax[tid] = -INFINITY;
    if (bad) *bflag = 1;
    __syncthreads();
    if (*bflag) {  // uniform: every thread reads the flag after the barrier
      for (int i = tid; i < N; i += NTHR) softb[i] = NAN;
      if (tid == 0 && P.logZ) P.logZ[b] = NAN;
      __syncthreads();
      if (tid == 0) *bflag = 0;
      __syncthreads();
      continue;
    }

    auto sweeps = [&](auto exact_tag) -> double {
      constexpr bool EXACT = decltype(exact_tag)::value;
      // The group-sum variant keeps the thread's 16*UPT codewords in VGPRs for the
      // sequence (formed here, per sequence: the opaque thread index keeps them
      // from being hoisted into a launch-long live range).  The exact-maximum
      // variant (T < kExactBelowTFwd4) forms each codeword where it is used, which
      // leaves its larger working set the registers the cache would hold.
      float hc[EXACT ? 1 : UPT][EXACT ? 1 : R][EXACT ? 1 : R];
      if constexpr (!EXACT) {
        const int ot = opaque(tid);
#pragma unroll
        for (int i = 0; i < UPT; ++i)
#pragma unroll
          for (int p = 0; p < R; ++p)
#pragma unroll
            for (int r = 0; r < R; ++r) hc[i][p][r] = h_of(ot, i, p, r);
      }
      // In the exact variant the thread index is made opaque once per butterfly,
      // so the hashes stay inside the step loop instead of being hoisted.
      int otx = tid;
      auto hv = [&](int i, int p, int r) -> float {
        if constexpr (EXACT) {
          return h_of(otx, i, p, r);
        } else {
          return hc[i][p][r];
        }
      };

      // ------------------------------ alpha sweep ------------------------------
      double C = 0.0;  // C_{t-1}
      for (int t = 0; t < N; ++t) {
        const float* prev = mbuf + ((t + 1) & 1) * NT;
        float* cur = mbuf + (t & 1) * NT;
        const float O = t > 0 ? uniform_f(block_max(wmax + ((t + 1) & 1) * kMaxWaves)) : (float)KV;
        if (tid == 0) cvec[t] = C;
        C = uniform_d(C + (double)O);
        const float nw = uniform_f(-wbuf[t] * sk);
        float* slot_t = slot + (size_t)t * NT;
        float tmax = -INFINITY;
        float mx[R];
#pragma unroll
        for (int p = 0; p < R; ++p) mx[p] = prev[p * NB + tid];
        // Butterflies: unrolled with the cached codewords; the exact variant,
        // which hashes them, runs them as a loop so one butterfly's registers serve all.
        for_units<EXACT, UPT>([&](int i) {
          __builtin_amdgcn_sched_barrier(0);
          const int u = tid + i * NTHR;
          if constexpr (EXACT) otx = opaque(tid);
          float m[R];
#pragma unroll
          for (int p = 0; p < R; ++p) m[p] = mx[p];
          if (i + 1 < UPT) {
#pragma unroll
            for (int p = 0; p < R; ++p) mx[p] = prev[p * NB + u + NTHR];
          }
          store_vec<R>(slot_t + R * u, m);
          const float M = max_of_inputs(m);
#pragma unroll
          for (int p = 0; p < R; ++p) m[p] -= M;
          const float off = M - O;
          float mo[R];
          if constexpr (EXACT) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float a[R];
#pragma unroll
              for (int p = 0; p < R; ++p) {
                const float d = fmaf(hv(i, p, r), ssk, nw);
                a[p] = fmaf(-d, d, m[p]);
              }
              const float Ma = max_of_inputs(a);
              float s = fexp2(a[0] - Ma);
#pragma unroll
              for (int p = 1; p < R; ++p) s += fexp2(a[p] - Ma);
              mo[r] = flog2(s) + (Ma + off);
            }
          } else {
            float sr[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float s = 0.0f;
#pragma unroll
              for (int p = 0; p < R; ++p) {
                const float d = fmaf(hv(i, p, r), ssk, nw);
                const float e = fexp2(fmaf(-d, d, m[p]));
                s = p ? s + e : e;
              }
              sr[r] = s;
            }
            const float smin = fminf(fminf(sr[0], sr[1]), fminf(sr[2], sr[3]));
#pragma unroll
            for (int r = 0; r < R; ++r) mo[r] = flog2(sr[r]) + off;
            materialise(mo[0], mo[1], mo[2], mo[3]);
            if (smin < kUnderflow) {  // a group underflowed: redo the butterfly against the group maxima
              const float nwx = opaque_f(nw);
#pragma unroll
              for (int r = 0; r < R; ++r) {
                float a[R];
#pragma unroll
                for (int p = 0; p < R; ++p) {
                  const float d = fmaf(hv(i, p, r), ssk, nwx);
                  a[p] = fmaf(-d, d, m[p]);
                }
                const float Ma = max_of_inputs(a);
                float s = fexp2(a[0] - Ma);
#pragma unroll
                for (int p = 1; p < R; ++p) s += fexp2(a[p] - Ma);
                mo[r] = flog2(s) + (Ma + off);
              }
            }
          }
          store_vec<R>(cur + R * u, mo);
          tmax = max_with(tmax, mo);
        });
        __builtin_amdgcn_sched_barrier(0);
        tmax = wave_max(tmax);
        if (lane == 0) wmax[(t & 1) * kMaxWaves + wave] = tmax;
        __syncthreads();
      }

      // log2 Z = C_{N-1} + LSE2 over the final reduced state.
      float* fin = mbuf + ((N - 1) & 1) * NT;
      const float Mz = uniform_f(block_max(wmax + ((N - 1) & 1) * kMaxWaves));
      float part = 0.0f;
      for (int j = tid; j < NT; j += NTHR) part += fexp2(fin[j] - Mz);
      part = wave_sum(part);
      if (lane == 0) wsum[wave] = part;
      __syncthreads();
      float Ssum = 0.0f;
#pragma unroll
      for (int w = 0; w < kMaxWaves; ++w) Ssum += wsum[w];
      const double logZ2 = uniform_d(C + (double)Mz + (double)flog2(Ssum));
      for (int j = tid; j < NT; j += NTHR) fin[j] = 0.0f;  // n~_{N-1} = 0
      __syncthreads();

      // ------------------------------ beta sweep -------------------------------
      // Raw alpha inputs come back from the slot two butterflies ahead of their
      // use, across step boundaries (consumption order: t descending, i ascending).
      auto slot_src = [&](int t, int i) { return slot + (size_t)t * NT + R * (tid + i * NTHR); };
      float pa[R], pb[R];
      load_vec<R>(slot_src(N - 1, 0), pa);
      if (UPT > 1) {
        load_vec<R>(slot_src(N - 1, 1), pb);
      } else if (N > 1) {
        load_vec<R>(slot_src(N - 2, 0), pb);
      }
      double D = 0.0;  // D_t
      for (int t = N - 1; t >= 0; --t) {
        const int k = 2 * N - 1 - t;  // buffer parity continues from the alpha sweep
        const float* prev = mbuf + ((k + 1) & 1) * NT;
        float* cur = mbuf + (k & 1) * NT;
        float Qv = 0.0f;
        if (t != N - 1) {
          Qv = uniform_f(block_max(wmax + ((k + 1) & 1) * kMaxWaves));
          if (wave == 0) {  // soft of step t+1 from its per-wave partials
            const float s = sum_of_waves(spart + ((k + 1) & 1) * kMaxWaves, kMaxWaves, 1);
            if (lane == 0) softb[t + 1] = s;
          }
        }
        const float Kt = uniform_f((float)(cvec[t] + D - logZ2));
        const float nw = uniform_f(-wbuf[t] * sk);
        float acc = 0.0f, tmax = -INFINITY;
        float nx[R];
        load_vec<R>(prev + R * tid, nx);
        for_units<EXACT, UPT>([&](int i) {
          __builtin_amdgcn_sched_barrier(0);
          const int u = tid + i * NTHR;
          if constexpr (EXACT) otx = opaque(tid);
          float n[R], pm[R];
#pragma unroll
          for (int c = 0; c < R; ++c) {
            n[c] = nx[c];
            pm[c] = pa[c];
            pa[c] = pb[c];
          }
          {  // fetch the butterfly two ahead
            const int tt = i + 2 < UPT ? t : t - 1 - (i + 2 - UPT) / UPT;
            const int ii = i + 2 < UPT ? i + 2 : (i + 2 - UPT) % UPT;
            if (tt >= 0) load_vec<R>(slot_src(tt, ii), pb);
          }
          if (i + 1 < UPT) load_vec<R>(prev + R * (u + NTHR), nx);
          const float M = max_of_inputs(n);
#pragma unroll
          for (int c = 0; c < R; ++c) n[c] -= M;
          const float kts = Kt + M;
          const float off = M - Qv;
          float no[R], ua = 0.0f;
          if constexpr (EXACT) {
#pragma unroll
            for (int p = 0; p < R; ++p) {
              float y[R];
#pragma unroll
              for (int c = 0; c < R; ++c) {
                const float d = fmaf(hv(i, p, c), ssk, nw);
                y[c] = fmaf(-d, d, n[c]);
              }
              const float My = max_of_inputs(y);
              float s = 0.0f, ec = 0.0f;
#pragma unroll
              for (int c = 0; c < R; ++c) {
                const float e = fexp2(y[c] - My);
                s = c ? s + e : e;
                ec = c ? fmaf(e, hv(i, p, c), ec) : e * hv(i, p, c);
              }
              ua = fmaf(fexp2(pm[p] + kts + My), ec, ua);
              no[p] = flog2(s) + (My + off);
            }
          } else {
            float sp[R];
#pragma unroll
            for (int p = 0; p < R; ++p) {
              float s = 0.0f, ec = 0.0f;
#pragma unroll
              for (int c = 0; c < R; ++c) {
                const float d = fmaf(hv(i, p, c), ssk, nw);
                const float e = fexp2(fmaf(-d, d, n[c]));
                s = c ? s + e : e;
                ec = c ? fmaf(e, hv(i, p, c), ec) : e * hv(i, p, c);
              }
              sp[p] = s;
              const float G = fexp2(pm[p] + kts);
              ua = p ? fmaf(G, ec, ua) : G * ec;
              no[p] = flog2(s) + off;
            }
            const float smin = fminf(fminf(sp[0], sp[1]), fminf(sp[2], sp[3]));
            materialise(no[0], no[1], no[2], no[3]);
            materialise(ua, smin);
            if (smin < kUnderflow) {  // redo the butterfly against the group maxima
              const float nwx = opaque_f(nw);
              ua = 0.0f;
#pragma unroll
              for (int p = 0; p < R; ++p) {
                float y[R];
#pragma unroll
                for (int c = 0; c < R; ++c) {
                  const float d = fmaf(hv(i, p, c), ssk, nwx);
                  y[c] = fmaf(-d, d, n[c]);
                }
                const float My = max_of_inputs(y);
                float s = 0.0f, ec = 0.0f;
#pragma unroll
                for (int c = 0; c < R; ++c) {
                  const float e = fexp2(y[c] - My);
                  s = c ? s + e : e;
                  ec = c ? fmaf(e, hv(i, p, c), ec) : e * hv(i, p, c);
                }
                ua = fmaf(fexp2(pm[p] + kts + My), ec, ua);
                no[p] = flog2(s) + (My + off);
              }
            }
          }
          acc += ua;
#pragma unroll
          for (int p = 0; p < R; ++p) cur[p * NB + u] = no[p];
          tmax = max_with(tmax, no);
        });
        __builtin_amdgcn_sched_barrier(0);
        D = uniform_d(D + (double)Qv);
        acc = wave_sum(acc);
        if (lane == 0) spart[(k & 1) * kMaxWaves + wave] = acc * CT::kSigma;
        tmax = wave_max(tmax);
        if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
        __syncthreads();
      }
      return logZ2;
    };
    const double logZ2 = Tb < kExactBelowTFwd4 ? sweeps(std::true_type{}) : sweeps(std::false_type{});

    // soft of step 0: the last beta step (k = 2N - 1, odd) wrote buffer 1
    if (wave == 0) {
      const float s = sum_of_waves(spart + kMaxWaves, kMaxWaves, 1);
      if (lane == 0) {
        softb[0] = s;
        if (P.logZ) P.logZ[b] = (float)(logZ2 * kLn2);
        *bflag = 0;  // every thread read it after the first barrier
      }
    }
    __syncthreads();
  }
}

const void* fwd4_kernel_ptr(int code, int upt) {
#define BCJR_FWD4_CASE(CODE_, UPT_) \
  if (code == CODE_ && upt == UPT_) return reinterpret_cast<const void*>(&bcjr_fwd4_kernel<CODE_, UPT_>);
  BCJR_FWD4_CASE(CODE_TABLE, 1)
  BCJR_FWD4_CASE(CODE_TABLE, 2)
  BCJR_FWD4_CASE(CODE_TABLE, 4)
  BCJR_FWD4_CASE(CODE_1MAD, 1)
  BCJR_FWD4_CASE(CODE_1MAD, 2)
  BCJR_FWD4_CASE(CODE_1MAD, 4)
  BCJR_FWD4_CASE(CODE_3INST, 1)
  BCJR_FWD4_CASE(CODE_3INST, 2)
  BCJR_FWD4_CASE(CODE_3INST, 4)
#undef BCJR_FWD4_CASE
  return nullptr;
}

}  // namespace bcjr
