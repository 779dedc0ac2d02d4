// Soft forward pass of the BCJR node: soft codewords E_P[c(s_t)] and log Z.
//
// Replaces the compute of bcjr_forward_backward (src/bcjr/forward_backward.py:190-232)
// and the forward of BcjrForwardBackwardMonolithic (src/bcjr/bcjr_monolithic.py:161-189).
//
// One workgroup processes one sequence at a time (grid-stride over sequences) and
// owns one scratch slot of N * NT floats in HBM.
//
// Alpha sweep (t = 0..N-1), butterfly u of step t:
//   mi[p]  = m~_{t-1}(p*NB + u) - O_t            (O_t: max of m~_{t-1}, from the
//                                                  per-wave maxima of step t-1)
//   a[p][r] = mi[p] + ll2_t(p*NT + R*u + r)
//   m~_t(R*u + r) = LSE2_p a[p][r]                 (exact per-group max, exp2/log2)
//   The butterfly's normalised inputs mi[0..R-1] are also written, as one
//   contiguous R-float vector, to slot[t][u]: exactly what the beta sweep needs.
//   True log-alpha: alpha2_t(s) = ll2_t(s) + mi[p] + C_t with C_t = sum_{tau<=t} O_tau.
// log2 Z = C_{N-1} + LSE2_j m~_{N-1}(j).
// Beta sweep (t = N-1..0), same butterfly (transposed data flow):
//   ni[c] = n~_t(R*u + c) - Q_t,  y[p][c] = ni[c] + ll2_t(p*NT + R*u + c),
//   n~_{t-1}(p*NB + u) = M_p + log2(sum_c 2^(y - M_p)),
//   P_t(s) = 2^(y + mi[p] + K_t) with K_t = C_t + Q_t + D_t - log2 Z (D_t: beta offsets),
//   so the marginal costs one multiply per state and one exp2 per group:
//   P = e[p][c] * 2^(M_p + mi[p] + K_t).  soft_t = sum_s P_t(s) c(s).
// Both sweeps normalise by a block-uniform offset every step, so all values stay
// O(1)-O(100) in float32; offsets accumulate in double.
#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace bcjr {

template <int KV, int V, int CODE, int UPT, bool CACHE>
__global__ __launch_bounds__(512) void bcjr_fwd_kernel(FwdParams P) {
  constexpr int R = 1 << KV;
  constexpr int RO = R < 4 ? R : 4;  // outputs per unit
  constexpr int NSUB = R / RO;       // units per butterfly
  static_assert(!CACHE || NSUB == 1, "codeword cache needs whole butterflies per thread");

  extern __shared__ __align__(16) unsigned char smem[];
  const int L = P.L, N = P.N;
  const int NT = 1 << (L - KV);
  const int NB = NT >> KV;
  const int NU = NB * NSUB;
  const int lgNB = L - 2 * KV;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;

  double* cvec = reinterpret_cast<double*>(smem);  // N    C_t
  float* mbuf = reinterpret_cast<float*>(cvec + N);  // 2*NT reduced state, double-buffered
  float* wmax = mbuf + 2 * NT;                       // 2*kMaxWaves
  float* wsum = wmax + 2 * kMaxWaves;                // kMaxWaves
  float* wbuf = wsum + kMaxWaves;                    // N*V   sequence
  float* spart = wbuf + N * V;                       // N*nwaves*V per-wave soft partials
  float* lut = spart + N * nwaves * V;               // HYB LUT

  if constexpr (CODE == CODE_HYB) {
    const int nl = 2 << P.Q;
    for (int i = tid; i < nl; i += nthr) lut[i] = P.table[i];
    __syncthreads();
  }

  float cw[CACHE ? UPT : 1][CACHE ? R : 1][CACHE ? R : 1][V];
  if constexpr (CACHE) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = min(tid + i * nthr, NU - 1);
#pragma unroll
      for (int p = 0; p < R; ++p)
#pragma unroll
        for (int r = 0; r < R; ++r)
          codeword<CODE, V, true>((uint32_t)(p * NT + R * u + r), P.table, lut, P.Q, cw[i][p][r]);
    }
  }

  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    float* slot = P.ws + (size_t)blockIdx.x * (size_t)N * (size_t)NT;
    const float Tb = P.T[P.t_per_seq ? b : 0];
    const float sk = sqrtf(kLog2e / Tb);
    const float* seqb = P.seq + (size_t)b * N * V;
    for (int i = tid; i < N * V; i += nthr) wbuf[i] = seqb[i];
    __syncthreads();

    // ------------------------------ alpha sweep ------------------------------
    double C = 0.0;
    int k = 0;  // step counter across both sweeps: LDS buffer / wmax parity
    for (int t = 0; t < N; ++t, ++k) {
      const float* prev = mbuf + ((k + 1) & 1) * NT;
      float* cur = mbuf + (k & 1) * NT;
      float O = (float)KV;  // m~_{-1} = log2(R) for every j
      if (t > 0) {
        O = -INFINITY;
        for (int w = 0; w < nwaves; ++w) O = fmaxf(O, wmax[((k + 1) & 1) * kMaxWaves + w]);
      }
      C += (double)O;
      if (tid == 0) cvec[t] = C;
      float nw[V];
#pragma unroll
      for (int v = 0; v < V; ++v) nw[v] = -wbuf[t * V + v] * sk;
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int q = tid + i * nthr;
        __builtin_amdgcn_sched_barrier(0);
        if (q < NU) {
          const int u = (CACHE ? q : opaque(q)) & (NB - 1);
          const int sub = q >> lgNB;
          float mi[R];
#pragma unroll
          for (int p = 0; p < R; ++p) mi[p] = t ? prev[p * NB + u] - O : 0.0f;
          if (sub == 0) {
            float* dst = slot + ((size_t)t * NB + u) * R;
#pragma unroll
            for (int p = 0; p < R; ++p) dst[p] = mi[p];
          }
          float mo[RO];
#pragma unroll
          for (int r = 0; r < RO; ++r) {
            const int rr = sub * RO + r;
            float a[R];
#pragma unroll
            for (int p = 0; p < R; ++p) {
              float c[V];
              if constexpr (CACHE) {
#pragma unroll
                for (int v = 0; v < V; ++v) c[v] = cw[i][p][r][v];
              } else {
                codeword<CODE, V, false>((uint32_t)(p * NT + R * u + rr), P.table, lut, P.Q, c);
              }
              float acc = mi[p];
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const float d = fmaf(c[v], sk, nw[v]);
                acc = fmaf(-d, d, acc);
              }
              a[p] = acc;
            }
            float M = a[0];
#pragma unroll
            for (int p = 1; p < R; ++p) M = fmaxf(M, a[p]);
            float ssum = 0.0f;
#pragma unroll
            for (int p = 0; p < R; ++p) ssum += fexp2(a[p] - M);
            mo[r] = M + flog2(ssum);
            tmax = fmaxf(tmax, mo[r]);
          }
          float* o = cur + R * u + sub * RO;
#pragma unroll
          for (int r = 0; r < RO; ++r) o[r] = mo[r];
        }
      }
      tmax = wave_max(tmax);
      if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
      __syncthreads();
    }

    // log2 Z = C_{N-1} + LSE2 over the final reduced state.
    const float* fin = mbuf + ((k + 1) & 1) * NT;
    float Mz = -INFINITY;
    for (int w = 0; w < nwaves; ++w) Mz = fmaxf(Mz, wmax[((k + 1) & 1) * kMaxWaves + w]);
    float part = 0.0f;
    for (int j = tid; j < NT; j += nthr) part += fexp2(fin[j] - Mz);
    part = wave_sum(part);
    if (lane == 0) wsum[wave] = part;
    __syncthreads();
    float Ssum = 0.0f;
    for (int w = 0; w < nwaves; ++w) Ssum += wsum[w];
    const double logZ2 = C + (double)Mz + (double)flog2(Ssum);

    // ------------------------------ beta sweep -------------------------------
    double D = 0.0;
    for (int t = N - 1; t >= 0; --t, ++k) {
      const float* prev = mbuf + ((k + 1) & 1) * NT;
      float* cur = mbuf + (k & 1) * NT;
      float Qv = 0.0f;
      if (t != N - 1) {
        Qv = -INFINITY;
        for (int w = 0; w < nwaves; ++w) Qv = fmaxf(Qv, wmax[((k + 1) & 1) * kMaxWaves + w]);
      }
      const float Kt = (float)(cvec[t] + (double)Qv + D - logZ2);
      float nw[V];
#pragma unroll
      for (int v = 0; v < V; ++v) nw[v] = -wbuf[t * V + v] * sk;
      float acc[V];
#pragma unroll
      for (int v = 0; v < V; ++v) acc[v] = 0.0f;
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int q = tid + i * nthr;
        __builtin_amdgcn_sched_barrier(0);
        if (q < NU) {
          const int u = (CACHE ? q : opaque(q)) & (NB - 1);
          const int sub = q >> lgNB;
          float ni[R];
#pragma unroll
          for (int c = 0; c < R; ++c) ni[c] = (t != N - 1) ? prev[R * u + c] - Qv : 0.0f;
          const float* src = slot + ((size_t)t * NB + u) * R + sub * RO;
          float mi[RO];
#pragma unroll
          for (int pp = 0; pp < RO; ++pp) mi[pp] = src[pp];
#pragma unroll
          for (int pp = 0; pp < RO; ++pp) {
            const int p = sub * RO + pp;
            float y[R];
            float cc[R][V];
#pragma unroll
            for (int c = 0; c < R; ++c) {
              if constexpr (CACHE) {
#pragma unroll
                for (int v = 0; v < V; ++v) cc[c][v] = cw[i][pp][c][v];
              } else {
                codeword<CODE, V, false>((uint32_t)(p * NT + R * u + c), P.table, lut, P.Q, cc[c]);
              }
              float yy = ni[c];
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const float d = fmaf(cc[c][v], sk, nw[v]);
                yy = fmaf(-d, d, yy);
              }
              y[c] = yy;
            }
            float M = y[0];
#pragma unroll
            for (int c = 1; c < R; ++c) M = fmaxf(M, y[c]);
            float e[R];
            float ssum = 0.0f;
#pragma unroll
            for (int c = 0; c < R; ++c) {
              e[c] = fexp2(y[c] - M);
              ssum += e[c];
            }
            const float no = M + flog2(ssum);
            const float G = fexp2(M + mi[pp] + Kt);
            if (P.P_out) {  // diagnostics (small B): P, log alpha, log beta in nats
              const float Ct = (float)cvec[t];
              const float Dt = (float)(D + (double)Qv);
              const size_t base = ((size_t)b * N + t) * ((size_t)NT << KV) + (size_t)p * NT + (size_t)R * u;
#pragma unroll
              for (int c = 0; c < R; ++c) {
                P.P_out[base + c] = e[c] * G;
                P.la_out[base + c] = (y[c] - ni[c] + mi[pp] + Ct) * (float)kLn2;
                P.lb_out[base + c] = (ni[c] + Dt) * (float)kLn2;
              }
            }
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float ec = 0.0f;
#pragma unroll
              for (int c = 0; c < R; ++c) ec = fmaf(e[c], cc[c][v], ec);
              acc[v] = fmaf(G, ec, acc[v]);
            }
            cur[p * NB + u] = no;
            tmax = fmaxf(tmax, no);
          }
        }
      }
      D += (double)Qv;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float s = wave_sum(acc[v]);
        if (lane == 0) spart[(t * nwaves + wave) * V + v] = s;
      }
      tmax = wave_max(tmax);
      if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
      __syncthreads();
    }

    float* softb = P.soft + (size_t)b * N * V;
    for (int i = tid; i < N * V; i += nthr) {
      const int t = i / V, v = i - t * V;
      float s = 0.0f;
      for (int w = 0; w < nwaves; ++w) s += spart[(t * nwaves + w) * V + v];
      softb[i] = s;
    }
    if (tid == 0 && P.logZ) P.logZ[b] = (float)(logZ2 * kLn2);
    __syncthreads();
  }
}

#define BCJR_FWD_CASE(KV_, V_, CODE_, UPT_, CACHE_)                                        \
  if (KV == KV_ && V == V_ && code == CODE_ && upt == UPT_ && cache == CACHE_)             \
    return reinterpret_cast<const void*>(&bcjr_fwd_kernel<KV_, V_, CODE_, UPT_, CACHE_>);

#define BCJR_FWD_UPTS(KV_, V_, CODE_, CACHE_) \
  BCJR_FWD_CASE(KV_, V_, CODE_, 1, CACHE_)    \
  BCJR_FWD_CASE(KV_, V_, CODE_, 2, CACHE_)    \
  BCJR_FWD_CASE(KV_, V_, CODE_, 4, CACHE_)    \
  BCJR_FWD_CASE(KV_, V_, CODE_, 8, CACHE_)

const void* fwd_kernel_ptr(int KV, int V, int code, int upt, bool cache) {
  // kV = 1: k = 1, V = 1 (table only)
  BCJR_FWD_CASE(1, 1, CODE_TABLE, 1, true)
  // kV = 2, V = 1: the production scalar codes; cached codewords.
  BCJR_FWD_UPTS(2, 1, CODE_TABLE, true)
  BCJR_FWD_UPTS(2, 1, CODE_1MAD, true)
  BCJR_FWD_UPTS(2, 1, CODE_3INST, true)
  // kV = 2, V = 2 (k = 1): table / HYB, cached up to 4 units per thread.
  BCJR_FWD_CASE(2, 2, CODE_TABLE, 1, true)
  BCJR_FWD_CASE(2, 2, CODE_TABLE, 2, true)
  BCJR_FWD_CASE(2, 2, CODE_TABLE, 4, true)
  BCJR_FWD_CASE(2, 2, CODE_HYB, 1, true)
  BCJR_FWD_CASE(2, 2, CODE_HYB, 2, true)
  BCJR_FWD_CASE(2, 2, CODE_HYB, 4, true)
  // kV = 4: quarter butterflies per unit, codewords on the fly.
  BCJR_FWD_CASE(4, 1, CODE_TABLE, 1, false)
  BCJR_FWD_CASE(4, 1, CODE_TABLE, 2, false)
  BCJR_FWD_CASE(4, 1, CODE_1MAD, 1, false)
  BCJR_FWD_CASE(4, 1, CODE_1MAD, 2, false)
  BCJR_FWD_CASE(4, 1, CODE_3INST, 1, false)
  BCJR_FWD_CASE(4, 1, CODE_3INST, 2, false)
  BCJR_FWD_CASE(4, 2, CODE_TABLE, 1, false)
  BCJR_FWD_CASE(4, 2, CODE_TABLE, 2, false)
  BCJR_FWD_CASE(4, 2, CODE_HYB, 1, false)
  BCJR_FWD_CASE(4, 2, CODE_HYB, 2, false)
  return nullptr;
}

}  // namespace bcjr
