// Backward of the BCJR node: d seq for L = sum(g_soft * soft) + sum(g_logZ * logZ).
//
// Replaces the analytic backward of BcjrForwardBackwardMonolithic
// (src/bcjr/bcjr_monolithic.py:192-243), i.e. the eager autograd of
// src/bcjr/forward_backward.py:106-232.  Codebook and T get no gradient.
//
// Formulation (first-order expectation semiring).  With f_t(s) = g_t . c(s) and
// F = sum_t f_t(s_t), the gradient of sum(g*soft) + g_Z*logZ with respect to the
// log-emission is  dll_t(s) = P_t(s) (phi_t(s) + psi_t(s) - E[F] + g_Z),  where
//   phi_t(s) = E[sum_{tau<=t} f_tau | s_t = s] = f_t(s) + mu_{t-1}(s >> kV),
//   mu_{t-1}(j) = sum_p softmax_p(alpha_{t-1}(p*NT + j)) phi_{t-1}(p*NT + j),
//   psi_t(s) = E[sum_{tau>t} f_tau | s_t = s] = nu_t(s mod NT),
//   nu_{t-1}(j) = sum_c softmax_c(y_t(R*j + c)) (f_t + psi_t)(R*j + c).
// mu rides on the alpha sweep and nu on the beta sweep, reusing their exp2s.
// Then d seq_t[v] = (2/T) (sum_s dll_t(s) c_v(s) - w_t[v] sum_s dll_t(s)), the
// chain rule through ll = -||c - w||^2 / T used in bcjr_monolithic.py:228-239.
//
// Two vectors (m~, mu) or (n~, nu) of NT floats move through LDS each step, which
// at L = 16 fills 128 KiB; they are single-buffered, so each step reads all of a
// thread's inputs, synchronises, then computes and writes.  The alpha sweep writes
// each butterfly's normalised inputs (m~ and mu, 2R floats) to the scratch slot;
// the beta sweep reads them back to form P and phi.
#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace bcjr {

template <int KV, int V, int CODE, int UPT>
__global__ __launch_bounds__(512) void bcjr_bwd_kernel(BwdParams P) {
  constexpr int R = 1 << KV;
  constexpr int RO = R < 4 ? R : 4;
  constexpr int NSUB = R / RO;

  extern __shared__ __align__(16) unsigned char smem[];
  const int L = P.L, N = P.N;
  const int NT = 1 << (L - KV);
  const int NB = NT >> KV;
  const int NU = NB * NSUB;
  const int lgNB = L - 2 * KV;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;

  double* cvec = reinterpret_cast<double*>(smem);  // N
  float* mbuf = reinterpret_cast<float*>(cvec + N);  // NT (m~, then n~)
  float* mubuf = mbuf + NT;                          // NT (mu, then nu)
  float* wmax = mubuf + NT;                          // 2*kMaxWaves
  float* wsum = wmax + 2 * kMaxWaves;                // 2*kMaxWaves
  float* wbuf = wsum + 2 * kMaxWaves;                // N*V
  float* gbuf = wbuf + N * V;                        // N*V
  float* apart = gbuf + N * V;                       // N*nwaves*(V+1)
  float* lut = apart + N * nwaves * (V + 1);

  if constexpr (CODE == CODE_HYB) {
    const int nl = 2 << P.Q;
    for (int i = tid; i < nl; i += nthr) lut[i] = P.table[i];
    __syncthreads();
  }

  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    float* slot = P.ws + (size_t)blockIdx.x * (size_t)N * 2 * (size_t)NT;
    const float Tb = P.T[P.t_per_seq ? b : 0];
    const float sk = sqrtf(kLog2e / Tb);
    const float gZ = P.g_logZ ? P.g_logZ[b] : 0.0f;
    const float* seqb = P.seq + (size_t)b * N * V;
    const float* gb = P.g_soft + (size_t)b * N * V;
    for (int i = tid; i < N * V; i += nthr) {
      wbuf[i] = seqb[i];
      gbuf[i] = gb[i];
    }
    __syncthreads();

    // --------------------------- alpha + mu sweep ----------------------------
    double C = 0.0;
    int k = 0;
    for (int t = 0; t < N; ++t, ++k) {
      float O = (float)KV;
      if (t > 0) {
        O = -INFINITY;
        for (int w = 0; w < nwaves; ++w) O = fmaxf(O, wmax[((k + 1) & 1) * kMaxWaves + w]);
      }
      C += (double)O;
      if (tid == 0) cvec[t] = C;
      float nw[V], gt[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        nw[v] = -wbuf[t * V + v] * sk;
        gt[v] = gbuf[t * V + v];
      }
      float mi[UPT][R], mui[UPT][R];
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int u = opaque(tid + i * nthr) & (NB - 1);
#pragma unroll
        for (int p = 0; p < R; ++p) {
          mi[i][p] = t ? mbuf[p * NB + u] - O : 0.0f;
          mui[i][p] = t ? mubuf[p * NB + u] : 0.0f;
        }
      }
      __syncthreads();
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int q = tid + i * nthr;
        __builtin_amdgcn_sched_barrier(0);
        if (q < NU) {
          const int u = opaque(q) & (NB - 1);
          const int sub = q >> lgNB;
          if (sub == 0) {
            float* dst = slot + ((size_t)t * NB + u) * 2 * R;
#pragma unroll
            for (int p = 0; p < R; ++p) {
              dst[p] = mi[i][p];
              dst[R + p] = mui[i][p];
            }
          }
          float mo[RO], muo[RO];
#pragma unroll
          for (int r = 0; r < RO; ++r) {
            const int rr = sub * RO + r;
            float a[R], phi[R];
#pragma unroll
            for (int p = 0; p < R; ++p) {
              float c[V];
              codeword<CODE, V, false>((uint32_t)(p * NT + R * u + rr), P.table, lut, P.Q, c);
              float acc = mi[i][p];
              float ph = mui[i][p];
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const float d = fmaf(c[v], sk, nw[v]);
                acc = fmaf(-d, d, acc);
                ph = fmaf(gt[v], c[v], ph);
              }
              a[p] = acc;
              phi[p] = ph;
            }
            float M = a[0];
#pragma unroll
            for (int p = 1; p < R; ++p) M = fmaxf(M, a[p]);
            float ssum = 0.0f, ephi = 0.0f;
#pragma unroll
            for (int p = 0; p < R; ++p) {
              const float e = fexp2(a[p] - M);
              ssum += e;
              ephi = fmaf(e, phi[p], ephi);
            }
            mo[r] = M + flog2(ssum);
            muo[r] = ephi * frcp(ssum);
            tmax = fmaxf(tmax, mo[r]);
          }
#pragma unroll
          for (int r = 0; r < RO; ++r) {
            mbuf[R * u + sub * RO + r] = mo[r];
            mubuf[R * u + sub * RO + r] = muo[r];
          }
        }
      }
      tmax = wave_max(tmax);
      if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
      __syncthreads();
    }

    // log2 Z and E[F] = sum_j 2^(m_{N-1}(j) - log2 Z) mu_{N-1}(j).
    float Mz = -INFINITY;
    for (int w = 0; w < nwaves; ++w) Mz = fmaxf(Mz, wmax[((k + 1) & 1) * kMaxWaves + w]);
    float ps = 0.0f, pe = 0.0f;
    for (int j = tid; j < NT; j += nthr) {
      const float e = fexp2(mbuf[j] - Mz);
      ps += e;
      pe = fmaf(e, mubuf[j], pe);
    }
    ps = wave_sum(ps);
    pe = wave_sum(pe);
    if (lane == 0) {
      wsum[wave] = ps;
      wsum[kMaxWaves + wave] = pe;
    }
    __syncthreads();
    float Ssum = 0.0f, Esum = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      Ssum += wsum[w];
      Esum += wsum[kMaxWaves + w];
    }
    const double logZ2 = C + (double)Mz + (double)flog2(Ssum);
    const float EF = Esum / Ssum;

    // -------------------------- beta + nu + grad sweep -----------------------
    double D = 0.0;
    for (int t = N - 1; t >= 0; --t, ++k) {
      float Qv = 0.0f;
      if (t != N - 1) {
        Qv = -INFINITY;
        for (int w = 0; w < nwaves; ++w) Qv = fmaxf(Qv, wmax[((k + 1) & 1) * kMaxWaves + w]);
      }
      const float Kt = (float)(cvec[t] + (double)Qv + D - logZ2);
      float nw[V], gt[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        nw[v] = -wbuf[t * V + v] * sk;
        gt[v] = gbuf[t * V + v];
      }
      float ni[UPT][R], nui[UPT][R];
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int u = opaque(tid + i * nthr) & (NB - 1);
#pragma unroll
        for (int c = 0; c < R; ++c) {
          ni[i][c] = (t != N - 1) ? mbuf[R * u + c] - Qv : 0.0f;
          nui[i][c] = (t != N - 1) ? mubuf[R * u + c] : 0.0f;
        }
      }
      __syncthreads();
      float A0 = 0.0f, A1[V];
#pragma unroll
      for (int v = 0; v < V; ++v) A1[v] = 0.0f;
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int q = tid + i * nthr;
        __builtin_amdgcn_sched_barrier(0);
        if (q < NU) {
          const int u = opaque(q) & (NB - 1);
          const int sub = q >> lgNB;
          const float* src = slot + ((size_t)t * NB + u) * 2 * R + sub * RO;
          float m4[RO], mu4[RO];
#pragma unroll
          for (int pp = 0; pp < RO; ++pp) {
            m4[pp] = src[pp];
            mu4[pp] = src[R + pp];
          }
#pragma unroll
          for (int pp = 0; pp < RO; ++pp) {
            const int p = sub * RO + pp;
            float y[R], z[R], cc[R][V];
#pragma unroll
            for (int c = 0; c < R; ++c) {
              codeword<CODE, V, false>((uint32_t)(p * NT + R * u + c), P.table, lut, P.Q, cc[c]);
              float yy = ni[i][c];
              float zz = nui[i][c];
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const float d = fmaf(cc[c][v], sk, nw[v]);
                yy = fmaf(-d, d, yy);
                zz = fmaf(gt[v], cc[c][v], zz);
              }
              y[c] = yy;
              z[c] = zz;
            }
            float M = y[0];
#pragma unroll
            for (int c = 1; c < R; ++c) M = fmaxf(M, y[c]);
            const float Dp = mu4[pp] - EF + gZ;
            float ssum = 0.0f, ez = 0.0f, a1[V];
#pragma unroll
            for (int v = 0; v < V; ++v) a1[v] = 0.0f;
#pragma unroll
            for (int c = 0; c < R; ++c) {
              const float e = fexp2(y[c] - M);
              ssum += e;
              const float ezc = e * z[c];
              ez += ezc;
              const float w = fmaf(e, Dp, ezc);  // e * (z + Dp)
#pragma unroll
              for (int v = 0; v < V; ++v) a1[v] = fmaf(w, cc[c][v], a1[v]);
            }
            const float G = fexp2(M + m4[pp] + Kt);
            A0 = fmaf(G, fmaf(Dp, ssum, ez), A0);
#pragma unroll
            for (int v = 0; v < V; ++v) A1[v] = fmaf(G, a1[v], A1[v]);
            const float no = M + flog2(ssum);
            mbuf[p * NB + u] = no;
            mubuf[p * NB + u] = ez * frcp(ssum);
            tmax = fmaxf(tmax, no);
          }
        }
      }
      D += (double)Qv;
      A0 = wave_sum(A0);
      if (lane == 0) apart[(t * nwaves + wave) * (V + 1)] = A0;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float s = wave_sum(A1[v]);
        if (lane == 0) apart[(t * nwaves + wave) * (V + 1) + 1 + v] = s;
      }
      tmax = wave_max(tmax);
      if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
      __syncthreads();
    }

    const float twoT = 2.0f / Tb;
    float* gout = P.g_seq + (size_t)b * N * V;
    for (int i = tid; i < N * V; i += nthr) {
      const int t = i / V, v = i - t * V;
      float a0 = 0.0f, a1 = 0.0f;
      for (int w = 0; w < nwaves; ++w) {
        a0 += apart[(t * nwaves + w) * (V + 1)];
        a1 += apart[(t * nwaves + w) * (V + 1) + 1 + v];
      }
      gout[i] = twoT * (a1 - wbuf[i] * a0);
    }
    __syncthreads();
  }
}

#define BCJR_BWD_CASE(KV_, V_, CODE_, UPT_) \
  if (KV == KV_ && V == V_ && code == CODE_ && upt == UPT_) \
    return reinterpret_cast<const void*>(&bcjr_bwd_kernel<KV_, V_, CODE_, UPT_>);

#define BCJR_BWD_UPTS(KV_, V_, CODE_) \
  BCJR_BWD_CASE(KV_, V_, CODE_, 1)    \
  BCJR_BWD_CASE(KV_, V_, CODE_, 2)    \
  BCJR_BWD_CASE(KV_, V_, CODE_, 4)    \
  BCJR_BWD_CASE(KV_, V_, CODE_, 8)

const void* bwd_kernel_ptr(int KV, int V, int code, int upt) {
  BCJR_BWD_CASE(1, 1, CODE_TABLE, 1)
  BCJR_BWD_UPTS(2, 1, CODE_TABLE)
  BCJR_BWD_UPTS(2, 1, CODE_1MAD)
  BCJR_BWD_UPTS(2, 1, CODE_3INST)
  BCJR_BWD_UPTS(2, 2, CODE_TABLE)
  BCJR_BWD_UPTS(2, 2, CODE_HYB)
  BCJR_BWD_CASE(4, 1, CODE_TABLE, 1)
  BCJR_BWD_CASE(4, 1, CODE_TABLE, 2)
  BCJR_BWD_CASE(4, 1, CODE_1MAD, 1)
  BCJR_BWD_CASE(4, 1, CODE_1MAD, 2)
  BCJR_BWD_CASE(4, 1, CODE_3INST, 1)
  BCJR_BWD_CASE(4, 1, CODE_3INST, 2)
  BCJR_BWD_CASE(4, 2, CODE_TABLE, 1)
  BCJR_BWD_CASE(4, 2, CODE_TABLE, 2)
  BCJR_BWD_CASE(4, 2, CODE_HYB, 1)
  BCJR_BWD_CASE(4, 2, CODE_HYB, 2)
  return nullptr;
}

}  // namespace bcjr
