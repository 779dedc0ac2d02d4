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
// Log-sum-exps use the butterfly-normalised group sums of the forward kernel;
// codewords are formed per state from the hash (c = kSigma * h),
// so f_t(s) = (kSigma g_t) . h(s) and the sums over h are scaled once at the end.
//
// Two vectors (m~, mu) or (n~, nu) of NT floats move through LDS each step, which
// at L = 16 fills 128 KiB, so they are single-buffered, interleaved as 8-byte
// pairs, in the in-place rotated layout of Swizzle: a thread reads its
// butterfly's R pairs, computes, and writes its R outputs to the same pairs, with
// one barrier per step and the next butterfly's pairs read ahead of the current
// one's arithmetic.  The alpha sweep writes each butterfly's raw inputs to the
// scratch slot as R (m~, mu) pairs, [m~_0 mu_0 m~_1 mu_1 ...], the form in which
// they leave LDS; the beta sweep reads them back two butterflies ahead to form
// P and phi.  The codewords of a thread's first few
// butterflies stay in VGPRs for the launch (bwd_cached_units).
//
// Group sums take the zero-shift form; a butterfly with any
// underflowed group (sum < kUnderflow) is recomputed against the group maxima
// (rare at T >= kExactBelowT; below it every group uses the maxima).
#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace bcjr {

// Unroll of the loop over a butterfly's outputs: full for 2 or 4 states.
template <int R>
constexpr int kOuterUnroll = R <= 4 ? R : 1;

// A butterfly's slot entry: R (m~, mu) pairs, 8-byte aligned.  Each pair is
// stored from the two registers the LDS read filled, so no register moves
// assemble a wider store.
template <int R>
__device__ __forceinline__ void store_pairs(float* dst, const float (&m)[R], const float (&mu)[R]) {
#pragma unroll
  for (int p = 0; p < R; ++p) *reinterpret_cast<float2*>(dst + 2 * p) = make_float2(m[p], mu[p]);
}
// ... read back 16 bytes (two pairs) at a time (16-byte aligned, R even).
template <int R>
__device__ __forceinline__ void load_pairs(const float* src, float (&m)[R], float (&mu)[R]) {
  static_assert(R % 2 == 0, "pairs are read two at a time");
#pragma unroll
  for (int p = 0; p < R; p += 2) {
    const float4 v = *reinterpret_cast<const float4*>(src + 2 * p);
    m[p] = v.x;
    mu[p] = v.y;
    m[p + 1] = v.z;
    mu[p + 1] = v.w;
  }
}

template <int KV, int V, int CODE, int UPT, int CU, int CUA>
__global__ __launch_bounds__(CODE == CODE_HYB_COL ? 256 : 512, CODE == CODE_HYB_COL ? 3 : 1) void bcjr_bwd_kernel(BwdParams P) {
  constexpr int R = 1 << KV;
  // Butterflies whose slot inputs are in flight ahead of the beta sweep's use
  // (3 or 4 measured no faster at L=16: the HBM latency is already covered).
  constexpr int kSlotAhead = 2;
  using CT = CodeTraits<CODE>;
  // Butterflies of 2 or 4 states run fully unrolled with their slot-side
  // inputs prefetched in registers; 16-state butterflies loop over outputs and
  // read those inputs from the slot as they go (the loop unrolled on the HYB
  // column walk, whose LUT offsets are then immediates).
  constexpr bool kPair = R <= 4;
  static_assert((CU == 0 && CUA == 0) || kPair, "codeword cache is for butterflies of at most 4 states");
  static_assert(CU <= UPT && CUA <= UPT, "at most UPT cached butterflies");
  constexpr bool kCol = CODE == CODE_HYB_COL;  // HYB column walk: one butterfly per thread
  static_assert(!kCol || (KV == 4 && UPT == 1), "the column walk is for L = 16, kV = 4");
  constexpr bool kColUnroll = kCol;  // outputs unrolled: immediate LUT offsets
  // Its alpha + mu sweep reads each state's emission and path feature from a
  // per-step table (below).
  constexpr bool kETab = kColUnroll;

  extern __shared__ __align__(16) unsigned char smem[];
  const int L = P.L, N = P.N;
  const int nb = L - KV;  // reduced-state bits
  const int NT = 1 << nb;
  const int NB = NT >> KV;
  const uint32_t ANT = opaque_uniform(CT::A * (uint32_t)NT);  // hash offset of p * NT
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
  // The column-walk instance gives thread tid butterfly col_walk_unit(tid), so
  // that a half-wave's LUT reads hit distinct banks (the host picks the state
  // swizzle for that lane map); elsewhere u = tid.
  const int utid = kColUnroll ? (int)col_walk_unit((uint32_t)tid) : tid;
  const Swizzle swz = P.swz;

  // LDS: the (m~, mu) pairs sit at byte kPairBase (0, or 16 KiB behind the
  // column walk's tables), so a pair's byte address is kPairBase plus 8 times
  // its element index.
  constexpr uint32_t kPairBase = kETab ? 16384u : 0u;
  float2* mm = reinterpret_cast<float2*>(smem + kPairBase);                    // NT (m~, mu) then (n~, nu)
  double* cvec = reinterpret_cast<double*>(smem + kPairBase + (size_t)8 * NT);  // N  C_{t-1}
  float* wmax = reinterpret_cast<float*>(cvec + ((N + 1) & ~1));    // 2*kMaxWaves
  float* wsum = wmax + 2 * kMaxWaves;                               // 2*kMaxWaves
  // Last wsum word: the block-wide input flag (at most 8 waves use wsum, launch
  // bounds 512 threads), 0 outside the check at the start of each sequence.
  int* bflag = reinterpret_cast<int*>(wsum + kMaxWaves - 1);
  float* wbuf = wsum + 2 * kMaxWaves;                               // N*V
  float* gbuf = wbuf + N * V;                                       // N*V
  float* apart = gbuf + N * V;                                      // 2*nwaves*(V+1) per-wave partials
  // HYB: signed LUT (code_hyb_signed), 8-byte aligned; kETab: the column walk's
  // per-step tables at byte 0.
  float* lut = kETab ? reinterpret_cast<float*>(smem)
                     : reinterpret_cast<float*>(smem) +
                           ((apart + 2 * nwaves * (V + 1) - reinterpret_cast<float*>(smem) + 1) & ~1);

  if constexpr (CODE == CODE_HYB) {
    stage_hyb_signed(reinterpret_cast<float2*>(lut), P.table, P.Q, tid, nthr);
    __syncthreads();
  }
  const unsigned char* lutb = reinterpret_cast<const unsigned char*>(lut);
  // Table of the column-walk alpha + mu sweep, in the LUT's place until the beta
  // sweep stages the LUT: per step, the float2 at entry k of the column-walk
  // layout (32 rows of 64, rows 16..31 repeating 0..15) is (-|d|^2, sg . h) of
  // that LUT entry h, d = h ssk + nw_t, so a state's pair sits at the byte its
  // codeword has in the LUT.  The kernel runs 256 threads here; thread tid forms
  // entries tid + 256j (j < 4) and their row copies, reading the codewords from
  // the (2^Q, 2) table as stage_hyb_col does.
  auto load_codewords = [&](float (&h)[4][2]) {
    const int ncol = 1 << (P.Q - 3), mask = (1 << P.Q) - 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = tid + 256 * j, col = k & 63, i = col + ncol * (k >> 6), ie = i & mask;
      h[j][0] = col < ncol ? P.table[2 * ie] : 0.0f;
      const float y = col < ncol ? P.table[2 * ie + 1] : 0.0f;
      h[j][1] = (i >> P.Q) ? -y : y;
    }
  };
  auto build_etab = [&](const float (&h)[4][2], const float (&nw)[V], const float (&sg)[V], float ssk) {
    float2* et = reinterpret_cast<float2*>(lut);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float e = 0.0f, f = 0.0f;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float d = fmaf(h[j][v], ssk, nw[v]);
        e = fmaf(-d, d, e);
        f = fmaf(sg[v], h[j][v], f);
      }
      const int k = tid + 256 * j;
      et[k] = make_float2(e, f);
      et[k + 1024] = make_float2(e, f);
    }
  };
  // Column-walk bases of this thread's butterfly u = utid, input c (state R*u + c),
  // for the beta sweep; the alpha sweep forms its output's base as it goes.
  uint32_t cbs[kCol ? R : 1];
  if constexpr (kCol) {
#pragma unroll
    for (int c = 0; c < R; ++c) cbs[c] = hyb_col_base((uint32_t)(R * min(utid, NB - 1) + c), P.Q);
  }

  // Raw codewords h of this thread's first NC butterflies (hcx[i][p][c] for
  // state p*NT + R*u + c); the others are hashed per state.  Each sweep fills
  // its own cache when it starts (CUA butterflies for alpha + mu, CU for beta
  // + nu + grad, whose working set is larger), so neither cache is live in the
  // other sweep.  The opaque thread index keeps the fill inside the sequence
  // loop instead of hoisted to the launch, where both caches would be live.
  auto fill_cache = [&](auto& hcx, auto count_tag) {
    constexpr int NC = decltype(count_tag)::value;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int u = min(opaque(utid) + i * nthr, NB - 1);
      const uint32_t xu = CT::A * (uint32_t)(R * u) + CT::B;
#pragma unroll
      for (int p = 0; p < R; ++p)
#pragma unroll
        for (int c = 0; c < R; ++c)
          raw_codeword<CODE, V>(xu, CT::A * (uint32_t)(p * NT + c), (uint32_t)(p * NT + R * u + c), P.table, lut,
                                P.Q, hcx[i][p][c]);
    }
  };

  // Byte address of slot k of butterfly utid + i*nthr at rotation rho:
  // 8 S(rotr(utid + i*nthr + k*NB)) = yb ^ unit_off(i) ^ slot_off(k), the last
  // two uniform (utid, i*nthr and k*NB occupy disjoint bits; S and rotr are
  // linear).
  auto base_off = [&](int rho) -> uint32_t {
    return swizzle(rotr_bits((uint32_t)min(utid, NB - 1), rho, nb), swz) << 3;
  };
  auto unit_off = [&](int i, int rho) -> uint32_t {
    return swizzle(rotr_bits((uint32_t)(i * nthr), rho, nb), swz) << 3;
  };
  auto slot_off = [&](int k, int rho) -> uint32_t {
    return swizzle(rotr_bits((uint32_t)(k * NB), rho, nb), swz) << 3;
  };
  auto lds_pair = [&](uint32_t off) -> float2& { return *reinterpret_cast<float2*>(smem + kPairBase + off); };

  if (tid == 0) *bflag = 0;
  __syncthreads();

  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    float* slot = P.ws + (size_t)blockIdx.x * (size_t)N * 2 * (size_t)NT;
    const float Tb = P.T[P.t_per_seq ? b : 0];
    const float sk = sqrtf(kLog2e / Tb);
    const float ssk = CT::kSigma * sk;
    const float gZ = P.g_logZ ? P.g_logZ[b] : 0.0f;
    const float* seqb = P.seq + (size_t)b * N * V;
    const float* gb = P.g_soft + (size_t)b * N * V;
    float* gout = P.g_seq + (size_t)b * N * V;
    const float twoT = 2.0f / Tb;
    // d seq_t[v] from the per-wave sums of step t in partial buffer `par`, summed
    // in wave order
    auto grad_out = [&](int t, int par, int v) {
      float a0 = 0.0f, a1 = 0.0f;
      for (int w = 0; w < nwaves; ++w) {
        a0 += apart[(par * nwaves + w) * (V + 1)];
        a1 += apart[(par * nwaves + w) * (V + 1) + 1 + v];
      }
      gout[t * V + v] = twoT * (a1 - wbuf[t * V + v] * a0);
    };
    // T must be finite and > 0, the weights and upstream gradients finite;
    // otherwise the sequence's gradient is NaN.
    int bad = !(Tb > 0.0f && Tb < INFINITY) || !__builtin_isfinite(gZ);
    for (int i = tid; i < N * V; i += nthr) {
      const float w = seqb[i], gg = gb[i];
      wbuf[i] = w;
      gbuf[i] = gg;
      bad |= !__builtin_isfinite(w) || !__builtin_isfinite(gg);
    }
    // (m~_{-1}, mu_{-1}) = (log2(R), 0) for every state: what step 0 reads.
    for (int j = tid; j < NT; j += nthr) mm[j] = make_float2((float)KV, 0.0f);
    if (tid < 2 * kMaxWaves) wmax[tid] = -INFINITY;  // waves that do not exist
    if (bad) *bflag = 1;
    __syncthreads();
    if (*bflag) {  // uniform: every thread reads the flag after the barrier
      for (int i = tid; i < N * V; i += nthr) gout[i] = NAN;
      __syncthreads();
      if (tid == 0) *bflag = 0;
      __syncthreads();
      continue;
    }

    // Below kExactBelowT most groups would underflow the zero-shift sums, so
    // the whole sequence uses the group maxima.  The choice is a uniform branch
    // around both sweeps: each variant gets its own register allocation.
    auto sweeps = [&](auto exact_tag) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      using Fast = std::integral_constant<bool, EXACT>;

      // --------------------------- alpha + mu sweep ----------------------------
      float hca[CUA > 0 ? CUA : 1][CUA > 0 ? R : 1][CUA > 0 ? R : 1][V];
      fill_cache(hca, std::integral_constant<int, CUA>{});
      // kETab: this thread's 4 LUT entries for the per-step tables, held over the sweep
      float hE[4][2];
      if constexpr (kETab) load_codewords(hE);
      double C = 0.0;  // C_{t-1}
      int k = 0;
      int rho = nb - KV;  // kV * (t - 1) mod nb at t = 0
      for (int t = 0; t < N; ++t, ++k) {
        float O = (float)KV;
        if (t > 0) {
          O = -INFINITY;
          O = block_max(wmax + ((k + 1) & 1) * kMaxWaves);
        }
        if (tid == 0) cvec[t] = C;
        C += (double)O;
        float nw[V], sg[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          nw[v] = -wbuf[t * V + v] * sk;
          sg[v] = CT::kSigma * gbuf[t * V + v];  // f = g . c = sg . h
        }
        if constexpr (kETab) {  // every wave has left step t-1's table (barrier at its end)
          build_etab(hE, nw, sg, ssk);
          __syncthreads();
        }
        const uint32_t yb = base_off(rho);
        uint32_t Ku[UPT], Kk[R];  // uniform per step
#pragma unroll
        for (int i = 0; i < UPT; ++i) Ku[i] = unit_off(i, rho);
        if constexpr (kPair) {
#pragma unroll
          for (int c = 0; c < R; ++c) Kk[c] = slot_off(c, rho);
        }
        auto koff = [&](int c) -> uint32_t {
          if constexpr (kPair) {
            return Kk[c];
          } else {
            return slot_off(c, rho);
          }
        };

        // Output r of butterfly u: m~ and mu of state R*u + r from the shifted
        // inputs m[p] (maximum 0) and the raw mu inputs; returns the group sum.
        // cb: the column-walk base of state R*u + r (kCol only).
        auto alpha_out = [&](auto shift_tag, int i, int r, uint32_t xu, int u, const float (&m)[R],
                             const float (&mui)[R], float oout, float& mo, float& muo, uint32_t cb) -> float {
          constexpr bool SHIFT = decltype(shift_tag)::value;
          float a[R], phi[R];
#pragma unroll
          for (int p = 0; p < R; ++p) {
            if constexpr (kETab) {
              const float2 ef = hyb_col_read(lutb, cb + hyb_col_step(p, r));
              a[p] = m[p] + ef.x;
              phi[p] = mui[p] + ef.y;
              continue;
            }
            float h[V];
            if (i < CUA) {
#pragma unroll
              for (int v = 0; v < V; ++v) h[v] = hca[i < CUA ? i : 0][p][r][v];
            } else {
              raw_codeword<CODE, V>(xu, p * ANT + CT::A * (uint32_t)r, (uint32_t)(p * NT + R * u + r), P.table,
                                    lut, P.Q, h);
            }
            float acc = m[p];
            float ph = mui[p];
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float d = fmaf(h[v], ssk, nw[v]);
              acc = fmaf(-d, d, acc);
              ph = fmaf(sg[v], h[v], ph);
            }
            a[p] = acc;
            phi[p] = ph;
          }
          float M = 0.0f;
          if constexpr (SHIFT) {
            M = max_of_inputs(a);
          }
          float e = fexp2(a[0] - M);
          float s = e, ephi = e * phi[0];
#pragma unroll
          for (int p = 1; p < R; ++p) {
            e = fexp2(a[p] - M);
            s += e;
            ephi = fmaf(e, phi[p], ephi);
          }
          mo = flog2(s) + (M - oout);
          muo = ephi * frcp(s);
          return s;
        };

        auto read_in = [&](int i, float (&m)[R], float (&mu)[R]) {
          const uint32_t yi = yb ^ Ku[i];
#pragma unroll
          for (int p = 0; p < R; ++p) {
            const float2 v2 = lds_pair(yi ^ koff(p));
            m[p] = v2.x;
            mu[p] = v2.y;
          }
        };
        // Inputs of the next butterfly are read before the current one's
        // arithmetic: its pairs are disjoint from every pair written here.
        float nx[R], nxu[R];
        read_in(0, nx, nxu);
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
          const int q = utid + i * nthr;
          float mi[R], mui[R];
#pragma unroll
          for (int p = 0; p < R; ++p) {
            mi[p] = nx[p];
            mui[p] = nxu[p];
          }
          if (i + 1 < UPT) read_in(i + 1, nx, nxu);
          if (q < NB) {
            const int u = i < CUA ? q : opaque(q);
            {
              store_pairs(slot + ((size_t)t * NB + u) * 2 * R, mi, mui);
            }
            const float Mu = max_of_inputs(mi);
            const float sh = -Mu;
            float m[R];
#pragma unroll
            for (int p = 0; p < R; ++p) m[p] = mi[p] + sh;
            const uint32_t xu = CT::A * (uint32_t)(R * u) + CT::B;
            const float oout = sh + O;
            const uint32_t yi = yb ^ Ku[i];
            if constexpr (kPair) {
              float mo[R], muo[R], smin = 0.0f;
#pragma unroll
              for (int r = 0; r < R; ++r) {
                const float s = alpha_out(Fast{}, i, r, xu, u, m, mui, oout, mo[r], muo[r], 0u);
                smin = r ? fminf(smin, s) : s;
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
#pragma unroll
                  for (int r = 0; r < R; ++r)
                    alpha_out(std::true_type{}, i, r, xu, u, m, mui, oout, mo[r], muo[r], 0u);
                }
              }
#pragma unroll
              for (int r = 0; r < R; ++r) {
                lds_pair(yi ^ koff(r)) = make_float2(mo[r], muo[r]);
              }
              tmax = max_with(tmax, mo);
            } else if constexpr (kColUnroll) {
              // Outputs unrolled, so every state's LUT offset is an immediate; a
              // butterfly with an underflowed group is redone output by output
              // (its inputs are in registers, its outputs overwrite the pairs).
              float smin = 0.0f;
#pragma unroll
              for (int r = 0; r < R; ++r) {
                float mo, muo;
                const float s = alpha_out(Fast{}, i, r, xu, u, m, mui, oout, mo, muo, cbs[r]);
                smin = r ? fminf(smin, s) : s;
                lds_pair(yi ^ koff(r)) = make_float2(mo, muo);
                tmax = vmax_raw(tmax, mo);
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
#pragma unroll 1
                  for (int r = 0; r < R; ++r) {
                    float mo, muo;
                    alpha_out(std::true_type{}, i, r, xu, u, m, mui, oout, mo, muo,
                              hyb_col_base((uint32_t)(R * u + r), P.Q));
                    lds_pair(yi ^ koff(r)) = make_float2(mo, muo);
                    tmax = vmax_raw(tmax, mo);
                  }
                }
              }
            } else {
#pragma unroll kOuterUnroll<R>
              for (int r = 0; r < R; ++r) {
                float mo, muo;
                const float s = alpha_out(Fast{}, i, r, xu, u, m, mui, oout, mo, muo, 0u);
                if (!EXACT && s < kUnderflow) alpha_out(std::true_type{}, i, r, xu, u, m, mui, oout, mo, muo, 0u);
                lds_pair(yi ^ koff(r)) = make_float2(mo, muo);
                tmax = vmax_raw(tmax, mo);
              }
            }
          }
        }
        tmax = wave_max(tmax);
        if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
        rho = rho + KV >= nb ? rho + KV - nb : rho + KV;
        __syncthreads();
      }

      // kETab: the beta sweep's table replaces the alpha sweep's (every wave has
      // left it at the last alpha step's barrier; the barriers below come before
      // its first read): float4 entry k = (-|d|^2, sg . h, h) of LUT entry k,
      // rows 0..15 only, its codeword written here and (e, f) per step.  A
      // state's entry is at twice its codeword's LUT byte, its row wrapped mod 16
      // (cbs doubled for the sweep).
      if constexpr (kETab) {
        float4* et = reinterpret_cast<float4*>(lut);
#pragma unroll
        for (int j = 0; j < 4; ++j) et[tid + 256 * j] = make_float4(0.0f, 0.0f, hE[j][0], hE[j][1]);
#pragma unroll
        for (int c = 0; c < R; ++c) cbs[c] <<= 1;
      }

      // log2 Z and E[F] = sum_j 2^(m_{N-1}(j) - log2 Z) mu_{N-1}(j); m~ and mu of a
      // state share a pair, so the sums run over pairs.
      float Mz = -INFINITY;
      Mz = block_max(wmax + ((k + 1) & 1) * kMaxWaves);
      float ps = 0.0f, pe = 0.0f;
      for (int j = tid; j < NT; j += nthr) {
        const float2 v2 = mm[j];
        const float e = fexp2(v2.x - Mz);
        ps += e;
        pe = fmaf(e, v2.y, pe);
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
      const float EFg = Esum / Ssum - gZ;  // E[F] - g_Z
      // (n~_{N-1}, nu_{N-1}) = (0, 0): what step N-1 of the beta sweep reads.
      for (int j = tid; j < NT; j += nthr) mm[j] = make_float2(0.0f, 0.0f);
      __syncthreads();

      // -------------------------- beta + nu + grad sweep -----------------------
      float hcb[CU > 0 ? CU : 1][CU > 0 ? R : 1][CU > 0 ? R : 1][V];
      fill_cache(hcb, std::integral_constant<int, CU>{});
      // Raw alpha-side inputs (m~, mu) of step t come back from HBM two
      // butterflies ahead of their use, across step boundaries.
      auto slot_src = [&](int t, int i) {
        const int q = min(utid + i * nthr, NB - 1);
        return slot + ((size_t)t * NB + q) * 2 * R;
      };
      // The next two butterflies in consumption order (t descending, i
      // ascending).
      // A shift register of the next kSlotAhead butterflies' (m~, mu) inputs.
      float pf[kSlotAhead][R], pfu[kSlotAhead][R];
      if constexpr (kPair) {
#pragma unroll
        for (int d = 0; d < kSlotAhead; ++d) {
          const int tt = N - 1 - d / UPT;
          if (tt >= 0) {
            load_pairs(slot_src(tt, d % UPT), pf[d], pfu[d]);
          }
        }
      }
      double D = 0.0;  // D_t
      // rho_t = kV * (t - 1) mod nb at t = N - 1
      rho = (int)(((long long)KV * (N - 2) % nb + nb) % nb);
      for (int t = N - 1; t >= 0; --t, ++k) {
        float Qv = 0.0f;
        if (t != N - 1) {
          Qv = -INFINITY;
          Qv = block_max(wmax + ((k + 1) & 1) * kMaxWaves);
          // gradient of step t+1 from its per-wave partials (the other parity buffer)
          if (tid < V) grad_out(t + 1, (k + 1) & 1, tid);
        }
        const float Kt = (float)(cvec[t] + D - logZ2);
        float nw[V], sg[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          nw[v] = -wbuf[t * V + v] * sk;
          sg[v] = CT::kSigma * gbuf[t * V + v];
        }
        if constexpr (kETab) {  // every wave has left step t+1's table (barrier at its end)
          float4* et = reinterpret_cast<float4*>(lut);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int kk = tid + 256 * j;
            const float2 h = *reinterpret_cast<const float2*>(&et[kk].z);
            float e = 0.0f, f = 0.0f;
            const float d0 = fmaf(h.x, ssk, nw[0]);
            e = fmaf(-d0, d0, e);
            f = fmaf(sg[0], h.x, f);
            const float d1 = fmaf(h.y, ssk, nw[1]);
            e = fmaf(-d1, d1, e);
            f = fmaf(sg[1], h.y, f);
            *reinterpret_cast<float2*>(&et[kk]) = make_float2(e, f);
          }
          __syncthreads();
        }
        const uint32_t yb = base_off(rho);
        uint32_t Ku[UPT], Kk[R];  // uniform per step
#pragma unroll
        for (int i = 0; i < UPT; ++i) Ku[i] = unit_off(i, rho);
        if constexpr (kPair) {
#pragma unroll
          for (int c = 0; c < R; ++c) Kk[c] = slot_off(c, rho);
        }
        auto koff = [&](int c) -> uint32_t {
          if constexpr (kPair) {
            return Kk[c];
          } else {
            return slot_off(c, rho);
          }
        };
        // kETab: the table bases, opaque per step, so that the 16 x 16 wrapped
        // addresses are formed where they are read, not hoisted out of the loop.
        uint32_t cbo[kETab ? R : 1];
        if constexpr (kETab) {
#pragma unroll
          for (int c = 0; c < R; ++c) cbo[c] = (uint32_t)opaque((int)cbs[c]);
        }

        // Output p of butterfly u: n~ and nu of state p*NB + u from the shifted
        // inputs nr[c] (maximum 0) and raw nu inputs, and the butterfly's
        // contribution to the gradient sums (a0 for sum dll, a1 for sum dll h).
        // pms = raw m~_{t-1}(p*NB + u) + Kt - sh.  Returns the group sum.
        auto beta_out = [&](auto shift_tag, int i, int p, uint32_t xu, int u, const float (&nr)[R],
                            const float (&nui)[R], float pms, float pmu, float oout, float& no, float& nuo,
                            float& a0, float (&a1)[V]) -> float {
          constexpr bool SHIFT = decltype(shift_tag)::value;
          if constexpr (kETab && !SHIFT) {
            // Group-sum variant (M = 0): each input's terms are summed as its
            // table entry is read, so one entry at a time is live (the same
            // operations as the general form below).
            const float Dp = pmu - EFg;
            float s = 0.0f, ez = 0.0f, ga[V];
#pragma unroll
            for (int c = 0; c < R; ++c) {
              const float4 ef = *reinterpret_cast<const float4*>(smem + ((cbo[c] + 2 * hyb_col_step(p, c)) & 0x3FFFu));
              const float e = fexp2(nr[c] + ef.x);
              const float ezc = e * (nui[c] + ef.y);
              s = c ? s + e : e;
              ez = c ? ez + ezc : ezc;
              const float wgt = fmaf(e, Dp, ezc);
              ga[0] = c ? fmaf(wgt, ef.z, ga[0]) : wgt * ef.z;
              ga[1] = c ? fmaf(wgt, ef.w, ga[1]) : wgt * ef.w;
            }
            const float G = fexp2(pms);
            a0 = G * fmaf(Dp, s, ez);
#pragma unroll
            for (int v = 0; v < V; ++v) a1[v] = G * ga[v];
            no = flog2(s) + (0.0f - oout);
            nuo = ez * frcp(s);
            return s;
          }
          float y[R], z[R], hh[R][V];
#pragma unroll
          for (int c = 0; c < R; ++c) {
            if constexpr (kETab) {
              const float4 ef = *reinterpret_cast<const float4*>(smem + ((cbo[c] + 2 * hyb_col_step(p, c)) & 0x3FFFu));
              y[c] = nr[c] + ef.x;
              z[c] = nui[c] + ef.y;
              hh[c][0] = ef.z;
              hh[c][1] = ef.w;
              continue;
            }
            if (i < CU) {
#pragma unroll
              for (int v = 0; v < V; ++v) hh[c][v] = hcb[i < CU ? i : 0][p][c][v];
            } else {
              raw_codeword<CODE, V>(xu, p * ANT + CT::A * (uint32_t)c, (uint32_t)(p * NT + R * u + c), P.table,
                                    lut, P.Q, hh[c]);
            }
            float yy = nr[c];
            float zz = nui[c];
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float d = fmaf(hh[c][v], ssk, nw[v]);
              yy = fmaf(-d, d, yy);
              zz = fmaf(sg[v], hh[c][v], zz);
            }
            y[c] = yy;
            z[c] = zz;
          }
          float M = 0.0f;
          if constexpr (SHIFT) {
            M = max_of_inputs(y);
          }
          const float Dp = pmu - EFg;  // mu_{t-1} - E[F] + g_Z
          float s = 0.0f, ez = 0.0f, ga[V];
#pragma unroll
          for (int v = 0; v < V; ++v) ga[v] = 0.0f;
#pragma unroll
          for (int c = 0; c < R; ++c) {
            const float e = fexp2(y[c] - M);
            const float ezc = e * z[c];
            s = c ? s + e : e;
            ez = c ? ez + ezc : ezc;
            const float wgt = fmaf(e, Dp, ezc);  // e * (z + Dp)
#pragma unroll
            for (int v = 0; v < V; ++v) ga[v] = c ? fmaf(wgt, hh[c][v], ga[v]) : wgt * hh[c][v];
          }
          // (pms + 0 does not fold: -0 + 0 is +0)
          const float G = SHIFT ? fexp2(pms + M) : fexp2(pms);
          // sum_s dll_t(s) is g_Z in exact arithmetic, but its computed value
          // cancels the common-mode rounding of (phi + psi - E[F]) in
          // A1 - w A0, which grows with N: it is accumulated, not assumed.
          a0 = G * fmaf(Dp, s, ez);
#pragma unroll
          for (int v = 0; v < V; ++v) a1[v] = G * ga[v];
          no = flog2(s) + (M - oout);
          nuo = ez * frcp(s);
          return s;
        };

        auto read_in = [&](int i, float (&n)[R], float (&nu)[R]) {
          const uint32_t yi = yb ^ Ku[i];
#pragma unroll
          for (int c = 0; c < R; ++c) {
            const float2 v2 = lds_pair(yi ^ koff(c));
            n[c] = v2.x;
            nu[c] = v2.y;
          }
        };
        float nx[R], nxu[R];
        read_in(0, nx, nxu);
        float A0 = 0.0f, A1[V];
#pragma unroll
        for (int v = 0; v < V; ++v) A1[v] = 0.0f;
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
          const int q = utid + i * nthr;
          float pm[R], pmu[R], ni[R], nui[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if constexpr (kPair) {
              pm[r] = pf[0][r];
              pmu[r] = pfu[0][r];
#pragma unroll
              for (int d = 0; d + 1 < kSlotAhead; ++d) {
                pf[d][r] = pf[d + 1][r];
                pfu[d][r] = pfu[d + 1][r];
              }
            }
            ni[r] = nx[r];
            nui[r] = nxu[r];
          }
          if constexpr (kPair) {  // fetch the butterfly kSlotAhead ahead
            const int tt = t - (i + kSlotAhead) / UPT;
            const int ii = (i + kSlotAhead) % UPT;
            if (tt >= 0) {
              load_pairs(slot_src(tt, ii), pf[kSlotAhead - 1], pfu[kSlotAhead - 1]);
            }
          }
          if (i + 1 < UPT) read_in(i + 1, nx, nxu);
          if (q < NB) {
            const int u = i < CU ? q : opaque(q);
            const float Mu = max_of_inputs(ni);
            const float sh = -Mu;
            float nr[R];
#pragma unroll
            for (int c = 0; c < R; ++c) nr[c] = ni[c] + sh;
            const uint32_t xu = CT::A * (uint32_t)(R * u) + CT::B;
            const float oout = sh + Qv;
            const float kts = Kt - sh;
            const uint32_t yi = yb ^ Ku[i];
            if constexpr (kPair) {
              float no[R], nuo[R], smin = 0.0f, ua0 = 0.0f, ua1[V];
#pragma unroll
              for (int p = 0; p < R; ++p) {
                float a0, a1[V];
                const float s = beta_out(Fast{}, i, p, xu, u, nr, nui, pm[p] + kts, pmu[p], oout, no[p], nuo[p], a0, a1);
                smin = p ? fminf(smin, s) : s;
                ua0 = p ? ua0 + a0 : a0;
#pragma unroll
                for (int v = 0; v < V; ++v) ua1[v] = p ? ua1[v] + a1[v] : a1[v];
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
                  ua0 = 0.0f;
#pragma unroll
                  for (int v = 0; v < V; ++v) ua1[v] = 0.0f;
#pragma unroll
                  for (int p = 0; p < R; ++p) {
                    float a0, a1[V];
                    beta_out(std::true_type{}, i, p, xu, u, nr, nui, pm[p] + kts, pmu[p], oout, no[p], nuo[p], a0, a1);
                    ua0 += a0;
#pragma unroll
                    for (int v = 0; v < V; ++v) ua1[v] += a1[v];
                  }
                }
              }
              A0 += ua0;
#pragma unroll
              for (int v = 0; v < V; ++v) A1[v] += ua1[v];
#pragma unroll
              for (int p = 0; p < R; ++p) {
                lds_pair(yi ^ koff(p)) = make_float2(no[p], nuo[p]);
              }
              tmax = max_with(tmax, no);
            } else if constexpr (kColUnroll) {
              // Outputs unrolled (immediate LUT offsets); the butterfly's gradient
              // sums are redone when a group underflowed.
              const float* src = slot_src(t, i);
              float smin = 0.0f, ua0 = 0.0f, ua1[V];
#pragma unroll
              for (int p = 0; p < R; ++p) {
                float no, nuo, a0, a1[V];
                const float pms = src[2 * p] + kts, pmup = src[2 * p + 1];
                const float s = beta_out(Fast{}, i, p, xu, u, nr, nui, pms, pmup, oout, no, nuo, a0, a1);
                smin = p ? fminf(smin, s) : s;
                ua0 = p ? ua0 + a0 : a0;
#pragma unroll
                for (int v = 0; v < V; ++v) ua1[v] = p ? ua1[v] + a1[v] : a1[v];
                lds_pair(yi ^ koff(p)) = make_float2(no, nuo);
                tmax = vmax_raw(tmax, no);
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
                  ua0 = 0.0f;
#pragma unroll
                  for (int v = 0; v < V; ++v) ua1[v] = 0.0f;
#pragma unroll 1
                  for (int p = 0; p < R; ++p) {
                    float no, nuo, a0, a1[V];
                    const float pms = src[2 * p] + kts, pmup = src[2 * p + 1];
                    beta_out(std::true_type{}, i, p, xu, u, nr, nui, pms, pmup, oout, no, nuo, a0, a1);
                    ua0 += a0;
#pragma unroll
                    for (int v = 0; v < V; ++v) ua1[v] += a1[v];
                    lds_pair(yi ^ koff(p)) = make_float2(no, nuo);
                    tmax = vmax_raw(tmax, no);
                  }
                }
              }
              A0 += ua0;
#pragma unroll
              for (int v = 0; v < V; ++v) A1[v] += ua1[v];
            } else {
              const float* src = slot_src(t, i);
#pragma unroll kOuterUnroll<R>
              for (int p = 0; p < R; ++p) {
                float no, nuo, a0, a1[V];
                const float pms = src[2 * p] + kts, pmup = src[2 * p + 1];
                const float s = beta_out(Fast{}, i, p, xu, u, nr, nui, pms, pmup, oout, no, nuo, a0, a1);
                if (!EXACT && s < kUnderflow)
                  beta_out(std::true_type{}, i, p, xu, u, nr, nui, pms, pmup, oout, no, nuo, a0, a1);
                A0 += a0;
#pragma unroll
                for (int v = 0; v < V; ++v) A1[v] += a1[v];
                lds_pair(yi ^ koff(p)) = make_float2(no, nuo);
                tmax = vmax_raw(tmax, no);
              }
            }
          }
        }
        D += (double)Qv;
        A0 = wave_sum(A0);
        if (lane == 0) apart[((k & 1) * nwaves + wave) * (V + 1)] = A0;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float s = wave_sum(A1[v]);
          if (lane == 0) apart[((k & 1) * nwaves + wave) * (V + 1) + 1 + v] = s * CT::kSigma;
        }
        tmax = wave_max(tmax);
        if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
        rho = rho - KV < 0 ? rho - KV + nb : rho - KV;
        __syncthreads();
      }
      if constexpr (kETab) {  // the alpha sweep's undoubled bases
#pragma unroll
        for (int c = 0; c < R; ++c) cbs[c] >>= 1;
      }
    };
    if (Tb < kExactBelowT) {
      sweeps(std::true_type{});
    } else {
      sweeps(std::false_type{});
    }

    // step 0's partials sit in the buffer of the last beta step's parity ((2N - 1) & 1)
    if (tid < V) grad_out(0, 1, tid);
    if (tid == 0) *bflag = 0;  // every thread read it after the first barrier
    __syncthreads();
  }
}

#define BCJR_BWD_CASE(KV_, V_, CODE_, UPT_)                                                  \
  if (KV == KV_ && V == V_ && code == CODE_ && upt == UPT_)                                 \
    return reinterpret_cast<const void*>(                                                   \
        &bcjr_bwd_kernel<KV_, V_, CODE_, UPT_, bwd_cached_units(KV_, V_, UPT_, CODE_),   \
                         bwd_alpha_cached_units(KV_, V_, UPT_)>);

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
  // kV = 4: whole 16-state butterflies, at most 256 per sequence (L <= 16).
  BCJR_BWD_CASE(4, 1, CODE_TABLE, 1)
  BCJR_BWD_CASE(4, 1, CODE_1MAD, 1)
  BCJR_BWD_CASE(4, 1, CODE_3INST, 1)
  BCJR_BWD_CASE(4, 2, CODE_TABLE, 1)
  BCJR_BWD_CASE(4, 2, CODE_HYB, 1)
  BCJR_BWD_CASE(4, 2, CODE_HYB_COL, 1)
  return nullptr;
}

}  // namespace bcjr
