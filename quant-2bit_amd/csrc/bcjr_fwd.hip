// Soft forward pass of the BCJR node: soft codewords E_P[c(s_t)] and log Z.
//
// Replaces the compute of bcjr_forward_backward (src/bcjr/forward_backward.py:190-232)
// and the forward of BcjrForwardBackwardMonolithic (src/bcjr/bcjr_monolithic.py:161-189).
//
// One workgroup processes one sequence at a time (grid-stride over sequences) and
// owns one scratch slot of N * NT floats in HBM.  All log values are base 2.
//
// Alpha sweep (t = 0..N-1), butterfly u of step t, raw inputs m[p] = m~_{t-1}(p*NB + u)
// (true m_{t-1} = m~_{t-1} + C_{t-1}):
//   sh = -max_p m[p];   a[p][r] = m[p] + sh + ll2_t(p*NT + R*u + r)  (<= 0)
//   m~_t(R*u + r) = log2(sum_p 2^a[p][r]) - sh - O_t   (group sum, zero shift)
//   where O_t = max_j m~_{t-1}(j) (block-uniform, from the per-wave maxima) keeps
//   values O(1), and C_t = C_{t-1} + O_t.  One exp2 per state; one log2 per group.
//   The raw inputs m[0..R-1] go to slot[t][u] (R contiguous floats): exactly
//   what the beta sweep needs at step t.
// log2 Z = C_{N-1} + LSE2_j m~_{N-1}(j).
// Beta sweep (t = N-1..0), same butterfly with the transposed data flow, raw
// inputs n[c] = n~_t(R*u + c) (true n_t = n~_t + D_t):
//   sh = -max_c n[c];  y[p][c] = n[c] + sh + ll2_t(p*NT + R*u + c)
//   e = 2^y,  n~_{t-1}(p*NB + u) = log2(sum_c e) - sh - Q_t,  D_{t-1} = D_t + Q_t
//   P_t(s) = e * 2^(m[p] - sh + K_t),  K_t = C_{t-1} + D_t - log2 Z,
//   so a marginal costs one multiply per state and one exp2 per group, and
//   soft_t = sum_s P_t(s) c(s) accumulates per thread, then per wave.
// Offsets accumulate in double on every thread (they are block-uniform).
//
// Group sums take the zero-shift form (the inputs are normalised by the
// butterfly maximum, so each term is <= 1 and needs no group maximum); a
// butterfly with any underflowed group (sum < kUnderflow) is recomputed against
// the group maxima, rare at T >= kExactBelowT; below it every group uses them.
// A unit is one whole butterfly: R inputs, R outputs, R*R states.
//
// The per-wave soft partials of a beta step are double-buffered in LDS and
// summed (in wave order) at the start of the next step, so LDS does not grow
// with N.  The diagnostics instance (INTERNALS) also writes P, log alpha and
// log beta per state when asked, and the marginal entropy -sum_s P log P of
// each step, accumulated beside the soft partials.
#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace bcjr {

template <int KV, int V, int CODE, int UPT, int CU, bool INTERNALS>
__global__ __launch_bounds__(CODE == CODE_HYB_COL ? 256 : 512, CODE == CODE_HYB_COL && !INTERNALS ? 3 : 1) void bcjr_fwd_kernel(
    FwdParams P) {
  constexpr int R = 1 << KV;
  // Butterflies of 2 or 4 states run fully unrolled with their slot inputs
  // prefetched in registers; 16-state butterflies loop over outputs (unrolled
  // too on the HYB column walk, whose LUT offsets are then immediates).
  constexpr bool kPair = R <= 4;
  static_assert(CU == 0 || kPair, "codeword cache is for butterflies of at most 4 states");
  static_assert(CU <= UPT, "at most UPT cached butterflies");
  constexpr bool kCol = CODE == CODE_HYB_COL;  // HYB column walk: one butterfly per thread
  static_assert(!kCol || (KV == 4 && UPT == 1), "the column walk is for L = 16, kV = 4");
  // Its outputs are unrolled except in the diagnostics instance, which would spill.
  constexpr bool kColUnroll = kCol && !INTERNALS;
  // Its sweeps read each state's emission (and, in the beta sweep, codeword)
  // from a per-step table, and keep one state vector, updated in place (below).
  constexpr bool kETab = kColUnroll;
  using CT = CodeTraits<CODE>;

  extern __shared__ __align__(16) unsigned char smem[];
  const int L = P.L, N = P.N;
  const int NT = 1 << (L - KV);
  const int NB = NT >> KV;
  const uint32_t ANT = opaque_uniform(CT::A * (uint32_t)NT);  // hash offset of p * NT
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
  // The column-walk instance gives thread tid butterfly col_walk_unit(tid), so
  // that its table reads hit distinct banks; elsewhere u = tid.
  const int utid = kColUnroll ? (int)col_walk_unit((uint32_t)tid) : tid;
  // kETab: the one state vector is updated in place.  At step t (either sweep)
  // butterfly u reads and writes the elements st_el(k*NB + u, rho_t), k < R,
  // rho_t = kV (t - 1) mod nb: rotr(R*u + r, kV) = r*NB + u, so its outputs land
  // on its inputs, and col_walk_state_el keeps every access conflict-free.
  const int nbits = L - KV;
  auto st_el = [&](uint32_t j, int rho) -> uint32_t { return col_walk_state_el(rotr_bits(j, rho, nbits)); };

  double* cvec = reinterpret_cast<double*>(smem);                // N    C_{t-1}
  // Reduced state (16-B aligned): 2*NT floats, double-buffered by step; kETab:
  // NT floats, then the 32 KiB table region.
  float* mbuf = reinterpret_cast<float*>(cvec + ((N + 1) & ~1));
  float* wmax = mbuf + (kETab ? NT + 8192 : 2 * NT);              // 2*kMaxWaves
  float* wsum = wmax + 2 * kMaxWaves;                             // kMaxWaves
  // Last wsum word: the block-wide input flag (at most 8 waves use wsum, launch
  // bounds 512 threads), 0 outside the check at the start of each sequence.
  int* bflag = reinterpret_cast<int*>(wsum + kMaxWaves - 1);
  float* wbuf = wsum + kMaxWaves;                                 // N*V   sequence
  // Per-wave partials of the step's soft codeword (V values) and, in the
  // diagnostics variant, of sum_s P log2 P (one more), double-buffered by step.
  constexpr int SP = V + 1;
  float* spart = wbuf + N * V;                                    // 2*nwaves*SP per-wave partials
  // HYB: signed LUT (code_hyb_signed) or column-walk LUT (hyb_col_base), 8-byte
  // aligned; kETab: the per-step tables after the state vector, 16-byte aligned.
  float* lut = kETab ? mbuf + NT
                     : reinterpret_cast<float*>(smem) +
                           ((spart + 2 * nwaves * SP - reinterpret_cast<float*>(smem) + 1) & ~1);

  if constexpr (CODE == CODE_HYB) {
    stage_hyb_signed(reinterpret_cast<float2*>(lut), P.table, P.Q, tid, nthr);
    __syncthreads();
  } else if constexpr (kCol && !kETab) {
    stage_hyb_col(reinterpret_cast<float2*>(lut), P.table, P.Q, tid, nthr);
    __syncthreads();
  }
  const unsigned char* lutb = reinterpret_cast<const unsigned char*>(lut);
  float2* hcomp = reinterpret_cast<float2*>(lut + 4096);  // kETab, alpha sweep
  // Per-step tables of the column walk, in the 32 KiB region.  Alpha sweep:
  // float k of the table (the column-walk layout: 32 rows of 64, rows 16..31
  // repeating 0..15) holds the emission -|d|^2 of LUT entry k, d = c sk - w_t sk;
  // two tables, for the step parities, take 16 KiB.  State s's emission sits at
  // a quarter of the byte its codeword would have in a float4 table (plus 8 KiB
  // for odd steps), and a wave's 64 reads fall in distinct banks (col_walk_unit).
  // Beta sweep: one float4 table, entry k = (c, -|d|^2, 0) of LUT entry k, whose
  // emissions are rewritten per step behind a barrier.  The kernel runs 256
  // threads here; thread tid forms entries tid + 256j (j < 4) and their row
  // copies.  The codewords come from the LDS: during the alpha sweep from a
  // float2 copy of LUT entries 0..1023 in the region's second half (hcomp,
  // filled per sequence from the (2^Q, 2) table as stage_hyb_col forms them),
  // during the beta sweep from the float4 table itself.
  auto col_codeword = [&](int kk, float& h0, float& h1) {
    const int ncol = 1 << (P.Q - 3), mask = (1 << P.Q) - 1;
    const int col = kk & 63, ii = col + ncol * (kk >> 6), ie = ii & mask;
    h0 = col < ncol ? P.table[2 * ie] : 0.0f;
    const float y = col < ncol ? P.table[2 * ie + 1] : 0.0f;
    h1 = (ii >> P.Q) ? -y : y;
  };
  // Column-walk bases of this thread's butterfly u = utid, input c (state R*u + c)
  // (kETab: doubled, the float4 table's byte of the row 0 entry).
  uint32_t cbs[kCol ? R : 1];
  if constexpr (kCol) {
#pragma unroll
    for (int c = 0; c < R; ++c) cbs[c] = hyb_col_base((uint32_t)(R * min(utid, NB - 1) + c), P.Q) << (kETab ? 1 : 0);
  }

  // Raw codewords h of this thread's first CU butterflies, fixed for the
  // whole launch; the others are hashed per state.
  float hc[CU > 0 ? CU : 1][CU > 0 ? R : 1][CU > 0 ? R : 1][V];
  if constexpr (CU > 0) {
#pragma unroll
    for (int i = 0; i < CU; ++i) {
      const int u = min(utid + i * nthr, NB - 1);
      const uint32_t xu = CT::A * (uint32_t)(R * u) + CT::B;
#pragma unroll
      for (int p = 0; p < R; ++p)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t s = (uint32_t)(p * NT + R * u + r);
          raw_codeword<CODE, V>(xu, CT::A * (uint32_t)(p * NT + r), s, P.table, lut, P.Q, hc[i][p][r]);
        }
    }
  }

  if (tid == 0) *bflag = 0;
  __syncthreads();

  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    float* slot = P.ws + (size_t)blockIdx.x * (size_t)N * (size_t)NT;
    const float Tb = P.T[P.t_per_seq ? b : 0];
    const float sk = sqrtf(kLog2e / Tb);
    const float ssk = CT::kSigma * sk;  // d = (c - w) * sk = h * ssk - w * sk
    const float* seqb = P.seq + (size_t)b * N * V;
    float* softb = P.soft + (size_t)b * N * V;
    // Soft codeword of step t and, in the diagnostics variant, its marginal
    // entropy in nats (-ln 2 * sum_s P log2 P), from the per-wave sums in partial
    // buffer `par`; called by wave 0.
    auto step_out = [&](int t, int par) {
      const float* sp = spart + par * nwaves * SP;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float sacc = sum_of_waves(sp + v, nwaves, SP);
        if (lane == 0) softb[t * V + v] = sacc;
      }
      if (INTERNALS && P.H_out) {
        const float h = sum_of_waves(sp + V, nwaves, SP);
        if (lane == 0) P.H_out[(size_t)b * N + t] = -h * (float)kLn2;
      }
    };
    // T must be finite and > 0 and the weights finite; otherwise the sequence's
    // outputs are NaN (the check is one barrier per sequence).
    int bad = !(Tb > 0.0f && Tb < INFINITY);
    for (int i = tid; i < N * V; i += nthr) {
      const float w = seqb[i];
      wbuf[i] = w;
      bad |= !__builtin_isfinite(w);
    }
    // m~_{-1} = log2(R) everywhere: the buffer step 0 reads from.
    for (int j = tid; j < NT; j += nthr) mbuf[(kETab ? 0 : NT) + j] = (float)KV;
    if constexpr (kETab) {  // the previous sequence's last barrier ended every table read
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float h0, h1;
        col_codeword(tid + 256 * j, h0, h1);
        hcomp[tid + 256 * j] = make_float2(h0, h1);
      }
    }
    if (tid < 2 * kMaxWaves) wmax[tid] = -INFINITY;  // waves that do not exist
    if (bad) *bflag = 1;
    __syncthreads();
    if (*bflag) {  // uniform: every thread reads the flag after the barrier
      for (int i = tid; i < N * V; i += nthr) softb[i] = NAN;
      if (tid == 0 && P.logZ) P.logZ[b] = NAN;
      if constexpr (INTERNALS) {
        if (P.H_out)
          for (int t = tid; t < N; t += nthr) P.H_out[(size_t)b * N + t] = NAN;
        if (P.P_out) {
          const size_t per = (size_t)N << L;
          for (size_t i = tid; i < per; i += nthr) {
            P.P_out[(size_t)b * per + i] = NAN;
            P.la_out[(size_t)b * per + i] = NAN;
            P.lb_out[(size_t)b * per + i] = NAN;
          }
        }
      }
      __syncthreads();
      if (tid == 0) *bflag = 0;
      __syncthreads();
      continue;
    }

    double logZ2 = 0.0;
    // Below kExactBelowT most groups would underflow the zero-shift sums, so
    // the whole sequence uses the group maxima.  The choice is a uniform branch
    // around both sweeps: each variant gets its own register allocation.
    auto sweeps = [&](auto exact_tag) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      using Fast = std::integral_constant<bool, EXACT>;

      // ------------------------------ alpha sweep ------------------------------
      // Emission table of step t into table t & 1 (kETab).
      auto build_etab = [&](int t) {
        float nwt[V];
#pragma unroll
        for (int v = 0; v < V; ++v) nwt[v] = -wbuf[t * V + v] * sk;
        float* et = lut + 2048 * (t & 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float2 h = hcomp[tid + 256 * j];
          const float d0 = fmaf(h.x, ssk, nwt[0]);
          const float d1 = fmaf(h.y, ssk, nwt[1]);
          const float e = fmaf(-d1, d1, fmaf(-d0, d0, 0.0f));
          const int k = tid + 256 * j;
          et[k] = e;
          et[k + 1024] = e;
        }
      };
      if constexpr (kETab) {
        build_etab(0);
        __syncthreads();
      }
      double C = 0.0;  // C_{t-1}
      int k = 0;       // step counter across both sweeps: LDS buffer / wmax parity
      int rho = nbits - KV;  // kV (t - 1) mod nb at t = 0 (kETab)
      for (int t = 0; t < N; ++t, ++k) {
        const float* prev = mbuf + (kETab ? 0 : ((k + 1) & 1) * NT);
        float* cur = mbuf + (kETab ? 0 : (k & 1) * NT);
        // kETab: element st_el(k*NB + u, rho) = ebase ^ Kel[k] of butterfly u = utid
        const uint32_t ebase = kETab ? st_el((uint32_t)utid, rho) : 0u;
        uint32_t Kel[kETab ? R : 1];
        if constexpr (kETab) {
#pragma unroll
          for (int q = 0; q < R; ++q) Kel[q] = st_el((uint32_t)(q * NB), rho);
        }
        float O = (float)KV;  // m~_{-1} = log2(R) for every j
        if (t > 0) {
          O = -INFINITY;
          O = block_max(wmax + ((k + 1) & 1) * kMaxWaves);
        }
        if (tid == 0) cvec[t] = C;
        C += (double)O;
        float nw[V];
#pragma unroll
        for (int v = 0; v < V; ++v) nw[v] = -wbuf[t * V + v] * sk;
        // The next step's emission table goes where step t - 1's was, which
        // every wave has left (barrier at the end of each step).
        if (kETab && t + 1 < N) build_etab(t + 1);
        const uint32_t eoff = 8192u * (uint32_t)(t & 1);

        // Output r of butterfly u (unit i) from the shifted inputs m[p]
        // (maximum 0): returns the group sum, mo = m~_t(R*u + r).
        // cb: the column-walk base of state R*u + r (kCol only).
        auto alpha_out = [&](auto shift_tag, int i, int r, uint32_t xu, int u, const float (&m)[R], float oout,
                             float& mo, uint32_t cb) -> float {
          constexpr bool SHIFT = decltype(shift_tag)::value;
          float a[R];
#pragma unroll
          for (int p = 0; p < R; ++p) {
            float acc = m[p];
            // The two-rounding d_3inst form is kept out of the low-temperature
            // variant, where |d| reaches ~1e2 and float32 precision is tightest.
            const bool cached = i < CU;
            if constexpr (kETab) {  // cb: the table byte of state R*u + r's row 0 entry
              acc += *reinterpret_cast<const float*>(lutb + cb + (hyb_col_step(p, r) >> 1));
            } else if (!cached && CODE == CODE_3INST && !EXACT) {
              const float d = d_3inst(xu + p * ANT + CT::A * (uint32_t)r, ssk, nw[0]);
              acc = fmaf(-d, d, acc);
            } else {
              float h[V];
              if (cached) {
#pragma unroll
                for (int v = 0; v < V; ++v) h[v] = hc[cached ? i : 0][p][r][v];
              } else if constexpr (kCol) {
                const float2 cw = hyb_col_read(lutb, cb + hyb_col_step(p, r));
                h[0] = cw.x;
                h[1] = cw.y;
              } else {
                raw_codeword<CODE, V>(xu, p * ANT + CT::A * (uint32_t)r, (uint32_t)(p * NT + R * u + r), P.table,
                                      lut, P.Q, h);
              }
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const float d = fmaf(h[v], ssk, nw[v]);
                acc = fmaf(-d, d, acc);
              }
            }
            a[p] = acc;
          }
          float M = 0.0f;
          if constexpr (SHIFT) {
            M = max_of_inputs(a);
          }
          float s = fexp2(a[0] - M);
#pragma unroll
          for (int p = 1; p < R; ++p) s += fexp2(a[p] - M);
          mo = flog2(s) + (M - oout);
          return s;
        };

        // Inputs of butterfly utid + i*nthr; the next butterfly's are read
        // before the current one's arithmetic (prev is read-only this step; in
        // place, a thread's elements are its own).
        auto read_in = [&](int i, float (&m)[R]) {
          const int qq = min(utid + i * nthr, NB - 1);
          if constexpr (kETab) {
#pragma unroll
            for (int p = 0; p < R; ++p) m[p] = prev[ebase ^ Kel[p]];
          } else {
#pragma unroll
            for (int p = 0; p < R; ++p) m[p] = prev[p * NB + qq];
          }
        };
        float nx[R];
        read_in(0, nx);
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
          const int q = utid + i * nthr;
          float m[R];
#pragma unroll
          for (int p = 0; p < R; ++p) m[p] = nx[p];
          if (i + 1 < UPT) read_in(i + 1, nx);
          if (q < NB) {
            const int u = i < CU ? q : opaque(q);
            store_vec<R>(slot + ((size_t)t * NB + u) * R, m);
            const float Mu = max_of_inputs(m);
            const float sh = -Mu;
#pragma unroll
            for (int p = 0; p < R; ++p) m[p] += sh;
            const uint32_t xu = CT::A * (uint32_t)(R * u) + CT::B;
            const float oout = sh + O;
            if constexpr (kPair) {
              float mo[R], smin = 0.0f;
#pragma unroll
              for (int r = 0; r < R; ++r) {
                const float s = alpha_out(Fast{}, i, r, xu, u, m, oout, mo[r], 0u);
                smin = r ? fminf(smin, s) : s;
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
#pragma unroll
                  for (int r = 0; r < R; ++r) alpha_out(std::true_type{}, i, r, xu, u, m, oout, mo[r], 0u);
                }
              }
              store_vec<R>(cur + R * u, mo);
              tmax = max_with(tmax, mo);
            } else if constexpr (kColUnroll) {
              // Outputs unrolled, so every state's LUT offset is an immediate;
              // a butterfly with an underflowed group is redone output by output.
              float smin = 0.0f;
#pragma unroll
              for (int r = 0; r < R; ++r) {
                float mo;
                const float s = alpha_out(Fast{}, i, r, xu, u, m, oout, mo, (cbs[r] >> 2) + eoff);
                smin = r ? fminf(smin, s) : s;
                cur[ebase ^ Kel[r]] = mo;
                tmax = vmax_raw(tmax, mo);
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
#pragma unroll 1
                  for (int r = 0; r < R; ++r) {
                    float mo;
                    alpha_out(std::true_type{}, i, r, xu, u, m, oout, mo,
                              (hyb_col_base((uint32_t)(R * u + r), P.Q) >> 1) + eoff);
                    cur[ebase ^ Kel[r]] = mo;
                    tmax = vmax_raw(tmax, mo);
                  }
                }
              }
            } else {
#pragma unroll 1
              for (int r = 0; r < R; ++r) {
                float mo;
                const uint32_t cb = kCol ? hyb_col_base((uint32_t)(R * u + r), P.Q) : 0u;
                const float s = alpha_out(Fast{}, i, r, xu, u, m, oout, mo, cb);
                if (!EXACT && s < kUnderflow) alpha_out(std::true_type{}, i, r, xu, u, m, oout, mo, cb);
                cur[R * u + r] = mo;
                tmax = vmax_raw(tmax, mo);
              }
            }
          }
        }
        tmax = wave_max(tmax);
        if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
        rho = rho + KV >= nbits ? rho + KV - nbits : rho + KV;
        __syncthreads();
      }

      // kETab: this thread's codewords, before the float4 table overwrites hcomp
      float2 hv[kETab ? 4 : 1];
      if constexpr (kETab) {
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = hcomp[tid + 256 * j];
      }

      // log2 Z = C_{N-1} + LSE2 over the final reduced state.
      const float* fin = mbuf + (kETab ? 0 : ((k + 1) & 1) * NT);
      float Mz = -INFINITY;
      Mz = block_max(wmax + ((k + 1) & 1) * kMaxWaves);
      float part = 0.0f;
      for (int j = tid; j < NT; j += nthr) part += fexp2(fin[j] - Mz);
      part = wave_sum(part);
      if (lane == 0) wsum[wave] = part;
      __syncthreads();
      float Ssum = 0.0f;
      for (int w = 0; w < nwaves; ++w) Ssum += wsum[w];
      logZ2 = C + (double)Mz + (double)flog2(Ssum);
      // n~_{N-1} = 0: the buffer step N-1 of the beta sweep reads from.
      for (int j = tid; j < NT; j += nthr) mbuf[(kETab ? 0 : ((k + 1) & 1) * NT) + j] = 0.0f;
      if constexpr (kETab) {  // codewords of the float4 table (every wave read hcomp before the barrier above)
        float4* et = reinterpret_cast<float4*>(lut);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kk = tid + 256 * j;
          et[kk] = make_float4(hv[j].x, hv[j].y, 0.0f, 0.0f);
          et[kk + 1024] = make_float4(hv[j].x, hv[j].y, 0.0f, 0.0f);
        }
      }
      __syncthreads();

      // ------------------------------ beta sweep -------------------------------
      // Raw alpha inputs of step t come back from HBM two butterflies ahead of
      // their use, across step boundaries (the next two in consumption order:
      // t descending, i ascending).
      auto slot_src = [&](int t, int i) {
        const int q = min(utid + i * nthr, NB - 1);
        return slot + ((size_t)t * NB + q) * R;
      };
      float pa[R], pb[R];
      if constexpr (kPair) {
        load_vec<R>(slot_src(N - 1, 0), pa);
        if (UPT > 1 || N > 1) load_vec<R>(UPT > 1 ? slot_src(N - 1, 1) : slot_src(N - 2, 0), pb);
      }
      double D = 0.0;  // D_t
      // rho_t = kV * (t - 1) mod nb at t = N - 1 (kETab)
      rho = (int)(((long long)KV * (N - 2) % nbits + nbits) % nbits);
      for (int t = N - 1; t >= 0; --t, ++k) {
        const float* prev = mbuf + (kETab ? 0 : ((k + 1) & 1) * NT);
        float* cur = mbuf + (kETab ? 0 : (k & 1) * NT);
        const uint32_t ebase = kETab ? st_el((uint32_t)utid, rho) : 0u;
        uint32_t Kel[kETab ? R : 1];
        if constexpr (kETab) {
#pragma unroll
          for (int q = 0; q < R; ++q) Kel[q] = st_el((uint32_t)(q * NB), rho);
        }
        float Qv = 0.0f;
        if (t != N - 1) {
          Qv = -INFINITY;
          Qv = block_max(wmax + ((k + 1) & 1) * kMaxWaves);
          // soft of step t+1 from its per-wave partials (the other parity buffer)
          if (wave == 0) step_out(t + 1, (k + 1) & 1);
        }
        const float Kt = (float)(cvec[t] + D - logZ2);
        float nw[V];
#pragma unroll
        for (int v = 0; v < V; ++v) nw[v] = -wbuf[t * V + v] * sk;
        if constexpr (kETab) {  // every wave has left step t+1's table (barrier at its end)
          float4* et = reinterpret_cast<float4*>(lut);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int kk = tid + 256 * j;
            const float2 h = *reinterpret_cast<const float2*>(&et[kk]);
            const float d0 = fmaf(h.x, ssk, nw[0]);
            const float d1 = fmaf(h.y, ssk, nw[1]);
            const float e = fmaf(-d1, d1, fmaf(-d0, d0, 0.0f));
            et[kk].z = e;
            et[kk + 1024].z = e;
          }
          __syncthreads();
        }

        // Output p of butterfly u (unit i) from the shifted inputs nr[c]
        // (maximum 0): no = n~_{t-1}(p*NB + u) and the soft contribution
        // G * sum_c e_c h_c, with pms = raw m~_{t-1}(p*NB + u) + K_t - sh.
        // n holds the raw inputs and pmr the raw m~ (diagnostics only).
        // hs = sum over the output's R states of P log2 P (diagnostics variant).
        auto beta_out = [&](auto shift_tag, int i, int p, uint32_t xu, int u, const float (&nr)[R],
                            const float (&n)[R], float pms, float pmr, float oout, float& no,
                            float (&cs)[V], float& hs) -> float {
          constexpr bool SHIFT = decltype(shift_tag)::value;
          float y[R], hh[R][V];
#pragma unroll
          for (int c = 0; c < R; ++c) {
            if constexpr (kETab) {
              const float4 he = *reinterpret_cast<const float4*>(lutb + cbs[c] + 2 * hyb_col_step(p, c));
              y[c] = nr[c] + he.z;
              hh[c][0] = he.x;
              hh[c][1] = he.y;
              continue;
            }
            if (i < CU) {
#pragma unroll
              for (int v = 0; v < V; ++v) hh[c][v] = hc[i < CU ? i : 0][p][c][v];
            } else if constexpr (kCol) {
              const float2 cw = hyb_col_read(lutb, cbs[c] + hyb_col_step(p, c));
              hh[c][0] = cw.x;
              hh[c][1] = cw.y;
            } else {
              raw_codeword<CODE, V>(xu, p * ANT + CT::A * (uint32_t)c, (uint32_t)(p * NT + R * u + c), P.table,
                                    lut, P.Q, hh[c]);
            }
            float yy = nr[c];
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float d = fmaf(hh[c][v], ssk, nw[v]);
              yy = fmaf(-d, d, yy);
            }
            y[c] = yy;
          }
          float M = 0.0f;
          if constexpr (SHIFT) {
            M = max_of_inputs(y);
          }
          float e[R], s = 0.0f, ec[V];
#pragma unroll
          for (int c = 0; c < R; ++c) {
            e[c] = fexp2(y[c] - M);
            s = c ? s + e[c] : e[c];
#pragma unroll
            for (int v = 0; v < V; ++v) ec[v] = c ? fmaf(e[c], hh[c][v], ec[v]) : e[c] * hh[c][v];
          }
          const float G = fexp2(pms + M);
#pragma unroll
          for (int v = 0; v < V; ++v) cs[v] = G * ec[v];
          no = flog2(s) + (M - oout);
          hs = 0.0f;
          if constexpr (INTERNALS) {  // diagnostics: P, log alpha, log beta in nats; entropy
            if (P.P_out) {
              const float Ct = (float)cvec[t];
              const float Dt = (float)D;
              const size_t base = ((size_t)b * N + t) * ((size_t)NT << KV) + (size_t)p * NT + (size_t)R * u;
#pragma unroll
              for (int c = 0; c < R; ++c) {
                P.P_out[base + c] = e[c] * G;
                P.la_out[base + c] = (y[c] - nr[c] + pmr + Ct) * (float)kLn2;
                P.lb_out[base + c] = (n[c] + Dt) * (float)kLn2;
              }
            }
            // log2 P of state c is y[c] - M + (pms + M) = y[c] + pms, so
            // sum_c P log2 P = G (sum_c e_c y_c + pms s).
            float ey = 0.0f;
#pragma unroll
            for (int c = 0; c < R; ++c) ey = fmaf(e[c], y[c], ey);
            hs = G * fmaf(pms, s, ey);
          }
          return s;
        };

        auto read_in = [&](int i, float (&n)[R]) {
          const int qq = min(utid + i * nthr, NB - 1);
          if constexpr (kETab) {
#pragma unroll
            for (int c = 0; c < R; ++c) n[c] = prev[ebase ^ Kel[c]];
          } else {
            load_vec<R>(prev + R * qq, n);
          }
        };
        float nx[R];
        read_in(0, nx);
        float acc[V], hacc = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] = 0.0f;
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
          const int q = utid + i * nthr;
          float pm[R], n[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            n[r] = nx[r];
            if constexpr (kPair) {
              pm[r] = pa[r];
              pa[r] = pb[r];
            }
          }
          if constexpr (kPair) {  // fetch the butterfly two ahead
            const int tt = i + 2 < UPT ? t : t - 1 - (i + 2 - UPT) / UPT;
            const int ii = i + 2 < UPT ? i + 2 : (i + 2 - UPT) % UPT;
            if (tt >= 0) load_vec<R>(slot_src(tt, ii), pb);
          }
          if (i + 1 < UPT) read_in(i + 1, nx);
          if (q < NB) {
            const int u = i < CU ? q : opaque(q);
            const float Mu = max_of_inputs(n);
            const float sh = -Mu;
            float nr[R];
#pragma unroll
            for (int c = 0; c < R; ++c) nr[c] = n[c] + sh;
            const uint32_t xu = CT::A * (uint32_t)(R * u) + CT::B;
            const float oout = sh + Qv;
            const float kts = Kt - sh;
            if constexpr (kPair) {
              float no[R], smin = 0.0f, ua[V], uh = 0.0f;
#pragma unroll
              for (int v = 0; v < V; ++v) ua[v] = 0.0f;
#pragma unroll
              for (int p = 0; p < R; ++p) {
                float cs[V], hs;
                const float s = beta_out(Fast{}, i, p, xu, u, nr, n, pm[p] + kts, pm[p], oout, no[p], cs, hs);
                smin = p ? fminf(smin, s) : s;
#pragma unroll
                for (int v = 0; v < V; ++v) ua[v] += cs[v];
                uh += hs;
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
                  uh = 0.0f;
#pragma unroll
                  for (int v = 0; v < V; ++v) ua[v] = 0.0f;
#pragma unroll
                  for (int p = 0; p < R; ++p) {
                    float cs[V], hs;
                    beta_out(std::true_type{}, i, p, xu, u, nr, n, pm[p] + kts, pm[p], oout, no[p], cs, hs);
#pragma unroll
                    for (int v = 0; v < V; ++v) ua[v] += cs[v];
                    uh += hs;
                  }
                }
              }
              hacc += uh;
#pragma unroll
              for (int v = 0; v < V; ++v) acc[v] += ua[v];
#pragma unroll
              for (int p = 0; p < R; ++p) {
                cur[p * NB + u] = no[p];
              }
              tmax = max_with(tmax, no);
            } else if constexpr (kColUnroll) {
              // Outputs unrolled, so every state's LUT offset is an immediate;
              // the butterfly's sums are redone when a group underflowed.
              const float* src = slot_src(t, i);
              float smin = 0.0f, ua[V], uh = 0.0f;
#pragma unroll
              for (int v = 0; v < V; ++v) ua[v] = 0.0f;
#pragma unroll
              for (int p = 0; p < R; ++p) {
                float no, cs[V], hs;
                const float pmr = src[p];
                const float s = beta_out(Fast{}, i, p, xu, u, nr, n, pmr + kts, pmr, oout, no, cs, hs);
                smin = p ? fminf(smin, s) : s;
#pragma unroll
                for (int v = 0; v < V; ++v) ua[v] += cs[v];
                uh += hs;
                cur[ebase ^ Kel[p]] = no;
                tmax = vmax_raw(tmax, no);
              }
              if constexpr (!EXACT) {
                if (smin < kUnderflow) {
                  uh = 0.0f;
#pragma unroll
                  for (int v = 0; v < V; ++v) ua[v] = 0.0f;
#pragma unroll 1
                  for (int p = 0; p < R; ++p) {
                    float no, cs[V], hs;
                    const float pmr = src[p];
                    beta_out(std::true_type{}, i, p, xu, u, nr, n, pmr + kts, pmr, oout, no, cs, hs);
#pragma unroll
                    for (int v = 0; v < V; ++v) ua[v] += cs[v];
                    uh += hs;
                    cur[ebase ^ Kel[p]] = no;
                    tmax = vmax_raw(tmax, no);
                  }
                }
              }
              hacc += uh;
#pragma unroll
              for (int v = 0; v < V; ++v) acc[v] += ua[v];
            } else {
              const float* src = slot_src(t, i);
#pragma unroll 1
              for (int p = 0; p < R; ++p) {
                float no, cs[V], hs;
                const float pmr = src[p];
                const float s = beta_out(Fast{}, i, p, xu, u, nr, n, pmr + kts, pmr, oout, no, cs, hs);
                if (!EXACT && s < kUnderflow)
                  beta_out(std::true_type{}, i, p, xu, u, nr, n, pmr + kts, pmr, oout, no, cs, hs);
#pragma unroll
                for (int v = 0; v < V; ++v) acc[v] += cs[v];
                hacc += hs;
                cur[p * NB + u] = no;
                tmax = vmax_raw(tmax, no);
              }
            }
          }
        }
        D += (double)Qv;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float s = wave_sum(acc[v]);
          if (lane == 0) spart[((k & 1) * nwaves + wave) * SP + v] = s * CT::kSigma;
        }
        if constexpr (INTERNALS) {
          const float h = wave_sum(hacc);
          if (lane == 0) spart[((k & 1) * nwaves + wave) * SP + V] = h;
        }
        tmax = wave_max(tmax);
        if (lane == 0) wmax[(k & 1) * kMaxWaves + wave] = tmax;
        rho = rho - KV < 0 ? rho - KV + nbits : rho - KV;
        __syncthreads();
      }
    };
    if (Tb < kExactBelowT) {
      sweeps(std::true_type{});
    } else {
      sweeps(std::false_type{});
    }

    // soft of step 0: its partials sit in the buffer of the last beta step's parity
    const int par0 = (2 * N - 1) & 1;  // k after N alpha and N beta steps, minus one
    if (wave == 0) step_out(0, par0);
    if (tid == 0 && P.logZ) P.logZ[b] = (float)(logZ2 * kLn2);
    if (tid == 0) *bflag = 0;  // every thread read it after the first barrier
    __syncthreads();
  }
}

// The diagnostics variant carries more live values per butterfly, so it caches
// codewords within the backward's smaller register budget.
#define BCJR_FWD_CASE(KV_, V_, CODE_, UPT_)                                                      \
  if (KV == KV_ && V == V_ && code == CODE_ && upt == UPT_) {                                   \
    constexpr int CU_ = fwd_cached_units(KV_, V_, UPT_);                                        \
    constexpr int CUD_ = bwd_cached_units(KV_, V_, UPT_);                                       \
    return internals ? reinterpret_cast<const void*>(&bcjr_fwd_kernel<KV_, V_, CODE_, UPT_, CUD_, true>) \
                     : reinterpret_cast<const void*>(&bcjr_fwd_kernel<KV_, V_, CODE_, UPT_, CU_, false>); \
  }

#define BCJR_FWD_UPTS(KV_, V_, CODE_) \
  BCJR_FWD_CASE(KV_, V_, CODE_, 1)    \
  BCJR_FWD_CASE(KV_, V_, CODE_, 2)    \
  BCJR_FWD_CASE(KV_, V_, CODE_, 4)    \
  BCJR_FWD_CASE(KV_, V_, CODE_, 8)

const void* fwd_kernel_ptr(int KV, int V, int code, int upt, bool internals) {
  BCJR_FWD_CASE(1, 1, CODE_TABLE, 1)  // kV = 1: k = 1, V = 1 (L <= 11)
  BCJR_FWD_UPTS(2, 1, CODE_TABLE)
  BCJR_FWD_UPTS(2, 1, CODE_1MAD)
  BCJR_FWD_UPTS(2, 1, CODE_3INST)
  BCJR_FWD_UPTS(2, 2, CODE_TABLE)
  BCJR_FWD_UPTS(2, 2, CODE_HYB)
  // kV = 4: whole 16-state butterflies, at most 256 per sequence (L <= 16).
  BCJR_FWD_CASE(4, 1, CODE_TABLE, 1)
  BCJR_FWD_CASE(4, 1, CODE_1MAD, 1)
  BCJR_FWD_CASE(4, 1, CODE_3INST, 1)
  BCJR_FWD_CASE(4, 2, CODE_TABLE, 1)
  BCJR_FWD_CASE(4, 2, CODE_HYB, 1)
  BCJR_FWD_CASE(4, 2, CODE_HYB_COL, 1)
  return nullptr;
}

}  // namespace bcjr
