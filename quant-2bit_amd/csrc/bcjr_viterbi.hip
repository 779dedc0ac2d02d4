// T -> 0 mode of the node: min-sum Viterbi on the bitshift trellis, traceback,
// reconstruction, MSE and kV-bit packing, plus walk replay and codebook fill.
//
// Replaces viterbi_encode_v_batched_cuda (src/viterbi/cuda_kernel.py:166-220) and
// follows the semantics of the numpy encoder viterbi_encode_v
// (src/viterbi/encode.py:250-307), which fixes the float32 rounding and tie rules:
//   cum_0 = 0;  cum_t(s) = fl( min_p cum_{t-1}(p*NT + (s >> kV)) + E_t(s) ),
//   E_t(s)  = fl( sum_v fl( fl(c_v(s) - w_t[v])^2 ) )     (no FMA contraction),
//   the lowest p wins a tie, the lowest final state wins a tie,
//   walk_{t-1} = argmin_p cum_{t-1}(p*NT + (walk_t >> kV)) * NT + (walk_t >> kV),
//   start = bp_0(walk_0 >> kV) * NT + (walk_0 >> kV) = walk_0 >> kV,
//   bitstream_t = walk_t & (2^kV - 1), recon_t = c(walk_t).
// Min-sum has no transcendentals; the butterfly layout and the per-step LDS
// exchange are those of the soft kernels.  Backpointers (kV bits per reduced
// state and step where a thread's outputs fill a byte or half-word, else one
// byte) go to the caller's workspace and are staged back through LDS, as many
// rows as the 2*NT-float state buffers hold (32 at L=16, kV=2), for the
// traceback.  bcjr_viterbi_constrained adds the tail-biting constraint of
// encode.py:328-389 through the initial cost vector and the final argmin.
#pragma clang fp contract(off)

#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace bcjr {

// The cost of a state the tail-biting constraint excludes (float32(1e18), as
// in src/viterbi/encode.py:124); a sum with it rounds back to it.
constexpr float kVitInf = 1e18f;

// Strict (value, index) order: smaller value first, then lower index.
__device__ __forceinline__ bool vi_less(float a, int ia, float b, int ib) {
  return (a < b) || (a == b && ia < ib);
}

// MAXT is the largest workgroup the instance is built for: 1024 threads (four
// waves per SIMD, at most 128 VGPRs) where the codeword cache fits that budget,
// else 512.
template <int KV, int V, int CODE, int UPT, bool CACHE, int MAXT>
__global__ __launch_bounds__(MAXT) void bcjr_viterbi_kernel(VitParams P) {
  constexpr int R = 1 << KV;
  constexpr int RO = R < 4 ? R : 4;
  constexpr int NSUB = R / RO;
  // Backpointers: kV bits per reduced state when a thread's RO outputs fill a
  // whole byte or half-word (kV = 2, 4), else one byte per state.
  constexpr bool PACK = RO * KV == 8 || RO * KV == 16;
  static_assert(!CACHE || NSUB == 1, "codeword cache needs whole butterflies per thread");

  extern __shared__ __align__(16) unsigned char smem[];
  const int L = P.L, N = P.N;
  const int NT = 1 << (L - KV);
  const int NB = NT >> KV;
  const int NU = NB * NSUB;
  const int lgNB = L - 2 * KV;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;

  double* redd = reinterpret_cast<double*>(smem);             // kMaxWaves
  float* rbuf = reinterpret_cast<float*>(redd + kMaxWaves);    // 2*NT (also traceback staging)
  float* wbuf = rbuf + 2 * NT;                                 // N*V
  float* redv = wbuf + N * V;                                  // kMaxWaves
  int* redi = reinterpret_cast<int*>(redv + kMaxWaves);        // kMaxWaves
  int* walkbuf = redi + kMaxWaves;                             // N
  // HYB LUT (16-byte aligned).  The uncached 1024-thread instances (kV = 4),
  // which look up a codeword per state and step, keep the signed LUT
  // (code_hyb_signed: index and sign in one bit field) as 2^rep interleaved
  // copies, lane l reading copy l mod 2^rep (code_hyb_signed_rep); the others,
  // whose codewords are cached or rarely formed, one plain copy.
  constexpr bool kSignedRep = (CODE == CODE_HYB) && !CACHE && MAXT == 1024;
  // CODE_HYB_COL (L = 16, kV = 4): the column-walk LUT (hyb_col_base) as
  // 2^kColRep interleaved copies, so a state's codeword is the thread's base for
  // its output plus a wave-uniform row step, with no per-state index arithmetic.
  constexpr bool kColV = CODE == CODE_HYB_COL;
  static_assert(!kColV || (KV == 4 && V == 2 && UPT == 1 && !CACHE), "the column walk is for L = 16, kV = 4");
  constexpr int kColRep = 2;
  const size_t lut_off = ((size_t)(reinterpret_cast<unsigned char*>(walkbuf + N) - smem) + 15) & ~(size_t)15;
  float2* lut2 = reinterpret_cast<float2*>(smem + lut_off);
  const float* lut = reinterpret_cast<const float*>(lut2);
  const int rep = kSignedRep ? hyb_lut_rep(P.Q) : (kColV ? kColRep : 0);
  const uint32_t copy = (uint32_t)lane & ((1u << rep) - 1u);
  // c(s) for the state loops: HYB through the LDS LUT, other codes as codeword().
  auto cword = [&](uint32_t s, float (&c)[V]) {
    if constexpr (kColV) {
      const uint32_t x = __umul24(s, s) + s;
      const uint32_t e = (((x >> 12) & 15u) << 6) | ((x >> (15 - P.Q)) & ((1u << (P.Q - 3)) - 1u));
      const float2 v = lut2[(e << kColRep) | copy];
      c[0] = v.x;
      c[1] = v.y;
    } else if constexpr (kSignedRep) {
      code_hyb_signed_rep(s, lut2, P.Q, rep, copy, c[0], c[1]);
    } else if constexpr (CODE == CODE_HYB) {
      code_hyb(s, lut, P.Q, c[0], c[1]);
    } else {
      codeword<CODE, V>(s, P.table, lut, P.Q, c);
    }
  };

  // Column-walk LUT entry k (row k >> 6 mod 16, column k & 63) as stage_hyb_col
  // forms it from the (2^Q, 2) table.
  auto col_entry = [&](int k) -> float2 {
    const int ncol = 1 << (P.Q - 3), mask = (1 << P.Q) - 1;
    const int col = k & 63, si = col + ncol * ((k >> 6) & 15);
    float2 v = make_float2(0.0f, 0.0f);
    if (col < ncol) {
      const int e = si & mask;
      const float y = P.table[2 * e + 1];
      v = make_float2(P.table[2 * e], (si >> P.Q) ? -y : y);
    }
    return v;
  };
  // The column-walk LUT's copies, staged after each sequence's state loop, which
  // holds per-step cost tables in their place (below), for the final pass and
  // the traceback.
  auto stage_col = [&]() {
    for (int i = tid; i < (32 * 64) << kColRep; i += nthr) lut2[i] = col_entry(i >> kColRep);
  };
  if constexpr (kSignedRep) {
    const int nl = (2 << P.Q) << rep, mask = (1 << P.Q) - 1;
    for (int i = tid; i < nl; i += nthr) {
      const int si = i >> rep, e = si & mask;
      const float y = P.table[2 * e + 1];
      lut2[i] = make_float2(P.table[2 * e], (si >> P.Q) ? -y : y);
    }
    __syncthreads();
  } else if constexpr (CODE == CODE_HYB) {
    const int nl = 2 << P.Q;
    float* lutw = reinterpret_cast<float*>(lut2);
    for (int i = tid; i < nl; i += nthr) lutw[i] = P.table[i];
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
          cword((uint32_t)(p * NT + R * u + r), cw[i][p][r]);
    }
  }

  // Column-walk byte bases of this thread's RO outputs (unit tid: sub-butterfly
  // tid >> lgNB, uniform over a wave, of butterfly tid mod NB).
  const unsigned char* lutb = reinterpret_cast<const unsigned char*>(lut2);
  uint32_t cbv[kColV ? RO : 1];
  int sub4 = 0;
  if constexpr (kColV) {
    const int q0 = min(tid, NU - 1);
    sub4 = __builtin_amdgcn_readfirstlane(q0 >> lgNB) * RO;
#pragma unroll
    for (int r = 0; r < RO; ++r)
      cbv[r] = (hyb_col_base((uint32_t)(R * (q0 & (NB - 1)) + sub4 + r), P.Q) << kColRep) + (copy << 3);
  }

  // Column walk: the LUT entry whose cost this thread forms each step (entry tid;
  // the instance runs 1024 threads), held for the launch.
  const float2 cv_own = kColV ? col_entry(min(tid, 16 * 64 - 1)) : make_float2(0.0f, 0.0f);

  const int row_bytes = PACK ? (NT * KV) >> 3 : NT;  // backpointer bytes per step
  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    uint8_t* bp = P.ws + (size_t)blockIdx.x * (size_t)N * (size_t)NT;
    const float* seqb = P.seq + (size_t)b * N * V;
    for (int i = tid; i < N * V; i += nthr) wbuf[i] = seqb[i];
    // cum_{-1}, the vector step 0 reads: 0, or for a constrained sequence
    // kVitInf where the top ob bits of the step-0 state differ from ov.  Those
    // bits lie in s_0 >> kV (ob <= L - kV), so kVitInf + E_0(s) = kVitInf is the
    // masked cum_0 of src/viterbi/encode.py:139-141 without touching the step.
    const bool cons = P.overlap != nullptr;
    const int ob = P.overlap_bits;
    const uint32_t ov = cons ? (uint32_t)P.overlap[b] & ((1u << ob) - 1u) : 0u;  // masked as encode.py:136
    for (int j = tid; j < NT; j += nthr)
      rbuf[NT + j] = (cons && ((uint32_t)j >> (L - KV - ob)) != ov) ? kVitInf : 0.0f;
    // Column walk: the cost E_t of every LUT entry, computed once per step as
    // the state loop would (same operations and order, so the same float), sits
    // in the LUT copies' place, one table per step parity (32 KiB each): entry
    // k's cost of step t is float (k << kColRep | copy) of table t & 1, at half
    // the byte of its codeword's float2 in the LUT copies, and a wave's reads fall
    // in distinct banks.  The LUT copies come back after the loop.
    static_assert(!kColV || (kColRep == 2 && MAXT == 1024), "one float4 per table entry, one entry per thread");
    auto build_cost = [&](int t) {
      float4* dst = reinterpret_cast<float4*>(reinterpret_cast<float*>(lut2) + 8192 * (t & 1));
      if (tid < 16 * 64) {  // entry tid
        const float d0 = cv_own.x - wbuf[t * V];
        const float d1 = cv_own.y - wbuf[t * V + 1];
        float e = 0.0f;
        e = e + d0 * d0;
        e = e + d1 * d1;
        dst[tid] = make_float4(e, e, e, e);  // the four copies
        dst[tid + 16 * 64] = make_float4(e, e, e, e);
      }
    };
    __syncthreads();
    if constexpr (kColV) {  // step 0's table, from the weights the barrier above published
      build_cost(0);
      __syncthreads();
    }

    for (int t = 0; t < N; ++t) {
      const float* prev = rbuf + ((t + 1) & 1) * NT;
      float* cur = rbuf + (t & 1) * NT;
      float w[V];
#pragma unroll
      for (int v = 0; v < V; ++v) w[v] = wbuf[t * V + v];
      // the next step's table goes where step t - 1's was (every wave has left
      // it: barrier at the end of each step)
      if (kColV && t + 1 < N) build_cost(t + 1);
      const uint32_t eoff = 32768u * (uint32_t)(t & 1);
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int q = tid + i * nthr;
        __builtin_amdgcn_sched_barrier(0);
        if (q < NU) {
          const int u = (CACHE ? q : opaque(q)) & (NB - 1);
          const int sub = q >> lgNB;
          float ri[R];
#pragma unroll
          for (int p = 0; p < R; ++p) ri[p] = prev[p * NB + u];
          float ro[RO];
          uint32_t bpw = 0;
          // The column walk's row step of output sub4 + r depends on it mod 8
          // (hyb_col_step), so each wave takes one of two unrolled copies
          // (sub4 mod 8 = SO, 0 or 4) whose cost reads are base + immediate.
          auto outputs = [&](auto so_tag) {
            constexpr int SO = decltype(so_tag)::value;
#pragma unroll
            for (int r = 0; r < RO; ++r) {
              const int rr = sub * RO + r;
              float best = 0.0f;
              int bi = 0;
              const uint32_t ebase = kColV ? (cbv[r] >> 1) + eoff : 0u;  // table byte of output r's row-0 entry
#pragma unroll
              for (int p = 0; p < R; ++p) {
                float c[V];
                float e = 0.0f;
                if constexpr (kColV) {
                  e = *reinterpret_cast<const float*>(lutb + ebase + (hyb_col_step(p, SO + r) << (kColRep - 1)));
                } else {
                  if constexpr (CACHE) {
#pragma unroll
                    for (int v = 0; v < V; ++v) c[v] = cw[i][p][r][v];
                  } else {
                    cword((uint32_t)(p * NT + R * u + rr), c);
                  }
#pragma unroll
                  for (int v = 0; v < V; ++v) {
                    const float d = c[v] - w[v];
                    const float d2 = d * d;
                    e = e + d2;
                  }
                }
                const float cum = ri[p] + e;
                if (p == 0 || cum < best) {
                  best = cum;
                  bi = p;
                }
              }
              ro[r] = best;
              bpw |= (uint32_t)bi << (8 * r);
            }
          };
          if (kColV && (sub4 & 4)) {
            outputs(std::integral_constant<int, 4>{});
          } else {
            outputs(std::integral_constant<int, 0>{});
          }
          store_vec<RO>(cur + R * u + sub * RO, ro);
          if constexpr (PACK) {  // entries R*u + sub*RO .. +RO-1 at kV bits each
            uint32_t bits = 0;
#pragma unroll
            for (int r = 0; r < RO; ++r) bits |= ((bpw >> (8 * r)) & (R - 1)) << (r * KV);
            uint8_t* row = bp + (size_t)t * row_bytes;
            const int e0 = R * u + sub * RO;
            if constexpr (RO * KV == 8) {
              row[(e0 * KV) >> 3] = (uint8_t)bits;
            } else {
              *reinterpret_cast<uint16_t*>(row + ((e0 * KV) >> 3)) = (uint16_t)bits;
            }
          } else {
            uint8_t* bdst = bp + (size_t)t * NT + R * u + sub * RO;
#pragma unroll
            for (int r = 0; r < RO; ++r) bdst[r] = (uint8_t)(bpw >> (8 * r));
          }
        }
      }
      __syncthreads();
    }

    if constexpr (kColV) {  // the LUT copies again (the last step's barrier ended every table read)
      stage_col();
      __syncthreads();
    }

    // Final state: lowest index among the minimal cum_{N-1}(s), recomputed from
    // min_p cum_{N-2} (still in LDS) in a separate pass over all states.
    float fbest = INFINITY;
    int fstate = 0x7fffffff;
    {
      const float* prev = rbuf + (N & 1) * NT;  // written at step N-2 (cum_{-1} when N = 1)
      float w[V];
#pragma unroll
      for (int v = 0; v < V; ++v) w[v] = wbuf[(N - 1) * V + v];
      {
        for (int s = tid; s < (NT << KV); s += nthr) {
          float c[V];
          cword((uint32_t)s, c);
          float e = 0.0f;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const float d = c[v] - w[v];
            const float d2 = d * d;
            e = e + d2;
          }
          float cum = prev[s >> KV] + e;
          // end constraint: s_{N-1} mod 2^ob == ov (encode.py:149-154)
          if (cons && ((uint32_t)s & ((1u << ob) - 1u)) != ov) cum = kVitInf;
          if (vi_less(cum, s, fbest, fstate)) {
            fbest = cum;
            fstate = s;
          }
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(fbest, o, 64);
      const int oi = __shfl_xor(fstate, o, 64);
      if (vi_less(ov, oi, fbest, fstate)) {
        fbest = ov;
        fstate = oi;
      }
    }
    if (lane == 0) {
      redv[wave] = fbest;
      redi[wave] = fstate;
    }
    __syncthreads();
    if (tid == 0) {
      float bv = redv[0];
      int bs = redi[0];
      for (int w = 1; w < nwaves; ++w)
        if (vi_less(redv[w], redi[w], bv, bs)) {
          bv = redv[w];
          bs = redi[w];
        }
      // Only a NaN input leaves no candidate; fall back to state 0 so the
      // traceback below always indexes inside the trellis.
      walkbuf[N - 1] = (bs >= 0 && bs < (NT << KV)) ? bs : 0;
      // A constrained sequence whose best end still costs kVitInf has no walk
      // meeting the constraint (encode.py:155-159): flagged through start.
      redi[0] = (cons && !(bv < 0.5f * kVitInf)) ? 1 : 0;
    }
    __syncthreads();

    // Traceback.  Row t of bp holds argmin_p cum_t(p*NT + j), i.e. the best
    // predecessor of the states of step t+1, so walk_{t} = bp_t(walk_{t+1} >> kV)
    // * NT + (walk_{t+1} >> kV).  Rows are staged in LDS, cap at a time, and
    // walked on one thread.
    const int cap = (int)((2 * (size_t)NT * sizeof(float)) / (size_t)row_bytes);
    uint8_t* stage = reinterpret_cast<uint8_t*>(rbuf);
    int s = walkbuf[N - 1];
    for (int hi = N - 2; hi >= 0; hi -= cap) {
      const int lo = max(0, hi - cap + 1);
      const int nbytes_rows = (hi - lo + 1) * row_bytes;
      if ((row_bytes & 3) == 0) {
        const uint32_t* srcw = reinterpret_cast<const uint32_t*>(bp + (size_t)lo * row_bytes);
        uint32_t* dstw = reinterpret_cast<uint32_t*>(stage);
        for (int i = tid; i < (nbytes_rows >> 2); i += nthr) dstw[i] = srcw[i];
      } else {
        for (int i = tid; i < nbytes_rows; i += nthr) stage[i] = bp[(size_t)lo * row_bytes + i];
      }
      __syncthreads();
      if (tid == 0) {
        for (int t = hi; t >= lo; --t) {
          const int j = s >> KV;
          const uint8_t* row = stage + (size_t)(t - lo) * row_bytes;
          int p;
          if constexpr (PACK) {
            p = (row[(j * KV) >> 3] >> ((j * KV) & 7)) & (R - 1);
          } else {
            p = row[j];
          }
          s = p * NT + j;
          walkbuf[t] = s;
        }
      }
      __syncthreads();
    }

    // Outputs.
    double se = 0.0;
    for (int t = tid; t < N; t += nthr) {
      const int st = walkbuf[t];
      if (P.walk) P.walk[(size_t)b * N + t] = st;
      if (P.bits) P.bits[(size_t)b * N + t] = st & (R - 1);
      float c[V];
      cword((uint32_t)st, c);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (P.recon) P.recon[((size_t)b * N + t) * V + v] = c[v];
        const double d = (double)c[v] - (double)wbuf[t * V + v];
        se += d * d;
      }
    }
    if (P.start && tid == 0) P.start[b] = redi[0] ? -1 : walkbuf[0] >> KV;
    if (P.packed) {
      constexpr int per = 8 / KV;
      const int nbytes = (N * KV + 7) / 8;
      for (int i = tid; i < nbytes; i += nthr) {
        uint32_t byte = 0;
#pragma unroll
        for (int qq = 0; qq < per; ++qq) {
          const int t = i * per + qq;
          if (t < N) byte |= ((uint32_t)walkbuf[t] & (R - 1)) << (qq * KV);
        }
        P.packed[(size_t)b * nbytes + i] = (uint8_t)byte;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) se += __shfl_xor(se, o, 64);
    if (lane == 0) redd[wave] = se;
    __syncthreads();
    if (tid == 0 && P.mse) {
      double tot = 0.0;
      for (int w = 0; w < nwaves; ++w) tot += redd[w];
      P.mse[b] = (float)(tot / (double)(N * V));
    }
    __syncthreads();
  }
}

// Walk replay: one thread per sequence.
template <int KV, int V, int CODE>
__global__ __launch_bounds__(256) void bcjr_decode_kernel(DecParams P) {
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= P.B) return;
  constexpr int R = 1 << KV;
  const uint32_t mask = (P.L >= 32) ? 0xFFFFFFFFu : ((1u << P.L) - 1u);
  const int nbytes = (P.N * KV + 7) / 8;
  uint32_t s = (uint32_t)P.start[b];
  for (int t = 0; t < P.N; ++t) {
    uint32_t bits;
    if (P.packed) {
      constexpr int per = 8 / KV;
      bits = ((uint32_t)P.packed[(size_t)b * nbytes + t / per] >> ((t % per) * KV)) & (R - 1);
    } else {
      bits = (uint32_t)P.bits[(size_t)b * P.N + t] & (R - 1);
    }
    s = ((s << KV) | bits) & mask;
    if (P.walk) P.walk[(size_t)b * P.N + t] = (int32_t)s;
    if (P.recon) {
      float c[V];
      codeword<CODE, V>(s, P.table, P.table, P.Q, c);
#pragma unroll
      for (int v = 0; v < V; ++v) P.recon[((size_t)b * P.N + t) * V + v] = c[v];
    }
  }
}

// The full lattice of the min-sum recursion, for viterbi_encode_v(...,
// return_trace=True) (src/viterbi/encode.py:250-307): trace[t][s] = cum_t(s)
// and backptr[t][s] = the predecessor state the minimum chose, for every state s
// of every step, with the rounding and tie rules of the Viterbi kernel above.
// A diagnostic of one or a few sequences: one workgroup per sequence
// (grid-stride), the reduced vector m_{t-1}(j) = min_p cum_{t-1}(p*NT + j) and
// its argmin p in LDS (NT floats + NT bytes).  Thread tid owns the reduced
// indices j = tid + i*nthr and, for each, the R states p*NT + j, whose
// predecessors are the states p'*NT + (s >> kV):
//   cum_t(s) = fl(m_{t-1}(s >> kV) + E_t(s)),
//   backptr_t(s) = argmin_{t-1}(s >> kV) * NT + (s >> kV),
// and m_t(j), argmin_t(j) over its R states (lowest p on a tie) are written
// back after a barrier.  cum_{-1} = 0: m = 0 and argmin = 0 at the start.
template <int KV, int V, int CODE>
__global__ __launch_bounds__(1024) void bcjr_viterbi_trace_kernel(TraceParams P) {
  constexpr int R = 1 << KV;
  constexpr int kMaxJ = 16;  // reduced indices per thread: NT <= 16 * 1024
  extern __shared__ __align__(16) unsigned char smem[];
  const int L = P.L, N = P.N;
  const int NT = 1 << (L - KV);
  const size_t S = (size_t)1 << L;
  const int tid = threadIdx.x, nthr = blockDim.x;
  float* mprev = reinterpret_cast<float*>(smem);                // NT
  uint8_t* aprev = reinterpret_cast<uint8_t*>(mprev + NT);       // NT
  for (long long b = blockIdx.x; b < P.B; b += gridDim.x) {
    for (int j = tid; j < NT; j += nthr) {
      mprev[j] = 0.0f;
      aprev[j] = 0;
    }
    __syncthreads();
    for (int t = 0; t < N; ++t) {
      float w[V];
#pragma unroll
      for (int v = 0; v < V; ++v) w[v] = P.seq[((size_t)b * N + t) * V + v];
      float* tr = P.trace + ((size_t)b * N + t) * S;
      int32_t* bp = P.backptr + ((size_t)b * N + t) * S;
      float mnew[kMaxJ];
      int anew[kMaxJ];
#pragma unroll
      for (int i = 0; i < kMaxJ; ++i) {
        const int j = tid + i * nthr;
        mnew[i] = 0.0f;
        anew[i] = 0;
        if (j < NT) {
#pragma unroll 1
          for (int p = 0; p < R; ++p) {
            const uint32_t s = (uint32_t)p * (uint32_t)NT + (uint32_t)j;
            float c[V];
            codeword<CODE, V>(s, P.table, P.table, P.Q, c);
            float e = 0.0f;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              const float d = c[v] - w[v];
              e = v ? e + d * d : d * d;
            }
            const uint32_t u = s >> KV;
            const float cum = mprev[u] + e;
            tr[s] = cum;
            bp[s] = (int32_t)((uint32_t)aprev[u] * (uint32_t)NT + u);
            if (p == 0 || cum < mnew[i]) {
              mnew[i] = cum;
              anew[i] = p;
            }
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kMaxJ; ++i) {
        const int j = tid + i * nthr;
        if (j < NT) {
          mprev[j] = mnew[i];
          aprev[j] = (uint8_t)anew[i];
        }
      }
      __syncthreads();
    }
  }
}

// Dequantize tiles straight into the matrix: out[row, col] = fl32(scale * c_v(s_t))
// (product in double, one rounding: the float64 product then float32 cast of
// src/quantize/serialize.py:106 and src/rht/transform.py:110)
// with the tile order of tile_for_viterbi (sequence b = col_block * n_row_blocks
// + row_block holds the Tx x Ty tile row-major, element e = t*V + v).  The walk
// state needs no serial replay: s_t = ((start << kV(t+1)) | sum_{tau<=t}
// bits_tau << kV(t - tau)) mod 2^L depends only on the last ceil(L/kV) steps (and
// on start while kV(t+1) < L), so every output element is decoded by its own thread
// and the writes are coalesced along rows.
template <int KV, int V, int CODE>
__global__ __launch_bounds__(256) void bcjr_dequant_kernel(DqParams P) {
  constexpr int R = 1 << KV;
  const uint32_t mask = (P.L >= 32) ? 0xFFFFFFFFu : ((1u << P.L) - 1u);
  const int steps = (P.L + KV - 1) / KV;  // steps whose bits reach a state
  const int nbytes = (P.N * KV + 7) / 8;
  const long long n_row = P.m / P.Tx;
  const long long total = P.m * P.n;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const long long row = idx / P.n, col = idx - row * P.n;
    const long long b = (col / P.Ty) * n_row + row / P.Tx;
    const int e = (int)((row % P.Tx) * P.Ty + col % P.Ty);
    const int t = e / V, v = e - (e / V) * V;
    uint32_t s = 0;
    if (KV * (t + 1) < P.L) s = ((uint32_t)P.start[b] << (KV * (t + 1))) & mask;
    const int lo = t - steps + 1 > 0 ? t - steps + 1 : 0;
    for (int tau = lo; tau <= t; ++tau) {
      uint32_t bits;
      if (P.packed) {
        constexpr int per = 8 / KV;
        bits = ((uint32_t)P.packed[(size_t)b * nbytes + tau / per] >> ((tau % per) * KV)) & (R - 1);
      } else if (P.bits8) {
        bits = (uint32_t)P.bits8[(size_t)b * P.N + tau] & (R - 1);
      } else {
        bits = (uint32_t)P.bits32[(size_t)b * P.N + tau] & (R - 1);
      }
      s |= bits << (KV * (t - tau));
    }
    s &= mask;
    float c[V];
    codeword<CODE, V>(s, P.table, P.table, P.Q, c);
    P.out[idx] = (float)((double)c[v] * P.scale);
  }
}

// Vector form of bcjr_dequant_kernel for Ty % 4 == 0, m*n/4 < 2^31 and a
// 16-byte aligned output: one thread writes 4 consecutive columns of a row with
// one 16-byte store.  The 4 elements are 4/V consecutive steps of one tile, so
// the state window is decoded once and then rolled forward step by step; index
// arithmetic is 32-bit, with shifts when Tx and Ty are powers of two.
template <int KV, int V, int CODE>
__global__ __launch_bounds__(256) void bcjr_dequant4_kernel(DqParams P) {
  constexpr int R = 1 << KV;
  constexpr int NS = 4 / V;  // steps per thread
  constexpr int per = 8 / KV;
  const uint32_t mask = (1u << P.L) - 1u;  // L <= 16
  const int win = (P.L + KV - 1) / KV;
  const uint32_t n4 = (uint32_t)(P.n >> 2);
  const uint32_t total4 = (uint32_t)((P.m * P.n) >> 2);
  const uint32_t n_row = (uint32_t)(P.m / P.Tx);
  const int nbytes = (P.N * KV + 7) / 8;
  auto bits_at = [&](size_t b, int tau) -> uint32_t {
    if (P.packed) return ((uint32_t)P.packed[b * nbytes + tau / per] >> ((tau % per) * KV)) & (R - 1);
    if (P.bits8) return (uint32_t)P.bits8[b * P.N + tau] & (R - 1);
    return (uint32_t)P.bits32[b * P.N + tau] & (R - 1);
  };
  for (uint32_t q = blockIdx.x * blockDim.x + threadIdx.x; q < total4; q += gridDim.x * blockDim.x) {
    const uint32_t row = q / n4;
    const uint32_t col = (q - row * n4) << 2;
    uint32_t rb, rr, cb, cc;
    if (P.tx_shift >= 0) {
      rb = row >> P.tx_shift;
      rr = row & ((1u << P.tx_shift) - 1u);
    } else {
      rb = row / (uint32_t)P.Tx;
      rr = row - rb * (uint32_t)P.Tx;
    }
    if (P.ty_shift >= 0) {
      cb = col >> P.ty_shift;
      cc = col & ((1u << P.ty_shift) - 1u);
    } else {
      cb = col / (uint32_t)P.Ty;
      cc = col - cb * (uint32_t)P.Ty;
    }
    const size_t b = (size_t)cb * n_row + rb;
    const int t0 = (int)(rr * (uint32_t)P.Ty + cc) / V;
    uint32_t s = 0;
    if (KV * (t0 + 1) < P.L) s = (uint32_t)P.start[b] << (KV * (t0 + 1));
    for (int tau = t0 - win + 1 > 0 ? t0 - win + 1 : 0; tau <= t0; ++tau) s |= bits_at(b, tau) << (KV * (t0 - tau));
    s &= mask;
    float o[4];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      if (j) s = ((s << KV) | bits_at(b, t0 + j)) & mask;
      float c[V];
      codeword<CODE, V>(s, P.table, P.table, P.Q, c);
#pragma unroll
      for (int v = 0; v < V; ++v) o[j * V + v] = (float)((double)c[v] * P.scale);
    }
    *reinterpret_cast<float4*>(P.out + (size_t)row * P.n + col) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// The reference's tile configuration (16x16 tiles, k = 2 bits per weight, so
// kV = 2 with V = 1 or kV = 4 with V = 2): a tile row is SR = 16 / V steps and
// exactly 32 bits of the packed bitstream.  Each thread writes 4 consecutive
// columns (one 16-byte store; a wave covers 256 contiguous bytes of 4 rows).  Its tile row's step indices come in one aligned load (a
// 32-bit word packed, 8 or 16 bytes as uint8, 32 or 64 bytes as int32).  The
// kernel needs blockDim.x == 256.
//
// No step-by-step replay: with g(w) the word w with the order of its kV-bit
// groups reversed (step j of the row moves to group SR-1-j), the 64-bit value
// H = (h << 32) | g(cur), where h is the start state for the first row of a
// tile and g(prev) for the others (the previous row's SR >= ceil(L/kV) steps
// fix the state), holds every state of the row: the state after step t of the
// row is (H >> (32 - kV (t+1))) mod 2^L.  The kernel runs at a handful of VALU
// instructions per weight: group reversal and one 64-bit shift per 4 columns, a
// bit-field extract, the codeword and the scale per step.
template <int FMT>
struct RowSteps;  // step indices of one tile row, as the packed 32-bit word: word()

template <>
struct RowSteps<BITS_FMT_PACKED> {
  uint32_t w;
  template <int KV, int SR>
  __device__ __forceinline__ void load(const DqParams& P, uint32_t b, int row) {
    w = reinterpret_cast<const uint32_t*>(P.packed)[b * 16u + (uint32_t)row];  // 64 bytes per tile
  }
  template <int KV, int SR>
  __device__ __forceinline__ uint32_t word() const { return w; }
};

template <>
struct RowSteps<BITS_FMT_U8> {
  uint32_t w[4];
  template <int KV, int SR>
  __device__ __forceinline__ void load(const DqParams& P, uint32_t b, int row) {
    const uint8_t* p = P.bits8 + (size_t)(b * (uint32_t)(SR * 16) + (uint32_t)(row * SR));
    if constexpr (SR == 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      w[0] = v.x; w[1] = v.y; w[2] = 0; w[3] = 0;
    }
  }
  template <int KV, int SR>
  __device__ __forceinline__ uint32_t word() const {  // the packed form: step j in bits [j*KV, (j+1)*KV)
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < SR; ++j) r |= ((w[j >> 2] >> ((j & 3) * 8)) & ((1u << KV) - 1u)) << (j * KV);
    return r;
  }
};

template <>
struct RowSteps<BITS_FMT_I32> {
  uint32_t w[16];
  template <int KV, int SR>
  __device__ __forceinline__ void load(const DqParams& P, uint32_t b, int row) {
    const uint4* p = reinterpret_cast<const uint4*>(P.bits32 + (size_t)(b * (uint32_t)(SR * 16) + (uint32_t)(row * SR)));
#pragma unroll
    for (int i = 0; i < SR / 4; ++i) {
      const uint4 v = p[i];
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  }
  template <int KV, int SR>
  __device__ __forceinline__ uint32_t word() const {
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < SR; ++j) r |= (w[j] & ((1u << KV) - 1u)) << (j * KV);
    return r;
  }
};

// Reverse the order of the KV-bit groups of a 32-bit word (KV = 2 or 4).
template <int KV>
__device__ __forceinline__ uint32_t reverse_groups(uint32_t w) {
  uint32_t r = __builtin_bitreverse32(w);  // reverses groups and the bits inside them
  r = ((r >> 1) & 0x55555555u) | ((r & 0x55555555u) << 1);  // restore bit order inside pairs
  if constexpr (KV == 4) r = ((r >> 2) & 0x33333333u) | ((r & 0x33333333u) << 2);  // ... and nibbles
  static_assert(KV == 2 || KV == 4, "group reversal for kV = 2 or 4");
  return r;
}

//
// The HYB LUT (2^Q x 2 floats, <= 32 KiB) is staged in LDS once per workgroup:
// its lookups are random 8-byte gathers, which from global memory cost one
// cache-line request per lane.  The grid is persistent (a few workgroups per
// CU) so the staging is amortised.
template <int KV, int V, int CODE, int FMT>
__global__ __launch_bounds__(256) void bcjr_dequant_t16_kernel(DqParams P) {
  constexpr int SR = 16 / V;  // steps per tile row
  constexpr int SQ = SR / 4;  // steps per 4-column quarter
  static_assert(SR * KV == 32, "k = 2: one 32-bit word of packed bits per tile row");
  extern __shared__ __align__(16) float lds_lut[];
  const float* table = P.table;
  if constexpr (CODE == CODE_HYB) {
    const int nlut = 2 << P.Q;
    for (int i = threadIdx.x; i < nlut; i += blockDim.x) lds_lut[i] = P.table[i];
    __syncthreads();
    table = lds_lut;
  }
  const uint32_t mask = (1u << P.L) - 1u;
  const uint32_t n4 = (uint32_t)(P.n >> 2);
  const uint32_t n_row = (uint32_t)(P.m >> 4);
  // Work unit of a workgroup: one band of 16 rows x 64 columns (4 tiles), thread
  // (tid / 16, tid % 16) -> (row in the band, 4-column quarter).  Each tile's
  // bits are read by one workgroup only, so they are fetched into one XCD's L2
  // once (rows of a band spread over workgroups would land on several XCDs).
  const uint32_t nchunk = (n4 + 15u) >> 4;
  const uint32_t units = n_row * nchunk;
  const int rr = (int)(threadIdx.x >> 4);
  for (uint32_t u = blockIdx.x; u < units; u += gridDim.x) {
    const uint32_t rbnd = u / nchunk, ch = u - rbnd * nchunk;
    const uint32_t c4 = (ch << 4) + (threadIdx.x & 15u);  // column / 4
    if (c4 >= n4) continue;
    const uint32_t row = (rbnd << 4) + (uint32_t)rr;
    const int jq = (int)(c4 & 3u);
    const uint32_t b = (c4 >> 2) * n_row + rbnd;
    RowSteps<FMT> rs;
    rs.template load<KV, SR>(P, b, rr);
    uint32_t hi;
    if (rr == 0) {
      hi = (uint32_t)P.start[b];
    } else {
      RowSteps<FMT> ps;
      ps.template load<KV, SR>(P, b, rr - 1);
      hi = reverse_groups<KV>(ps.template word<KV, SR>());
    }
    const uint64_t H = ((uint64_t)hi << 32) | reverse_groups<KV>(rs.template word<KV, SR>());
    // state after the quarter's last step in the low bits; the earlier ones sit
    // KV bits apart above it (L + KV (SQ-1) <= 22 bits)
    const uint32_t Hq = (uint32_t)(H >> (32 - KV * SQ * (jq + 1)));
    float o[4];
#pragma unroll
    for (int j = 0; j < SQ; ++j) {
      const uint32_t s = (Hq >> (KV * (SQ - 1 - j))) & mask;
      float c[V];
      codeword<CODE, V>(s, table, table, P.Q, c);
#pragma unroll
      for (int v = 0; v < V; ++v)
        o[j * V + v] = P.scale_is_f32 ? c[v] * (float)P.scale : (float)((double)c[v] * P.scale);
    }
    *reinterpret_cast<float4*>(P.out + (size_t)row * P.n + ((size_t)c4 << 2)) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// Codebook fill: one thread per state.
template <int CODE>
__global__ __launch_bounds__(256) void bcjr_codebook_kernel(CbParams P) {
  const long long s = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= P.S) return;
  if constexpr (CODE == CODE_HYB) {
    float c[2];
    codeword<CODE_HYB, 2>((uint32_t)s, nullptr, P.lut, P.Q, c);
    P.out[2 * s] = c[0];
    P.out[2 * s + 1] = c[1];
  } else {
    float c[1];
    codeword<CODE, 1>((uint32_t)s, nullptr, nullptr, P.Q, c);
    P.out[s] = c[0];
  }
}

#define BCJR_VIT_CASE(KV_, V_, CODE_, UPT_, CACHE_)                                              \
  if (!wide && KV == KV_ && V == V_ && code == CODE_ && upt == UPT_ && cache == CACHE_)          \
    return reinterpret_cast<const void*>(&bcjr_viterbi_kernel<KV_, V_, CODE_, UPT_, CACHE_, 512>);
#define BCJR_VIT_WIDE(KV_, V_, CODE_, UPT_, CACHE_)                                              \
  if (wide && KV == KV_ && V == V_ && code == CODE_ && upt == UPT_ && cache == CACHE_)           \
    return reinterpret_cast<const void*>(&bcjr_viterbi_kernel<KV_, V_, CODE_, UPT_, CACHE_, 1024>);

#define BCJR_VIT_UPTS(KV_, V_, CODE_, CACHE_) \
  BCJR_VIT_CASE(KV_, V_, CODE_, 1, CACHE_)    \
  BCJR_VIT_CASE(KV_, V_, CODE_, 2, CACHE_)    \
  BCJR_VIT_CASE(KV_, V_, CODE_, 4, CACHE_)    \
  BCJR_VIT_CASE(KV_, V_, CODE_, 8, CACHE_)
#define BCJR_VIT_WIDE_UPTS(KV_, V_, CODE_) \
  BCJR_VIT_WIDE(KV_, V_, CODE_, 1, true)   \
  BCJR_VIT_WIDE(KV_, V_, CODE_, 2, true)   \
  BCJR_VIT_WIDE(KV_, V_, CODE_, 4, true)

// wide: the 1024-thread instances, for units >= 1024 (L >= 14 at kV = 2, L = 16
// at kV = 4) whenever the thread's codewords fit 64 VGPRs or are not cached.
const void* vit_kernel_ptr(int KV, int V, int code, int upt, bool cache, bool wide) {
  BCJR_VIT_CASE(1, 1, CODE_TABLE, 1, true)
  BCJR_VIT_UPTS(2, 1, CODE_TABLE, true)
  BCJR_VIT_UPTS(2, 1, CODE_1MAD, true)
  BCJR_VIT_UPTS(2, 1, CODE_3INST, true)
  BCJR_VIT_CASE(2, 2, CODE_TABLE, 1, true)
  BCJR_VIT_CASE(2, 2, CODE_TABLE, 2, true)
  BCJR_VIT_CASE(2, 2, CODE_TABLE, 4, true)
  BCJR_VIT_CASE(2, 2, CODE_HYB, 1, true)
  BCJR_VIT_CASE(2, 2, CODE_HYB, 2, true)
  BCJR_VIT_CASE(2, 2, CODE_HYB, 4, true)
  BCJR_VIT_CASE(2, 2, CODE_HYB, 8, false)  // L = 16, k = 1: one plain LUT copy
  BCJR_VIT_CASE(4, 1, CODE_TABLE, 1, false)
  BCJR_VIT_CASE(4, 1, CODE_TABLE, 2, false)
  BCJR_VIT_CASE(4, 1, CODE_1MAD, 1, false)
  BCJR_VIT_CASE(4, 1, CODE_1MAD, 2, false)
  BCJR_VIT_CASE(4, 1, CODE_3INST, 1, false)
  BCJR_VIT_CASE(4, 1, CODE_3INST, 2, false)
  BCJR_VIT_CASE(4, 2, CODE_TABLE, 1, false)
  BCJR_VIT_CASE(4, 2, CODE_TABLE, 2, false)
  BCJR_VIT_CASE(4, 2, CODE_HYB, 1, false)
  BCJR_VIT_CASE(4, 2, CODE_HYB, 2, false)
  BCJR_VIT_WIDE_UPTS(2, 1, CODE_TABLE)
  BCJR_VIT_WIDE_UPTS(2, 1, CODE_1MAD)
  BCJR_VIT_WIDE_UPTS(2, 1, CODE_3INST)
  BCJR_VIT_WIDE(2, 2, CODE_TABLE, 1, true)
  BCJR_VIT_WIDE(2, 2, CODE_TABLE, 2, true)
  BCJR_VIT_WIDE(2, 2, CODE_HYB, 1, true)
  BCJR_VIT_WIDE(2, 2, CODE_HYB, 2, true)
  // k = 1, V = 2 at L = 16: 4 butterflies per thread, whose 128 codewords do not
  // fit the cache, so they are read per state.
  BCJR_VIT_WIDE(2, 2, CODE_TABLE, 4, false)
  BCJR_VIT_WIDE(2, 2, CODE_HYB, 4, false)
  BCJR_VIT_WIDE(4, 1, CODE_TABLE, 1, false)
  BCJR_VIT_WIDE(4, 1, CODE_1MAD, 1, false)
  BCJR_VIT_WIDE(4, 1, CODE_3INST, 1, false)
  BCJR_VIT_WIDE(4, 2, CODE_TABLE, 1, false)
  BCJR_VIT_WIDE(4, 2, CODE_HYB, 1, false)
  BCJR_VIT_WIDE(4, 2, CODE_HYB_COL, 1, false)
  return nullptr;
}

#define BCJR_DEC_CASE(KV_, V_, CODE_) \
  if (KV == KV_ && V == V_ && code == CODE_) \
    return reinterpret_cast<const void*>(&bcjr_decode_kernel<KV_, V_, CODE_>);

#define BCJR_DQ_CASE(KV_, V_, CODE_) \
  if (KV == KV_ && V == V_ && code == CODE_) \
    return vec4 ? reinterpret_cast<const void*>(&bcjr_dequant4_kernel<KV_, V_, CODE_>) \
                : reinterpret_cast<const void*>(&bcjr_dequant_kernel<KV_, V_, CODE_>);

const void* dequant_kernel_ptr(int KV, int V, int code, bool vec4) {
  BCJR_DQ_CASE(1, 1, CODE_TABLE)
  BCJR_DQ_CASE(2, 1, CODE_TABLE)
  BCJR_DQ_CASE(2, 1, CODE_1MAD)
  BCJR_DQ_CASE(2, 1, CODE_3INST)
  BCJR_DQ_CASE(2, 2, CODE_TABLE)
  BCJR_DQ_CASE(2, 2, CODE_HYB)
  BCJR_DQ_CASE(4, 1, CODE_TABLE)
  BCJR_DQ_CASE(4, 1, CODE_1MAD)
  BCJR_DQ_CASE(4, 1, CODE_3INST)
  BCJR_DQ_CASE(4, 2, CODE_TABLE)
  BCJR_DQ_CASE(4, 2, CODE_HYB)
  return nullptr;
}

#define BCJR_DQ16_CASE(KV_, V_, CODE_)                                                               \
  if (KV == KV_ && V == V_ && code == CODE_) {                                                        \
    if (fmt == BITS_FMT_PACKED)                                                                       \
      return reinterpret_cast<const void*>(&bcjr_dequant_t16_kernel<KV_, V_, CODE_, BITS_FMT_PACKED>); \
    if (fmt == BITS_FMT_U8)                                                                           \
      return reinterpret_cast<const void*>(&bcjr_dequant_t16_kernel<KV_, V_, CODE_, BITS_FMT_U8>);     \
    return reinterpret_cast<const void*>(&bcjr_dequant_t16_kernel<KV_, V_, CODE_, BITS_FMT_I32>);      \
  }

const void* dequant_t16_kernel_ptr(int KV, int V, int code, int fmt) {
  BCJR_DQ16_CASE(2, 1, CODE_TABLE)
  BCJR_DQ16_CASE(2, 1, CODE_1MAD)
  BCJR_DQ16_CASE(2, 1, CODE_3INST)
  BCJR_DQ16_CASE(4, 2, CODE_TABLE)
  BCJR_DQ16_CASE(4, 2, CODE_HYB)
  return nullptr;
}

const void* decode_kernel_ptr(int KV, int V, int code) {
  BCJR_DEC_CASE(1, 1, CODE_TABLE)
  BCJR_DEC_CASE(2, 1, CODE_TABLE)
  BCJR_DEC_CASE(2, 1, CODE_1MAD)
  BCJR_DEC_CASE(2, 1, CODE_3INST)
  BCJR_DEC_CASE(2, 2, CODE_TABLE)
  BCJR_DEC_CASE(2, 2, CODE_HYB)
  BCJR_DEC_CASE(4, 1, CODE_TABLE)
  BCJR_DEC_CASE(4, 1, CODE_1MAD)
  BCJR_DEC_CASE(4, 1, CODE_3INST)
  BCJR_DEC_CASE(4, 2, CODE_TABLE)
  BCJR_DEC_CASE(4, 2, CODE_HYB)
  return nullptr;
}

#define BCJR_TRACE_CASE(KV_, V_, CODE_) \
  if (KV == KV_ && V == V_ && code == CODE_) return reinterpret_cast<const void*>(&bcjr_viterbi_trace_kernel<KV_, V_, CODE_>);

const void* trace_kernel_ptr(int KV, int V, int code) {
  BCJR_TRACE_CASE(1, 1, CODE_TABLE)
  BCJR_TRACE_CASE(2, 1, CODE_TABLE)
  BCJR_TRACE_CASE(2, 1, CODE_1MAD)
  BCJR_TRACE_CASE(2, 1, CODE_3INST)
  BCJR_TRACE_CASE(2, 2, CODE_TABLE)
  BCJR_TRACE_CASE(2, 2, CODE_HYB)
  BCJR_TRACE_CASE(4, 1, CODE_TABLE)
  BCJR_TRACE_CASE(4, 1, CODE_1MAD)
  BCJR_TRACE_CASE(4, 1, CODE_3INST)
  BCJR_TRACE_CASE(4, 2, CODE_TABLE)
  BCJR_TRACE_CASE(4, 2, CODE_HYB)
  return nullptr;
}

const void* codebook_kernel_ptr(int code) {
  if (code == CODE_1MAD) return reinterpret_cast<const void*>(&bcjr_codebook_kernel<CODE_1MAD>);
  if (code == CODE_3INST) return reinterpret_cast<const void*>(&bcjr_codebook_kernel<CODE_3INST>);
  if (code == CODE_HYB) return reinterpret_cast<const void*>(&bcjr_codebook_kernel<CODE_HYB>);
  return nullptr;
}

}  // namespace bcjr
