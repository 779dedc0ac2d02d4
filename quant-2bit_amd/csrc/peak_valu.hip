// Issue-rate microbenchmarks that define the roofline peaks used by bench.py:
//   kind 0: v_exp_f32 only            (transcendental rate)
//   kind 1: v_log_f32 only
//   kind 2: v_fma_f32 only            (plain VALU rate)
//   kind 3: one v_exp_f32 + K v_fma_f32 per step (does the transcendental
//           unit overlap ordinary VALU work?)
// Each thread runs 16 independent dependency chains so the measurement is
// issue-bound, not latency-bound.  Results feed a sink store so nothing is
// optimised away.  Built into its own library (libbcjr_peak.so).
#include <hip/hip_runtime.h>

namespace {

constexpr int kChains = 16;

template <int KIND, int K>
__global__ __launch_bounds__(256) void peak_kernel(float* sink, int iters) {
  float x[kChains], y[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
    x[c] = 0.001f * (threadIdx.x + c);
    y[c] = 0.5f + 0.001f * c;
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
      if constexpr (KIND == 0) {
        x[c] = __builtin_amdgcn_exp2f(-x[c]);
      } else if constexpr (KIND == 1) {
        x[c] = __builtin_amdgcn_logf(x[c] + 1.5f);
      } else if constexpr (KIND == 2) {
        x[c] = fmaf(x[c], 0.999f, 0.001f);
      } else {
        x[c] = __builtin_amdgcn_exp2f(-x[c]);
#pragma unroll
        for (int j = 0; j < K; ++j) y[c] = fmaf(y[c], 0.999f, 0.0007f);
      }
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += x[c] + y[c];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int KIND, int K>
int launch(float* sink, int blocks, int iters, hipStream_t stream) {
  hipLaunchKernelGGL((peak_kernel<KIND, K>), dim3(blocks), dim3(256), 0, stream, sink, iters);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace

extern "C" {

// Chains per thread (ops per iteration per thread = kChains, plus K*kChains FMAs
// for kind 3).  sink must hold blocks*256 floats.
int bcjr_peak_chains(void) { return kChains; }

int bcjr_peak_launch(int kind, int K, float* sink, int blocks, int iters, hipStream_t stream) {
  if (!sink || blocks < 1 || iters < 1) return -1;
  switch (kind) {
    case 0: return launch<0, 0>(sink, blocks, iters, stream);
    case 1: return launch<1, 0>(sink, blocks, iters, stream);
    case 2: return launch<2, 0>(sink, blocks, iters, stream);
    case 3:
      switch (K) {
        case 1: return launch<3, 1>(sink, blocks, iters, stream);
        case 2: return launch<3, 2>(sink, blocks, iters, stream);
        case 4: return launch<3, 4>(sink, blocks, iters, stream);
        case 8: return launch<3, 8>(sink, blocks, iters, stream);
        default: return -1;
      }
    default: return -1;
  }
}

}  // extern "C"
