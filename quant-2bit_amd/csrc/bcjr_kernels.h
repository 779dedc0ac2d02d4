// Host-side view of the kernel instances: each kernel translation unit exposes a
// lookup from (kV, V, code, units-per-thread[, cache]) to the template instance,
// plus the LDS footprint its launch needs.  The C ABI (bcjr_capi.hip) owns
// validation, occupancy and launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace bcjr {

struct FwdParams;
struct BwdParams;
struct VitParams;

// Butterflies per thread (of upt) whose codewords the soft forward keeps in
// VGPRs for the whole launch: as many as fit kFwdCacheVgprs (R*R*V each);
// 16-state butterflies are never cached.
constexpr int kFwdCacheVgprs = 96;
constexpr int fwd_cached_units(int KV, int V, int upt) {
  return KV >= 4 ? 0
                 : (upt < kFwdCacheVgprs / ((1 << KV) * (1 << KV) * V) ? upt
                                                                        : kFwdCacheVgprs / ((1 << KV) * (1 << KV) * V));
}

// The same budget for the backward's beta + nu + grad sweep: 5 of 8
// butterflies at kV = 2, V = 1 (80 VGPRs beside that sweep's working set), 2 at
// V = 2.  The 3INST instance, whose hashed codewords need no table address,
// keeps a sixth (96 VGPRs; a seventh or eighth spills inside the step loop and
// runs 5 % slower); the table and 1MAD instances spill at 96.
constexpr int kBwdCacheVgprs = 80;
constexpr int kBwdCacheVgprs3Inst = 96;
constexpr int bwd_cached_units(int KV, int V, int upt, int code = -1) {
  return KV >= 4 ? 0
                 : (upt < (code == 2 ? kBwdCacheVgprs3Inst : kBwdCacheVgprs) / ((1 << KV) * (1 << KV) * V)
                        ? upt
                        : (code == 2 ? kBwdCacheVgprs3Inst : kBwdCacheVgprs) / ((1 << KV) * (1 << KV) * V));
}

// The alpha + mu sweep's own budget (its working set is smaller than the beta
// + nu + grad sweep's, and the two caches are never live together).
constexpr int kBwdAlphaCacheVgprs = 128;
constexpr int bwd_alpha_cached_units(int KV, int V, int upt) {
  return KV >= 4 ? 0
                 : (upt < kBwdAlphaCacheVgprs / ((1 << KV) * (1 << KV) * V)
                        ? upt
                        : kBwdAlphaCacheVgprs / ((1 << KV) * (1 << KV) * V));
}

const void* fwd_kernel_ptr(int KV, int V, int code, int upt, bool internals);
// The four-waves-per-SIMD forward (bcjr_fwd4.hip): kV = 2, V = 1, codes TABLE /
// 1MAD / 3INST, 1024 threads, upt = 2^(L-14) butterflies per thread (L = 14..16).
const void* fwd4_kernel_ptr(int code, int upt);
const void* bwd_kernel_ptr(int KV, int V, int code, int upt);
const void* vit_kernel_ptr(int KV, int V, int code, int upt, bool cache, bool wide);
const void* decode_kernel_ptr(int KV, int V, int code);
const void* trace_kernel_ptr(int KV, int V, int code);
const void* dequant_kernel_ptr(int KV, int V, int code, bool vec4);
const void* dequant_t16_kernel_ptr(int KV, int V, int code, int fmt);
const void* codebook_kernel_ptr(int code);

// Hadamard transforms (bcjr_rht.hip).  Rows: out[r] = scale * row_sign[r] *
// post .* H_n (pre .* x[r]), n a power of two <= 16384, out may equal x.
// Columns: x = scale * diag(row_sign) H_m x in place, m, n <= 16384 powers of two.
hipError_t launch_fwht_rows(const float* x, float* out, long long rows, int n, const float* pre,
                            const float* post, long long vec_rows, const float* row_sign, float scale,
                            int max_blocks, hipStream_t stream);
hipError_t launch_fwht_cols(float* x, int batch, int m, int n, const float* row_sign, float scale,
                            int max_blocks, hipStream_t stream);
hipError_t launch_fwht_tiled(const float* x, float* out, int batch, int m, int n, bool col, const float* pre,
                             const float* post, const float* row_mid, const float* row_end, float scale,
                             int max_blocks, hipStream_t stream);

// The kernel-side code of a soft launch, or of a 1024-thread Viterbi launch:
// HYB at L = 16, kV = 4, 3 <= Q <= 9 takes the column-walk LUT (code 4,
// CODE_HYB_COL in bcjr_device.h).
inline int soft_kernel_code(int code, int L, int KV, int Q) {
  return (code == 3 && L == 16 && KV == 4 && Q >= 3 && Q <= 9) ? 4 : code;
}

// LDS bytes for one workgroup (code as soft_kernel_code returns it).
inline size_t fwd_lds_bytes(int L, int KV, int V, int N, int nwaves, int code, int Q) {
  const size_t NT = (size_t)1 << (L - KV);
  size_t b = 8u * (size_t)((N + 1) & ~1);          // C_t (double), padded to 16 bytes
  b += 4u * (2 * NT + 3 * 16 + (size_t)N * V + 2 * (size_t)nwaves * (V + 1));
  if (code == 3) b += 8u + 8u * ((size_t)2 << Q);  // signed LUT, 8-byte aligned
  if (code == 4) b += 8u + 32u * 64u * 8u;         // column-walk LUT (32 rows of 64)
  return b;
}

inline size_t fwd4_lds_bytes(int L, int N) {
  const size_t NT = (size_t)1 << (L - 2);
  return 8u * (size_t)((N + 1) & ~1) + 4u * (2 * NT + 3 * 16 + 4 + (size_t)N + 2 * 16);
}

inline size_t bwd_lds_bytes(int L, int KV, int V, int N, int nwaves, int code, int Q) {
  const size_t NT = (size_t)1 << (L - KV);
  size_t b = 8u * (size_t)((N + 1) & ~1);
  b += 4u * (2 * NT + 4 * 16 + 2 * (size_t)N * V + 2 * (size_t)nwaves * (V + 1));
  if (code == 3) b += 8u + 8u * ((size_t)2 << Q);  // signed LUT, 8-byte aligned
  if (code == 4) b += 8u + 32u * 64u * 8u;         // column-walk LUT (32 rows of 64)
  return b;
}

// log2 of the signed HYB LUT copies the kV = 4 Viterbi keeps: 8, or as many as
// fit 64 KiB (2^(Q+1) entries of 8 bytes each).
__host__ __device__ constexpr int hyb_lut_rep(int Q) { return 12 - Q < 3 ? 12 - Q : 3; }

// rep_lut: a HYB LUT is staged as 2^hyb_lut_rep(Q) interleaved copies of the
// signed LUT (the uncached 1024-thread instances), else as one plain copy.
inline size_t vit_lds_bytes(int L, int KV, int V, int N, int nwaves, int code, int Q, bool rep_lut) {
  const size_t NT = (size_t)1 << (L - KV);
  (void)nwaves;
  size_t b = 8u * 16;                                           // per-wave MSE partials
  b += 4u * (2 * NT + (size_t)N * V + 2 * 16 + (size_t)N);      // state, seq, argmin, walk
  b = (b + 15) & ~(size_t)15;
  if (code == 3) b += rep_lut ? 8u * ((size_t)2 << Q << hyb_lut_rep(Q)) : 8u * ((size_t)1 << Q);
  if (code == 4) b += 8u * (32u * 64u << 2);  // column-walk LUT, 4 interleaved copies
  return b;
}

}  // namespace bcjr
