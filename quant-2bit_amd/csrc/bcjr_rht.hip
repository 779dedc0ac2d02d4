// Fast Walsh-Hadamard transforms for the random Hadamard transform (RHT) that
// wraps the BCJR quantizer:
//   RHT(W)     = s * H_m diag(sl) W diag(sr) H_n            (src/rht/transform.py:65-96)
//   RHT^-1(W~) = s * diag(sl) H_m W~ H_n diag(sr)           (src/rht/transform.py:99-126)
// with s = 1/sqrt(m*n) and H unscaled Sylvester-ordered Hadamard matrices.  The
// butterflies run in the reference's order (fwht_numpy, transform.py:26-42: h = 1,
// 2, 4, ..., x[i] = a + b, x[i+h] = a - b), so for each element the sequence of
// float32 additions is the reference's and the results agree bit for bit (the
// final scale is a multiply by s, exact whenever m*n is an even power of two).
//
// A batch of matrices (E, m, n) with per-matrix sign vectors (E, m), (E, n) runs
// in the same launches (expert-batched dispatch).
//
// Rows (last axis, contiguous): one workgroup per row, staged in LDS (n <= 16384).
// Columns (first axis, stride n): m = a*b with b = min(m, 128); a first pass does
// the stages h < b on tiles of b consecutive rows x 64 consecutive columns, a
// second the stages h >= b on tiles of a rows spaced b apart; every global access
// reads or writes 256 contiguous bytes of a row (4n bytes when n < 64).  No
// transposes.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <type_traits>

#include "bcjr_kernels.h"

namespace bcjr {

namespace {

constexpr int kRowThreads = 256;
constexpr int kColTile = 64;  // columns per column-pass tile (fewer when n < 64)
constexpr int kColThreads = 256;

// One butterfly stage of span h on n values in LDS: pairs (i, i + h) with
// i = 2h * (j / h) + j % h for j < n/2.
__device__ __forceinline__ void stage(float* v, int n, int h, int tid, int nthr) {
  for (int j = tid; j < (n >> 1); j += nthr) {
    const int i = ((j & ~(h - 1)) << 1) | (j & (h - 1));
    const float a = v[i], b = v[i + h];
    v[i] = a + b;
    v[i + h] = a - b;
  }
}

struct RowsParams {
  const float* x;
  float* out;
  long long rows;
  int n;
  const float* pre;       // (rows / vec_rows, n) multiplies x before the transform, or null
  const float* post;      // (rows / vec_rows, n) multiplies the result, or null
  long long vec_rows;     // consecutive rows sharing one pre/post vector (m of a batch)
  const float* row_sign;  // (rows) multiplies row r of the result, or null
  float scale;
};

__global__ __launch_bounds__(kRowThreads) void fwht_rows_kernel(RowsParams P) {
  extern __shared__ __align__(16) float v[];
  const int n = P.n, tid = threadIdx.x, nthr = blockDim.x;
  for (long long r = blockIdx.x; r < P.rows; r += gridDim.x) {
    const float* xr = P.x + (size_t)r * n;
    const size_t vo = (size_t)(r / P.vec_rows) * n;
    for (int i = tid; i < n; i += nthr) v[i] = P.pre ? xr[i] * P.pre[vo + i] : xr[i];
    __syncthreads();
    for (int h = 1; h < n; h <<= 1) {
      stage(v, n, h, tid, nthr);
      __syncthreads();
    }
    const float rs = P.row_sign ? P.row_sign[r] : 1.0f;
    float* orow = P.out + (size_t)r * n;
    for (int i = tid; i < n; i += nthr) {
      float y = v[i];
      if (P.post) y *= P.post[vo + i];
      orow[i] = (y * rs) * P.scale;
    }
    __syncthreads();
  }
}

struct ColsParams {
  float* x;               // (batch, m, n) transformed in place
  long long mat_stride;   // m * n
  int m;                  // rows per matrix (row_sign offset of matrix e is e * m)
  int n;
  int C;                  // tile width: min(kColTile, n), a power of two dividing n
  int len;                // transform length along the column (tile rows)
  long long step;         // floats between consecutive tile rows
  long long outer_stride; // floats between tiles of consecutive outer index
  int outer;              // outer index count
  int batch;              // matrices
  const float* row_sign;  // (batch, m) multiplies row o*row_o + p*row_p of the result, or null
  int row_o, row_p;
  float scale;
};

__global__ __launch_bounds__(kColThreads) void fwht_cols_kernel(ColsParams P) {
  extern __shared__ __align__(16) float t[];  // len x C
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int C = P.C;
  const int ncb = P.n / C;
  const long long per_mat = (long long)P.outer * ncb;
  const long long tiles = per_mat * P.batch;
  for (long long g = blockIdx.x; g < tiles; g += gridDim.x) {
    const long long e = g / per_mat, gm = g - e * per_mat;
    const int o = (int)(gm / ncb), cb = (int)(gm % ncb);
    float* base = P.x + (size_t)e * P.mat_stride + (size_t)o * P.outer_stride + (size_t)cb * C;
    const float* rsgn = P.row_sign ? P.row_sign + (size_t)e * P.m : nullptr;
    for (int e = tid; e < P.len * C; e += nthr) {
      const int p = e / C, c = e % C;
      t[e] = base[(size_t)p * P.step + c];
    }
    __syncthreads();
    // Stage h along the tile rows for every column: butterfly (p, p + h) of
    // column c is item j = q * C + c, q < len/2.
    for (int h = 1; h < P.len; h <<= 1) {
      for (int j = tid; j < (P.len >> 1) * C; j += nthr) {
        const int q = j / C, c = j % C;
        const int p = ((q & ~(h - 1)) << 1) | (q & (h - 1));
        const float a = t[p * C + c], b = t[(p + h) * C + c];
        t[p * C + c] = a + b;
        t[(p + h) * C + c] = a - b;
      }
      __syncthreads();
    }
    for (int e = tid; e < P.len * C; e += nthr) {
      const int p = e / C, c = e % C;
      float y = t[e];
      if (rsgn) y *= rsgn[o * P.row_o + p * P.row_p];
      base[(size_t)p * P.step + c] = y * P.scale;
    }
    __syncthreads();
  }
}

int grid_for(long long items, int max_blocks) {
  return (int)(items < max_blocks ? items : max_blocks);
}

// ---------------------------------------------------------------------------
// Tiled FWHT for n >= 64: a tile of up to 2^15 floats in LDS, stages done in
// registers a few at a time ("radix steps": each thread loads the E
// elements whose indices differ only in the step's bits, applies those stages
// in order, and stores them back).  Stage h acts on index bit log2(h) of the
// tile, so with rows laid out contiguously the row transform is the stages on
// bits [0, log2 n) and the column transform within the tile is the stages on
// the row bits above.  Every element sees the additions of fwht_numpy in the
// same order, so results are bit-identical to the per-stage kernels.
//
//   pass 1 (tile_rows_kernel): RB = 2^14 / n consecutive rows of a matrix (64
//     KiB, two workgroups per CU); radix step 0 (bits 0-4) loads 32
//     consecutive floats per thread from HBM, later steps (radix 8) go through LDS, the
//     last one stores to HBM; the column stages h < RB run on the same tile.
//   pass 2 (tile_cols_kernel): column stages h0 <= h < h0 * len on tiles of
//     len <= 1024 rows spaced h0 apart x 32 columns; loads and stores go
//     straight to HBM (32 lanes = 128 contiguous bytes of a row).
// An 8192 x 2048 matrix takes 2 passes over HBM (the per-stage kernels take 3).
// LDS rows of 32 floats carry 4 floats of padding, so radix step 0's
// per-thread 32-float runs (128-bit reads) and the later steps' strided accesses are
// free of bank conflicts.
// ---------------------------------------------------------------------------
// pass 1: 2^14-float tiles (72 KiB padded), 512 threads, two workgroups per CU
constexpr int kRowTileBits = 14;
constexpr int kRowTile = 1 << kRowTileBits;
constexpr int kRowThreads2 = kRowTile / 32;
// pass 2: 2^15-float tiles (144 KiB padded) of up to 1024 rows x 32 columns
constexpr int kColTileBits = 15;
constexpr int kColTileMax = 1 << kColTileBits;
constexpr int kColThreads2 = 1024;
constexpr int kColBits = 5;  // 32 columns: 128 contiguous bytes of a row
constexpr size_t padded_bytes(int floats) { return (size_t)(floats + (floats >> 5) * 4) * sizeof(float); }
// LDS of a pass: the padded tile plus its row factors (2 per row in pass 1, 1 in pass 2)
constexpr size_t rows_lds_bytes(int floats, int rows) { return padded_bytes(floats) + 2 * rows * sizeof(float); }
constexpr size_t cols_lds_bytes(int len) { return padded_bytes(len << kColBits) + len * sizeof(float); }

__device__ __forceinline__ uint32_t lds_pad(uint32_t i) { return i + ((i >> 5) << 2); }

// Butterflies of stages 1, 2, ..., E/2 (in slot space) on v[0..E).
template <int E>
__device__ __forceinline__ void slot_stages(float (&v)[E]) {
#pragma unroll
  for (int hs = 1; hs < E; hs <<= 1) {
#pragma unroll
    for (int s = 0; s < E; ++s) {
      if (!(s & hs)) {
        const float a = v[s], b = v[s + hs];
        v[s] = a + b;
        v[s + hs] = a - b;
      }
    }
  }
}

// One radix-E step on bits [k0, k0 + log2 E) of a tile of T floats: group g
// holds the E indices base + s * 2^k0.  LD(g, base, v) fills v, ST(g, base, v)
// stores it; each is written for one address space.
template <int E, typename LD, typename ST>
__device__ __forceinline__ void radix_step(uint32_t T, uint32_t k0, LD ld, ST st) {
  constexpr uint32_t LE = E == 2 ? 1 : E == 4 ? 2 : 3;
  static_assert(E == 2 || E == 4 || E == 8, "radix");
  const uint32_t lowmask = (1u << k0) - 1u;
  for (uint32_t g = threadIdx.x; g < T / E; g += blockDim.x) {
    const uint32_t base = ((g >> k0) << (k0 + LE)) | (g & lowmask);
    float v[E];
    ld(base, v);
    slot_stages<E>(v);
    st(base, v);
  }
}

template <int E>
struct LdsIO {  // LDS loads / stores of a radix step's E elements
  float* t;
  uint32_t k0;
  __device__ __forceinline__ void load(uint32_t base, float (&v)[E]) const {
#pragma unroll
    for (int s = 0; s < E; ++s) v[s] = t[lds_pad(base + ((uint32_t)s << k0))];
  }
  __device__ __forceinline__ void store(uint32_t base, const float (&v)[E]) const {
#pragma unroll
    for (int s = 0; s < E; ++s) t[lds_pad(base + ((uint32_t)s << k0))] = v[s];
  }
};

// Dispatch on the radix (3, 2 or 1 bits).  F(std::integral_constant<int, E>) runs the step.
template <typename F>
__device__ __forceinline__ void with_radix(uint32_t bits, F f) {
  if (bits == 3) f(std::integral_constant<int, 8>());
  else if (bits == 2) f(std::integral_constant<int, 4>());
  else f(std::integral_constant<int, 2>());
}

struct TileRowsParams {
  const float* x;
  float* out;
  int batch;
  int m;                  // rows per matrix
  int n;                  // row length, 64 <= n <= 16384, power of two
  int rb;                 // rows per tile (power of two, rb * n <= 2^14, rb | m)
  int col_stages;         // 1: also the column stages h < rb (the RHT); 0: rows only
  const float* pre;       // (batch, n) multiplies x before the row transform, or null
  const float* post;      // (batch, n) multiplies after the row transform, or null
  const float* row_mid;   // (batch, m) multiplies row r after the row transform, or null
  const float* row_end;   // (batch, m) multiplies row r at the store, or null
  float scale;            // multiplies every element at the store
};

// Factors are +-1 signs and one scale, so a product of them multiplies exactly
// like the separate multiplications: v * (r * s) == (v * r) * s.
__global__ __launch_bounds__(kRowThreads2) void tile_rows_kernel(TileRowsParams P) {
  extern __shared__ __align__(16) float t[];
  const uint32_t n = (uint32_t)P.n, rb = (uint32_t)P.rb;
  const uint32_t nb = (uint32_t)__builtin_ctz(n);
  const uint32_t T = rb * n;
  const uint32_t tb = (uint32_t)__builtin_ctz(T);
  const uint32_t cb_end = P.col_stages ? tb : nb;  // stage bits done by this pass
  float* f_mid = t + lds_pad(T);                    // rb row factors applied after the row stages
  float* f_end = f_mid + rb;                         // rb row factors (times scale) at the store
  const uint32_t tiles_per_mat = (uint32_t)P.m / rb;
  const long long tiles = (long long)P.batch * tiles_per_mat;
  // Radix steps: bits [0, 5) from HBM, then 3-bit chunks up to nb (row stages), then
  // 3-bit chunks up to cb_end (column stages); n >= 64, so at least one step
  // follows step 0, and the last one stores to HBM.
  uint32_t last_k0 = 5;
  for (uint32_t k = 5; k < nb; k += 3) last_k0 = k;
  for (uint32_t k = nb; k < cb_end; k += 3) last_k0 = k;
  for (long long tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int e = (int)(tile / tiles_per_mat);
    const uint32_t r0 = (uint32_t)(tile - (long long)e * tiles_per_mat) * rb;
    const size_t off = ((size_t)e * P.m + r0) * (size_t)n;  // the tile is rb consecutive rows
    const float* src = P.x + off;
    float* dst = P.out + off;
    const float* pre = P.pre ? P.pre + (size_t)e * n : nullptr;
    const float* post = P.post ? P.post + (size_t)e * n : nullptr;
    for (uint32_t i = threadIdx.x; i < rb; i += blockDim.x) {
      f_mid[i] = P.row_mid ? P.row_mid[(size_t)e * P.m + r0 + i] : 1.0f;
      f_end[i] = (P.row_end ? P.row_end[(size_t)e * P.m + r0 + i] : 1.0f) * P.scale;
    }
    // radix step 0: bits [0, 5) from HBM, 32 consecutive floats per thread
    for (uint32_t g = threadIdx.x; g < T / 32; g += blockDim.x) {
      float v[32];
      const float4* s4 = reinterpret_cast<const float4*>(src + g * 32);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float4 q = s4[j];
        v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
      }
      if (pre) {
        const float4* p4 = reinterpret_cast<const float4*>(pre + ((g * 32) & (n - 1)));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float4 q = p4[j];
          v[4 * j] *= q.x; v[4 * j + 1] *= q.y; v[4 * j + 2] *= q.z; v[4 * j + 3] *= q.w;
        }
      }
      slot_stages<32>(v);
      float4* d4 = reinterpret_cast<float4*>(t + lds_pad(g * 32));
#pragma unroll
      for (int j = 0; j < 8; ++j) d4[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    }
    __syncthreads();
    // row steps: bits [5, nb)
    for (uint32_t k0 = 5; k0 < nb; k0 += 3) {
      const uint32_t bits = nb - k0 < 3 ? nb - k0 : 3;
      with_radix(bits, [&](auto ec) {
        constexpr int E = decltype(ec)::value;
        const LdsIO<E> io{t, k0};
        auto ld = [&](uint32_t b, float (&v)[E]) { io.load(b, v); };
        if (k0 != last_k0) {
          radix_step<E>(T, k0, ld, [&](uint32_t b, const float (&v)[E]) { io.store(b, v); });
        } else {  // rows only: every factor at the store (columns vary within a group)
          radix_step<E>(T, k0, ld, [&](uint32_t b, const float (&v)[E]) {
#pragma unroll
            for (int s = 0; s < E; ++s) {
              const uint32_t i = b + ((uint32_t)s << k0);
              float f = f_mid[i >> nb] * f_end[i >> nb];
              if (post) f *= post[i & (n - 1)];
              dst[i] = v[s] * f;
            }
          });
        }
      });
      __syncthreads();
    }
    // column steps: bits [nb, cb_end); the group's column is fixed (bits < nb of base)
    for (uint32_t k0 = nb; k0 < cb_end; k0 += 3) {
      const uint32_t bits = cb_end - k0 < 3 ? cb_end - k0 : 3;
      with_radix(bits, [&](auto ec) {
        constexpr int E = decltype(ec)::value;
        const LdsIO<E> io{t, k0};
        auto ld_first = [&](uint32_t b, float (&v)[E]) {
          io.load(b, v);
          const float fc = post ? post[b & (n - 1)] : 1.0f;
#pragma unroll
          for (int s = 0; s < E; ++s) v[s] *= fc * f_mid[(b + ((uint32_t)s << k0)) >> nb];
        };
        auto ld = [&](uint32_t b, float (&v)[E]) { io.load(b, v); };
        auto st_lds = [&](uint32_t b, const float (&v)[E]) { io.store(b, v); };
        auto st_hbm = [&](uint32_t b, const float (&v)[E]) {
#pragma unroll
          for (int s = 0; s < E; ++s) {
            const uint32_t i = b + ((uint32_t)s << k0);
            dst[i] = v[s] * f_end[i >> nb];
          }
        };
        const bool first = k0 == nb, last = k0 == last_k0;
        if (first && last) radix_step<E>(T, k0, ld_first, st_hbm);
        else if (first) radix_step<E>(T, k0, ld_first, st_lds);
        else if (last) radix_step<E>(T, k0, ld, st_hbm);
        else radix_step<E>(T, k0, ld, st_lds);
      });
      __syncthreads();
    }
  }
}

struct TileColsParams {
  float* x;               // (batch, m, n) transformed in place
  int batch, m, n;
  int h0;                 // first stage span of the pass
  int len;                // rows per tile (power of two <= 1024): stages h0 .. h0 * len / 2
  const float* row_end;   // (batch, m) multiplies row r at the store, or null
  float scale;            // multiplies every element at the store
};

__global__ __launch_bounds__(kColThreads2) void tile_cols_kernel(TileColsParams P) {
  extern __shared__ __align__(16) float t[];
  constexpr uint32_t CB = kColBits, C = 1u << CB;
  const uint32_t n = (uint32_t)P.n, len = (uint32_t)P.len, h0 = (uint32_t)P.h0;
  const uint32_t T = len * C;
  const uint32_t tb = CB + (uint32_t)__builtin_ctz(len);
  const uint32_t per_mat_o = (uint32_t)P.m / len, ncb = n / C;
  float* f_end = t + lds_pad(T);  // len row factors (times scale) at the store
  const long long tiles = (long long)P.batch * per_mat_o * ncb;
  uint32_t last_k0 = CB;
  for (uint32_t k = CB; k < tb; k += 3) last_k0 = k;
  for (long long tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int e = (int)(tile / ((long long)per_mat_o * ncb));
    const uint32_t rest = (uint32_t)(tile - (long long)e * per_mat_o * ncb);
    const uint32_t o = rest / ncb, cb = rest - o * ncb;
    const uint32_t o_lo = o % h0, o_hi = o / h0;
    const uint32_t row0 = o_hi * h0 * len + o_lo;  // tile row p is matrix row row0 + p * h0
    float* base = P.x + (size_t)e * P.m * n + (size_t)row0 * n + (size_t)cb * C;
    for (uint32_t p = threadIdx.x; p < len; p += blockDim.x)
      f_end[p] = (P.row_end ? P.row_end[(size_t)e * P.m + row0 + p * h0] : 1.0f) * P.scale;
    __syncthreads();
    // tile index i = p * C + c  <->  base[p * h0 * n + c]
    const size_t rstride = (size_t)h0 * n;
    for (uint32_t k0 = CB; k0 < tb; k0 += 3) {
      const uint32_t bits = tb - k0 < 3 ? tb - k0 : 3;
      with_radix(bits, [&](auto ec) {
        constexpr int E = decltype(ec)::value;
        const LdsIO<E> io{t, k0};
        auto ld_hbm = [&](uint32_t b, float (&v)[E]) {
#pragma unroll
          for (int s = 0; s < E; ++s) {
            const uint32_t i = b + ((uint32_t)s << k0);
            v[s] = base[(size_t)(i >> CB) * rstride + (i & (C - 1))];
          }
        };
        auto st_hbm = [&](uint32_t b, const float (&v)[E]) {
#pragma unroll
          for (int s = 0; s < E; ++s) {
            const uint32_t i = b + ((uint32_t)s << k0);
            base[(size_t)(i >> CB) * rstride + (i & (C - 1))] = v[s] * f_end[i >> CB];
          }
        };
        auto ld = [&](uint32_t b, float (&v)[E]) { io.load(b, v); };
        auto st = [&](uint32_t b, const float (&v)[E]) { io.store(b, v); };
        const bool first = k0 == CB, last = k0 == last_k0;
        if (first && last) radix_step<E>(T, k0, ld_hbm, st_hbm);
        else if (first) radix_step<E>(T, k0, ld_hbm, st);
        else if (last) radix_step<E>(T, k0, ld, st_hbm);
        else radix_step<E>(T, k0, ld, st);
      });
      __syncthreads();
    }
  }
}

}  // namespace

// Host launchers used by the C ABI.  Shapes are validated by the caller.
hipError_t launch_fwht_rows(const float* x, float* out, long long rows, int n, const float* pre,
                            const float* post, long long vec_rows, const float* row_sign, float scale,
                            int max_blocks, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  RowsParams P = {x, out, rows, n, pre, post, vec_rows > 0 ? vec_rows : rows, row_sign, scale};
  const size_t lds = (size_t)n * sizeof(float);  // n <= 16384: at most 64 KiB
  hipLaunchKernelGGL(fwht_rows_kernel, dim3(grid_for(rows, max_blocks)), dim3(kRowThreads), lds, stream, P);
  return hipGetLastError();
}

// Tiled RHT / row transform for n >= 64 (see tile_rows_kernel).  Forward:
// pre = sign_r, row_mid = sign_l; inverse: post = sign_r, row_end = sign_l.
// col = false transforms rows only (m = row count, any value).
hipError_t launch_fwht_tiled(const float* x, float* out, int batch, int m, int n, bool col, const float* pre,
                             const float* post, const float* row_mid, const float* row_end, float scale,
                             int max_blocks, hipStream_t stream) {
  if (batch == 0 || m == 0) return hipSuccess;
  static bool attr_set[64] = {};  // per device: opt-in to > 64 KiB of dynamic LDS
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64 || !attr_set[dev]) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&tile_rows_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)rows_lds_bytes(kRowTile, kRowTile / 64));
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&tile_cols_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)cols_lds_bytes(kColTileMax >> kColBits));
    if (e != hipSuccess) return e;
    if (dev >= 0 && dev < 64) attr_set[dev] = true;
  }
  int rb = kRowTile / n;
  if (col) {
    if (rb > m) rb = m;
  } else {
    // rows only: tiles of rb rows must divide the row count; use the largest power of two that does
    while (rb > 1 && (m % rb)) rb >>= 1;
  }
  const int rows_in_pass1 = col ? rb : 1;  // column span covered by pass 1
  const bool single = !col || rows_in_pass1 == m;
  TileRowsParams P1 = {x, out, batch, m, n, rb, col ? 1 : 0, pre, post, row_mid,
                       single ? row_end : nullptr, single ? scale : 1.0f};
  const long long tiles1 = (long long)batch * (m / rb);
  hipLaunchKernelGGL(tile_rows_kernel, dim3(grid_for(tiles1, max_blocks)), dim3(kRowThreads2),
                     rows_lds_bytes(rb * n, rb), stream, P1);
  e = hipGetLastError();
  if (e != hipSuccess || single) return e;
  for (int h0 = rb; h0 < m;) {
    int len = m / h0;
    if (len > (kColTileMax >> kColBits)) len = kColTileMax >> kColBits;
    const bool fin = h0 * len == m;
    TileColsParams P2 = {out, batch, m, n, h0, len, fin ? row_end : nullptr, fin ? scale : 1.0f};
    const long long tiles2 = (long long)batch * (m / len) * (n >> kColBits);
    hipLaunchKernelGGL(tile_cols_kernel, dim3(grid_for(tiles2, max_blocks)), dim3(kColThreads2),
                       cols_lds_bytes(len), stream, P2);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    h0 *= len;
  }
  return hipSuccess;
}

// H_m applied to every column of each (m, n) matrix of x (batch of them), in
// place; the result is multiplied by row_sign (batch, m) (after the transform)
// and scale.  m, n powers of two.
hipError_t launch_fwht_cols(float* x, int batch, int m, int n, const float* row_sign, float scale,
                            int max_blocks, hipStream_t stream) {
  if (batch == 0) return hipSuccess;
  const long long ms = (long long)m * n;
  const int b = m < 128 ? m : 128;
  const int a = m / b;
  const int C = n < kColTile ? n : kColTile;
  // pass 1: stages h < b, tiles of b consecutive rows
  ColsParams P1 = {x, ms, m, n, C, b, n, (long long)b * n, a, batch, nullptr, 0, 0, 1.0f};
  if (a == 1) {  // the only pass: signs and scale here
    P1.row_sign = row_sign;
    P1.row_o = 0;
    P1.row_p = 1;
    P1.scale = scale;
  }
  hipLaunchKernelGGL(fwht_cols_kernel, dim3(grid_for((long long)batch * a * (n / C), max_blocks)),
                     dim3(kColThreads), (size_t)b * C * sizeof(float), stream, P1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a == 1) return e;
  // pass 2: stages h >= b, tiles of a rows spaced b apart (row = ia*b + ib)
  ColsParams P2 = {x, ms, m, n, C, a, (long long)b * n, n, b, batch, row_sign, 1, b, scale};
  hipLaunchKernelGGL(fwht_cols_kernel, dim3(grid_for((long long)batch * b * (n / C), max_blocks)),
                     dim3(kColThreads), (size_t)a * C * sizeof(float), stream, P2);
  return hipGetLastError();
}

}  // namespace bcjr
