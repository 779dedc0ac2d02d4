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
