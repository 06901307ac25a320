// Layout kernels of the stage entry points (the reference's kernels called one
// at a time): tile transposes between the reference's per-chunk tiles and the
// layouts the scans read, chunk rows to token rows and back, and B5's reverse
// cumsum.  Each is a plain copy-shaped kernel; none of them is on the fused
// forward's or backward's path.
#include <hip/hip_runtime.h>

#include "gdn2_common.h"
#include "gdn2_stage.h"

namespace gdn2 {

namespace {

// dst[m][c][r] = src[m][r][c] for matrices of R x C float32 (R, C multiples of
// 32), one 32 x 32 tile per workgroup; the grid covers the tiles of all matrices.
// With `shift` (groups of N matrices), source matrix i of a group goes to matrix
// i + 1 of the same group and the grid covers the first N - 1 of each group.
__global__ void __launch_bounds__(256) tile_transpose(const float* __restrict__ src,
                                                      float* __restrict__ dst, int R, int C,
                                                      int N, int shift) {
  __shared__ float t[32][33];
  const int tr = R / 32, tc = C / 32;
  size_t m = blockIdx.x / (size_t)(tr * tc);
  const int rem = (int)(blockIdx.x % (size_t)(tr * tc));
  size_t md = m;
  if (shift) {   // m counts the first N - 1 matrices of each group
    const size_t g = m / (N - 1), i = m % (N - 1);
    m = g * N + i;
    md = m + 1;
  }
  const int r0 = rem / tc * 32, c0 = rem % tc * 32;
  const float* s = src + m * R * C;
  float* d = dst + md * R * C;
  const int x = threadIdx.x & 31, y = threadIdx.x >> 5;
  for (int j = y; j < 32; j += 8) t[j][x] = s[(size_t)(r0 + j) * C + c0 + x];
  __syncthreads();
  for (int j = y; j < 32; j += 8) d[(size_t)(c0 + j) * R + r0 + x] = t[x][j];
}

// Rows between (B,H,N,BT,D) and (B,N*BT,H,D), four floats per thread.
__global__ void __launch_bounds__(256) rows_permute(const float* __restrict__ src,
                                                    float* __restrict__ dst, int B, int H,
                                                    int N, int BT, int D, int to_tokens,
                                                    int diff) {
  const size_t D4 = D / 4;
  const size_t total = (size_t)B * H * N * BT * D4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (size_t)gridDim.x * 256) {
    const size_t q = i % D4, row = i / D4;   // row of the chunk layout
    const int t = (int)(row % BT);
    const size_t cid = row / BT;             // (b, h, c)
    const int c = (int)(cid % N);
    const size_t bh = cid / N;
    const int h = (int)(bh % H);
    const size_t b = bh / H;
    const size_t crow = row * D + 4 * q;
    const size_t trow = (((b * N + c) * BT + t) * H + h) * D + 4 * q;
    if (to_tokens) {
      f32x4 v = *reinterpret_cast<const f32x4*>(src + crow);
      if (diff && t > 0) v -= *reinterpret_cast<const f32x4*>(src + crow - D);
      *reinterpret_cast<f32x4*>(dst + trow) = v;
    } else {
      *reinterpret_cast<f32x4*>(dst + crow) = *reinterpret_cast<const f32x4*>(src + trow);
    }
  }
}

// One thread per (tile, column): the suffix sums from the tile's last row up.
__global__ void __launch_bounds__(256) rev_cumsum(const float* __restrict__ dgc,
                                                  float* __restrict__ dg, size_t tiles, int BT,
                                                  int D) {
  const size_t total = tiles * D;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (size_t)gridDim.x * 256) {
    const size_t tile = i / D;
    const int col = (int)(i % D);
    const float* s = dgc + tile * BT * D + col;
    float* o = dg + tile * BT * D + col;
    float acc = 0.f;
    for (int r = BT - 1; r >= 0; --r) {
      acc += s[(size_t)r * D];
      o[(size_t)r * D] = sanitize(acc);
    }
  }
}

// dst[i] = sanitize(src[i]), or 0 without a source.
__global__ void __launch_bounds__(256) sanitize_copy(const float* __restrict__ src,
                                                     float* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    dst[i] = src ? sanitize(src[i]) : 0.f;
}

unsigned grid_for(size_t items) {
  const size_t blocks = (items + 255) / 256;
  return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

// One run of 32 floats per thread into the split pair layout.
__global__ void __launch_bounds__(256) split_run(const float* src, float* dst, size_t runs) {
  for (size_t r = (size_t)blockIdx.x * 256 + threadIdx.x; r < runs;
       r += (size_t)gridDim.x * 256) {
    f32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = load4f(src + r * 32 + 4 * j);
    char* row = reinterpret_cast<char*>(dst + r * 32);
#pragma unroll
    for (int j = 0; j < 8; ++j) split_store4(row, 4 * j, v[j]);
  }
}

}  // namespace

void split_runs(hipStream_t st, const float* src, float* dst, size_t runs) {
  if (runs > 0)
    hipLaunchKernelGGL(split_run, dim3(grid_for(runs)), dim3(256), 0, st, src, dst, runs);
}

void transpose_all(hipStream_t st, const float* src, float* dst, size_t n, int R, int C) {
  if (n > 0)
    hipLaunchKernelGGL(tile_transpose, dim3(n * (R / 32) * (C / 32)), dim3(256), 0, st, src, dst,
                       R, C, 0, 0);
}

void transpose_shift(hipStream_t st, const float* src, float* dst, size_t groups, int N, int R,
                     int C) {
  if (groups > 0 && N > 1)
    hipLaunchKernelGGL(tile_transpose, dim3(groups * (N - 1) * (R / 32) * (C / 32)), dim3(256),
                       0, st, src, dst, R, C, N, 1);
}

void chunk_rows_permute(hipStream_t st, const float* src, float* dst, int B, int H, int N,
                        int BT, int D, bool to_tokens, bool diff) {
  const size_t items = (size_t)B * H * N * BT * (D / 4);
  if (items > 0)
    hipLaunchKernelGGL(rows_permute, dim3(grid_for(items)), dim3(256), 0, st, src, dst, B, H, N,
                       BT, D, to_tokens ? 1 : 0, diff ? 1 : 0);
}

void reverse_cumsum(hipStream_t st, const float* dgc, float* dg, size_t tiles, int BT, int D) {
  if (tiles > 0 && D > 0)
    hipLaunchKernelGGL(rev_cumsum, dim3(grid_for(tiles * D)), dim3(256), 0, st, dgc, dg, tiles,
                       BT, D);
}

void sanitized_copy(hipStream_t st, const float* src, float* dst, size_t n) {
  if (n > 0)
    hipLaunchKernelGGL(sanitize_copy, dim3(grid_for(n)), dim3(256), 0, st, src, dst, n);
}

// This translation unit's clip bound on the current device (gdn2_set_clip).
hipError_t set_clip_stage(float c) { return set_unit_clip(c); }

}  // namespace gdn2
