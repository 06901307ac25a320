// Single-token recurrent step on the (B,H,D,D) float32 state -- the decode
// step of a model served with GDN-2 layers.  Per (b,h) and token
//   S <- Diag(e^g) S,  pred = (b*k)^T S,  S <- S + k (w*v - pred)^T,
//   o = scale q^T S,
// the chunked forward's math with a chunk of one token (its state and output
// are sanitized like every chunk state and output, gdn2_fwd.py:355-356).  The
// state layout is h0 / h_final's: S[b][h][dk][dv] (gdn2_fwd.py:342).
//
// One 256-thread workgroup per (b,h) and slice of 16 state columns (B H D / 16
// workgroups: enough to spread one decode step over the chip): thread (column
// quad c4, row group rg) keeps D / 64 state rows of four columns in registers,
// read and written with 16-byte accesses.  Both column reductions (pred and o)
// run over the rows, so the columns split freely; they are summed over the row
// groups of a wave by lane shuffles, then over the four waves in LDS.  The state
// is read and written once (memory-bound); h_out may alias h_in.
#include "gdn2_common.h"

namespace gdn2 {

template <int D>
constexpr int decode_cols() { return 16; }

// Sum of x over the lanes of a wave that hold the same column quad (lane & 3).
__device__ __forceinline__ f32x4 rowgroup_sum(f32x4 x) {
#pragma unroll
  for (int m = 4; m < 64; m *= 2)
#pragma unroll
    for (int c = 0; c < 4; ++c) x[c] += __shfl_xor(x[c], m);
  return x;
}

template <typename T, typename TG, int D>
__global__ void __launch_bounds__(256) decode_step(const T* q, const T* k, const T* v,
                                                   const T* w, const T* b, const TG* g,
                                                   float scale, const float* h_in,
                                                   float* h_out, float* out) {
  constexpr int CS = decode_cols<D>(), NSL = D / CS;
  constexpr int C4 = CS / 4, RG = 256 / C4, RPT = D / RG;   // row groups, rows per thread
  static_assert(RPT >= 1 && D % RG == 0, "rows must split over the row groups");
  __shared__ float sQ[D], sK[D], sBK[D], sEG[D];
  __shared__ f32x4 sRed[4][C4];   // per wave and column quad
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c4 = tid % C4, rg = tid / C4;
  const size_t bh = blockIdx.x / NSL;
  const int col = (blockIdx.x % NSL) * CS + 4 * c4;   // first of this thread's four columns
  const size_t vo = bh * D;                  // token vectors are (B,H,D) contiguous
  // the state rows and this thread's w, v first: their loads are in flight while
  // the token vectors are gathered into LDS (the step is latency-bound)
  const float* src = h_in ? h_in + bh * D * D : nullptr;
  f32x4 s[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    s[i] = src ? load4f(src + (size_t)(rg * RPT + i) * D + col) : f32x4{0.f, 0.f, 0.f, 0.f};
  float wv4[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) wv4[c] = to_f(w[vo + col + c]) * to_f(v[vo + col + c]);
  for (int i = tid; i < D; i += 256) {
    const float kv = to_f(k[vo + i]);
    sQ[i] = to_f(q[vo + i]);
    sK[i] = kv;
    sBK[i] = to_f(b[vo + i]) * kv;
    sEG[i] = __expf(to_f(g[vo + i]));
  }
  __syncthreads();
  f32x4 pred = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg * RPT + i;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s[i][c] = sanitize(s[i][c]) * sEG[d];
      pred[c] += sBK[d] * s[i][c];
    }
  }
  pred = rowgroup_sum(pred);
  if (lane < C4) sRed[wave][lane] = pred;
  __syncthreads();
  pred = sRed[0][c4] + sRed[1][c4] + sRed[2][c4] + sRed[3][c4];
  f32x4 delta;
#pragma unroll
  for (int c = 0; c < 4; ++c) delta[c] = wv4[c] - pred[c];
  __syncthreads();  // every thread has read sRed
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  float* dst = h_out + bh * D * D;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg * RPT + i;
    f32x4 nv;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      nv[c] = sanitize(s[i][c] + sK[d] * delta[c]);
      o[c] += sQ[d] * nv[c];
    }
    store4(dst + (size_t)d * D + col, nv);
  }
  o = rowgroup_sum(o);
  if (lane < C4) sRed[wave][lane] = o;
  __syncthreads();
  if (tid < C4) {
    const f32x4 t = sRed[0][tid] + sRed[1][tid] + sRed[2][tid] + sRed[3][tid];
    store4(out + vo + (blockIdx.x % NSL) * CS + 4 * tid, sanitize4(scale * t));
  }
}

template <typename T, typename TG, int D>
hipError_t launch_decode(hipStream_t st, int B, int H, const void* q, const void* k,
                         const void* v, const void* w, const void* b, const void* g,
                         float scale, const float* h_in, float* h_out, float* out) {
  launch_mark(st);
  hipLaunchKernelGGL((decode_step<T, TG, D>), dim3((size_t)B * H * (D / decode_cols<D>())),
                     dim3(256), 0, st,
                     (const T*)q, (const T*)k, (const T*)v, (const T*)w, (const T*)b,
                     (const TG*)g, scale, h_in, h_out, out);
  launch_mark(st);
  return hipGetLastError();
}

#define GDN2_INST_DEC(T, TG, D)                                                            \
  template hipError_t launch_decode<T, TG, D>(hipStream_t, int, int, const void*,         \
                                              const void*, const void*, const void*,      \
                                              const void*, const void*, float,            \
                                              const float*, float*, float*);
GDN2_INST_DEC(float, float, 64)
GDN2_INST_DEC(float, float, 128)
GDN2_INST_DEC(bf16_t, float, 64)
GDN2_INST_DEC(bf16_t, float, 128)
GDN2_INST_DEC(bf16_t, bf16_t, 64)
GDN2_INST_DEC(bf16_t, bf16_t, 128)
GDN2_INST_DEC(float, float, 256)
GDN2_INST_DEC(bf16_t, float, 256)
GDN2_INST_DEC(bf16_t, bf16_t, 256)

// This translation unit's clip bound on the current device (gdn2_set_clip).
hipError_t set_clip_decode(float c) { return set_unit_clip(c); }

}  // namespace gdn2
