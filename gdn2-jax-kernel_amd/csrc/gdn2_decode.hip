// Single-token recurrent step on the (B,H,D,D) float32 state -- the decode
// step of a model served with GDN-2 layers.  Per (b,h) and token
//   S <- Diag(e^g) S,  pred = (b*k)^T S,  S <- S + k (w*v - pred)^T,
//   o = scale q^T S,
// the chunked forward's math with a chunk of one token (its state and output
// are sanitized like every chunk state and output, gdn2_fwd.py:355-356).  The
// state layout is h0 / h_final's: S[b][h][dk][dv] (gdn2_fwd.py:342).
//
// One 256-thread workgroup per (b,h) and slice of 32 state columns (B H D / 32
// workgroups: enough to spread one decode step over the chip): thread (column
// e, row group rg) keeps D / 8 state rows of column e in registers.  Both
// column reductions (pred and o) run over the rows, so the columns split
// freely; they are summed over the 8 row groups in LDS.  The state is read and
// written once (memory-bound); h_out may alias h_in.
#include "gdn2_common.h"

namespace gdn2 {

template <int D>
constexpr int decode_cols() { return 32; }

template <typename T, typename TG, int D>
__global__ void __launch_bounds__(256) decode_step(const T* q, const T* k, const T* v,
                                                   const T* w, const T* b, const TG* g,
                                                   float scale, const float* h_in,
                                                   float* h_out, float* out) {
  constexpr int CS = decode_cols<D>(), NSL = D / CS;
  constexpr int RG = 256 / CS, RPT = D / RG;   // row groups, rows per thread
  __shared__ float sQ[D], sK[D], sBK[D], sEG[D];
  __shared__ float sRed[RG][CS];
  const int tid = threadIdx.x, e = tid % CS, rg = tid / CS;
  const size_t bh = blockIdx.x / NSL;
  const int col = (blockIdx.x % NSL) * CS + e;
  const size_t vo = bh * D;                  // token vectors are (B,H,D) contiguous
  for (int i = tid; i < D; i += 256) {
    const float kv = to_f(k[vo + i]);
    sQ[i] = to_f(q[vo + i]);
    sK[i] = kv;
    sBK[i] = to_f(b[vo + i]) * kv;
    sEG[i] = __expf(to_f(g[vo + i]));
  }
  __syncthreads();
  const float* src = h_in ? h_in + bh * D * D : nullptr;
  float s[RPT];
  float pred = 0.f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg * RPT + i;
    s[i] = (src ? sanitize(src[(size_t)d * D + col]) : 0.f) * sEG[d];
    pred += sBK[d] * s[i];
  }
  sRed[rg][e] = pred;
  __syncthreads();
  pred = 0.f;
#pragma unroll
  for (int r = 0; r < RG; ++r) pred += sRed[r][e];
  const float delta = to_f(w[vo + col]) * to_f(v[vo + col]) - pred;
  __syncthreads();  // every thread has read sRed
  float o = 0.f;
  float* dst = h_out + bh * D * D;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg * RPT + i;
    const float nv = sanitize(s[i] + sK[d] * delta);
    dst[(size_t)d * D + col] = nv;
    o += sQ[d] * nv;
  }
  sRed[rg][e] = o;
  __syncthreads();
  if (rg == 0) {
    o = 0.f;
#pragma unroll
    for (int r = 0; r < RG; ++r) o += sRed[r][e];
    out[vo + col] = sanitize(scale * o);
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

}  // namespace gdn2
