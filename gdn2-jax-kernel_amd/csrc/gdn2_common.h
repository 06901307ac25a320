// Device-side building blocks shared by the gfx950 GDN-2 kernels.
//
// MFMA tile conventions (64-lane wavefront, lane = 16*lg + li):
//   * An operand fragment is the 16-byte slice a lane feeds one k-group of a
//     16x16 MFMA: lane (li, lg) supplies row li of the left operand X and row
//     li of the right operand Y, at the k positions owned by lane-group lg.
//     The product of one k-group is D[m][n] += sum_k X[m][k] * Y[n][k].
//   * float32 k-group = 16 k positions, 4 instructions v_mfma_f32_16x16x4_f32;
//     lane-group lg owns k = 4*lg + e (e = 0..3) of each group.
//     bfloat16 k-group = 32 k positions, 1 instruction v_mfma_f32_16x16x32_bf16;
//     lane-group lg owns k = 8*lg + e (e = 0..7).  Which k a lane-group owns
//     only has to agree between the two operands, so either layout is a
//     16-byte contiguous slice of a row (byte offset 64*j + 16*lg in k-group j).
//   * The 16x16 fp32 result sits in "C layout": lane holds D[4*lg + r][li],
//     r = 0..3.  Feeding a C-layout tile back as an operand therefore uses the
//     k positions {4*lg + r} (fp32: exactly the owned set) or, for bf16, the
//     two tiles 2p, 2p+1 give k = {32p + 4lg + r} U {32p + 16 + 4lg + r}; the
//     other operand is then read with the matching "chained" pattern.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <type_traits>
#include <stddef.h>
#include <stdint.h>

namespace gdn2 {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16_t;

// Reference saturation constant, gdn2_fwd.py:33: the default clip bound.
constexpr float kClip = 1e4f;
// The clip bound in use: the reference's module constant CLIP, which its README
// overrides after import (README.md:87-92).  Every translation unit that
// launches kernels holds a copy in constant memory (kClip until set), which its
// host code sets on the current device with set_unit_clip (synchronous); the C
// ABI's gdn2_set_clip sets them all.
[[maybe_unused]] static __constant__ float g_clip = kClip;
[[maybe_unused]] static inline hipError_t set_unit_clip(float c) {
  return hipMemcpyToSymbol(HIP_SYMBOL(g_clip), &c, sizeof(c), 0, hipMemcpyHostToDevice);
}

// Largest log-decay the single-center factorisation of a diagonal 16 x 16 score
// block takes: a factor e^{+-60} times an operand keeps the product finite and,
// for operands down to 2e-12, normal in float32 and bfloat16 (MFMA may flush
// denormals).  Blocks with more decay between a token and the block's 8th are
// summed by the hierarchical fallback instead.
constexpr float kMaxDiagExp = 60.f;

// nan -> 0, +-inf -> +-CLIP, clip to [-CLIP, CLIP]: gdn2_fwd.py:42-44.
// max(x, 0) + min(x, 0) is x, or 0 for NaN (IEEE maxNum / minNum return the
// non-NaN operand); v_med3 then clamps (+-inf included).  Four independent
// VALU operations per value and no compare: a NaN test through VCC would
// serialise every element of a tile behind one register.
__device__ __forceinline__ float sanitize(float x) {
  const float y = fmaxf(x, 0.f) + fminf(x, 0.f);
  return __builtin_amdgcn_fmed3f(y, -g_clip, g_clip);
}
__device__ __forceinline__ f32x4 sanitize4(f32x4 v) {
  return f32x4{sanitize(v[0]), sanitize(v[1]), sanitize(v[2]), sanitize(v[3])};
}

template <typename T> struct Tr;
template <> struct Tr<float> {
  static constexpr int KC = 4;     // elements per lane per k-group
  static constexpr int KS = 16;    // k positions per k-group
  using Op = f32x4;
};
template <> struct Tr<bf16_t> {
  static constexpr int KC = 8;
  static constexpr int KS = 32;
  using Op = bf16x8;
};

__device__ __forceinline__ void mma(f32x4& acc, const f32x4& x, const f32x4& y) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[0], y[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[1], y[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[2], y[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[3], y[3], acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const bf16x8& x, const bf16x8& y) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, acc, 0, 0, 0);
}

// float32 products on the bfloat16 matrix cores ("split" form).  A float32
// operand element x is carried as hi = bf16(x) and lo = bf16(x - hi), so that
// x = hi + lo to about 2^-17 relative, and x y = hi_x hi_y + hi_x lo_y + lo_x hi_y
// + lo_x lo_y; the last term (2^-18 relative) is dropped.  Three 16x16x32 bfloat16
// MFMAs then replace the eight 16x16x4 float32 MFMAs of a 32-deep k step: the
// bfloat16 products are exact in the float32 accumulator.  The eight k positions
// a lane feeds are two consecutive float32 k-groups (elements e of both operands
// pair up, as in the float32 form), so the float32 operand layouts are unchanged.
struct Split8 {
  bf16x8 hi, lo;
};
__device__ __forceinline__ Split8 split8(const f32x4& a, const f32x4& b) {
  Split8 s;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    s.hi[e] = (bf16_t)a[e];
    s.hi[4 + e] = (bf16_t)b[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    s.lo[e] = (bf16_t)(a[e] - (float)s.hi[e]);
    s.lo[4 + e] = (bf16_t)(b[e] - (float)s.hi[4 + e]);
  }
  return s;
}
// Split pair layout of a float32 tile in LDS: in every 32-element run of a row
// (eight 16-byte chunks, chunk j = elements 4j .. 4j+3) the chunks j and 4 + j
// (j < 4) are replaced by the hi and the lo parts of their eight elements, in
// the order of split8(chunk j, chunk 4 + j).  A lane that reads chunks j and 4 + j
// for two consecutive k-groups of the float32 form then holds its split operand.
__device__ __forceinline__ Split8 split_read(const f32x4& chunk_hi, const f32x4& chunk_lo) {
  return Split8{__builtin_bit_cast(bf16x8, chunk_hi), __builtin_bit_cast(bf16x8, chunk_lo)};
}
// Byte offset, inside its 128-byte run, of the hi part of element e (0..31) of a
// run in the split pair layout (the lo part is 64 bytes further): chunk
// (e mod 16) / 4, slot 4 (e / 16) + e mod 4.  Four consecutive elements 4m .. 4m+3
// are one aligned 8-byte half chunk.
__host__ __device__ constexpr int split_pos(int e) {
  return ((e % 16) / 4) * 16 + ((e / 16) * 4 + e % 4) * 2;
}
struct Split4 {
  bf16x4 hi, lo;
};
__device__ __forceinline__ Split4 split4(const f32x4& a) {
  Split4 s;
#pragma unroll
  for (int e = 0; e < 4; ++e) s.hi[e] = (bf16_t)a[e];
#pragma unroll
  for (int e = 0; e < 4; ++e) s.lo[e] = (bf16_t)(a[e] - (float)s.hi[e]);
  return s;
}
// Four consecutive elements 4m .. 4m+3 (m = e / 4) of a row stored in the split
// pair layout, `row` the row's first byte.
__device__ __forceinline__ void split_store4(char* row, int e, const f32x4& v) {
  const Split4 s = split4(v);
  char* p = row + (e / 32) * 128 + split_pos(e % 32);
  *reinterpret_cast<bf16x4*>(p) = s.hi;
  *reinterpret_cast<bf16x4*>(p + 64) = s.lo;
}
__device__ __forceinline__ void split_store1(char* row, int e, float v) {
  const bf16_t hi = (bf16_t)v, lo = (bf16_t)(v - (float)hi);
  char* p = row + (e / 32) * 128 + split_pos(e % 32);
  *reinterpret_cast<bf16_t*>(p) = hi;
  *reinterpret_cast<bf16_t*>(p + 64) = lo;
}
// The four elements 4m .. 4m+3 of a row in the split pair layout, as hi and lo.
__device__ __forceinline__ Split4 split_load4(const char* row, int e) {
  const char* p = row + (e / 32) * 128 + split_pos(e % 32);
  return Split4{*reinterpret_cast<const bf16x4*>(p), *reinterpret_cast<const bf16x4*>(p + 64)};
}
__device__ __forceinline__ void mma3(f32x4& acc, const Split8& x, const Split8& y) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x.lo, y.hi, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x.hi, y.lo, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x.hi, y.hi, acc, 0, 0, 0);
}

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16_t x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float x) { return (bf16_t)x; }

// 16-byte operand fragment from KC floats.
__device__ __forceinline__ f32x4 make_op(const float* x, f32x4*) {
  return f32x4{x[0], x[1], x[2], x[3]};
}
__device__ __forceinline__ bf16x8 make_op(const float* x, bf16x8*) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16_t)x[e];
  return r;
}
template <typename T>
__device__ __forceinline__ typename Tr<T>::Op op_from(const float* x) {
  return make_op(x, (typename Tr<T>::Op*)nullptr);
}
template <typename T>
__device__ __forceinline__ typename Tr<T>::Op op_zero() {
  typename Tr<T>::Op r;
#pragma unroll
  for (int e = 0; e < Tr<T>::KC; ++e) r[e] = (T)0.f;
  return r;
}
template <typename T>
__device__ __forceinline__ typename Tr<T>::Op op_load(const T* p) {
  return *reinterpret_cast<const typename Tr<T>::Op*>(p);
}

// Load N consecutive elements of type X as floats (N*sizeof(X) a multiple of 8).
template <int N>
__device__ __forceinline__ void load_f(const float* p, float* out);
template <int N>
__device__ __forceinline__ void load_f(const bf16_t* p, float* out);

// Operand fragment of tile type T from elements stored as TI (T, or bfloat16
// widened to a float32 operand).
template <typename T, typename TI>
__device__ __forceinline__ typename Tr<T>::Op op_in(const TI* p) {
  if constexpr (std::is_same<T, TI>::value) {
    return op_load<T>(p);
  } else {
    float x[Tr<T>::KC];
    load_f<Tr<T>::KC>(p, x);
    return op_from<T>(x);
  }
}

template <int N>
__device__ __forceinline__ void load_f(const float* p, float* out) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    f32x4 t = *reinterpret_cast<const f32x4*>(p + i);
    out[i] = t[0]; out[i + 1] = t[1]; out[i + 2] = t[2]; out[i + 3] = t[3];
  }
}
template <int N>
__device__ __forceinline__ void load_f(const bf16_t* p, float* out) {
  static_assert(N % 4 == 0, "load_f reads groups of 4 or 8 elements");
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      bf16x8 t = *reinterpret_cast<const bf16x8*>(p + i);
#pragma unroll
      for (int e = 0; e < 8; ++e) out[i + e] = (float)t[e];
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      bf16x4 t = *reinterpret_cast<const bf16x4*>(p + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[i + e] = (float)t[e];
    }
  }
}

// Store 4 consecutive values of a C/R-layout row.
__device__ __forceinline__ void store4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void store4(bf16_t* p, f32x4 v) {
  bf16x4 r = {(bf16_t)v[0], (bf16_t)v[1], (bf16_t)v[2], (bf16_t)v[3]};
  *reinterpret_cast<bf16x4*>(p) = r;
}
__device__ __forceinline__ f32x4 load4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 load4f(const bf16_t* p) {
  bf16x4 t = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)t[0], (float)t[1], (float)t[2], (float)t[3]};
}

// Operand read from memory in the pattern that matches a C-layout chained
// operand (see header comment).  `p` points at k = 32p (bf16) / 16a (fp32).
__device__ __forceinline__ f32x4 op_chained(const float* p, int lg) {
  return *reinterpret_cast<const f32x4*>(p + 4 * lg);
}
__device__ __forceinline__ bf16x8 op_chained(const bf16_t* p, int lg) {
  bf16x4 lo = *reinterpret_cast<const bf16x4*>(p + 4 * lg);
  bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + 16 + 4 * lg);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
// Stored position of logical column c in the "chained order" used for bfloat16
// tiles that the serial state pass contracts over: inside each 32-column
// block, position 8*lg + 4*half + r holds column 16*half + 4*lg + r.  Then the
// k positions a lane-group feeds from two C-layout tiles (header comment) are
// one contiguous 16-byte run, and so are the values a lane holds of two
// consecutive C-layout tiles.  float32 tiles keep the identity order.
template <typename T>
__host__ __device__ constexpr int kpos(int c) {
  if constexpr (sizeof(T) == 4) {
    return c;
  } else {
    return (c & ~31) | (((c >> 2) & 3) << 3) | (((c >> 4) & 1) << 2) | (c & 3);
  }
}

// C-layout tiles as the other operand of a chained product.
__device__ __forceinline__ f32x4 op_from_c(const f32x4& t0, const f32x4&, f32x4*) { return t0; }
__device__ __forceinline__ bf16x8 op_from_c(const f32x4& t0, const f32x4& t1, bf16x8*) {
  bf16x8 r;
  r[0] = (bf16_t)t0[0]; r[1] = (bf16_t)t0[1]; r[2] = (bf16_t)t0[2]; r[3] = (bf16_t)t0[3];
  r[4] = (bf16_t)t1[0]; r[5] = (bf16_t)t1[1]; r[6] = (bf16_t)t1[2]; r[7] = (bf16_t)t1[3];
  return r;
}

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's bytes land at lds_base + 16*l, so
// `lds_base` must be the same for every lane of the wave.  Completion is
// tracked by vmcnt.
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)lds_base, 16,
                                   0, 0);
}
// 4 bytes per lane (global_load_lds_dword), lane l's bytes at lds_base + 4*l.
__device__ __forceinline__ void lds_dma4(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)lds_base, 4,
                                   0, 0);
}

// Wait until at most N vector memory instructions of this wave are in flight.
// Loads complete in issue order, so this waits for all but the last N issued.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Row-wise (16-lane) DPP helpers: inclusive prefix sum over lanes li = 0..15
// (row_shr 1,2,4,8 with out-of-row sources reading 0) and broadcast of lane n
// of each row (row_newbcast).
template <int CTRL>
__device__ __forceinline__ float row_shr_add(float x) {
  return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                 0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_scan16(float x) {
  x = row_shr_add<0x111>(x);
  x = row_shr_add<0x112>(x);
  x = row_shr_add<0x114>(x);
  return row_shr_add<0x118>(x);
}
// inclusive suffix sum over the 16 lanes of a row: lane i gets lanes i..15
// (row_shl steps; lanes shifted in from beyond the row read 0)
__device__ __forceinline__ float row_suffix16(float x) {
  x = row_shr_add<0x101>(x);
  x = row_shr_add<0x102>(x);
  x = row_shr_add<0x104>(x);
  return row_shr_add<0x108>(x);
}
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
             0, __builtin_bit_cast(int, x), 0x150 + N, 0xF, 0xF, false));
}

// Workgroup barrier for LDS data only: the wave's own LDS operations complete,
// then s_barrier.  Unlike __syncthreads() it does not drain vector memory
// operations, so global loads stay in flight and global stores (never read back
// by another wave of the workgroup where this is used) are not waited for.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Copy `rows` rows of `cols` elements (row pitch `gpitch` in global, `lpitch`
// in LDS) with 16-byte transactions spread over the workgroup.
template <typename T, int NT>
__device__ __forceinline__ void g2s(T* lds, int lpitch, const T* g, size_t gpitch, int rows,
                                    int cols, int tid) {
  constexpr int EPV = 16 / sizeof(T);
  const int cpr = cols / EPV;
  const int total = rows * cpr;
  for (int i = tid; i < total; i += NT) {
    const int r = i / cpr, cc = (i - r * cpr) * EPV;
    *reinterpret_cast<uint4*>(lds + r * lpitch + cc) =
        *reinterpret_cast<const uint4*>(g + r * gpitch + cc);
  }
}

// Compute units of the current device (host side; queried once per device).
inline int num_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Per-thread timing request set by gdn2_set_launch_events (host side).
struct LaunchEvents {
  void* const* ev = nullptr;
  int n = 0;
  int i = 0;
};
extern thread_local LaunchEvents g_launch_events;

// Record the next requested event on `st` (no-op without a request).
inline void launch_mark(hipStream_t st) {
  LaunchEvents& e = g_launch_events;
  if (e.ev && e.i < e.n) (void)hipEventRecord((hipEvent_t)e.ev[e.i], st);
  ++e.i;
}

}  // namespace gdn2
