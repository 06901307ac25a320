// C ABI of libgdn2_hip.so: validation, workspace sizing and dispatch to the
// templated gfx950 launchers.  Declared in include/gdn2.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gdn2.h"
#include "gdn2_common.h"
#include "gdn2_layout.h"
#include "gdn2_stage.h"

namespace gdn2 {

template <typename T, typename TG, int BT, int D, typename TI>
hipError_t launch_fwd(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                      const void* v, const void* w, const void* b, const void* g,
                      const float* h0, float scale, float* out, float* h_final, char* ws,
                      float* a_dbg, int flags, const Varlen* vl);

template <typename T, typename TG, int BT, int D, typename TI>
hipError_t launch_bwd(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                      const void* v, const void* w, const void* b, const void* g,
                      const float* h0, float scale, const float* dout, const float* dh_final,
                      void* dq, void* dk, void* dv, void* dw, void* db, void* dg, float* dh0,
                      const char* fws, char* ws, const int* cu_chunks, int nseq);

size_t bwd_ws_bytes(size_t nchunks, int BT, int D, size_t elem);
// The clip bound of each translation unit that launches kernels (gdn2_set_clip).
hipError_t set_clip_fwd(float c);
hipError_t set_clip_bwd(float c);
hipError_t set_clip_decode(float c);
hipError_t set_clip_stage(float c);
template <int D>
hipError_t launch_stage_dav(hipStream_t st, int B, int N, int H, const float* aqk,
                            const float* v_new, const float* dout, float* daqk, float* dv_new,
                            char* ws, size_t* need);
template <int D>
hipError_t launch_stage_dhu(hipStream_t st, int B, int N, int H, const float* dout,
                            const float* dv_partial, const float* w_pseudo, const float* qg,
                            const float* kg, const float* gc_last, float scale,
                            const float* dht, float* dh_all, float* dh0, float* dv_all,
                            char* ws, size_t* need);
template <int D>
hipError_t launch_stage_wy_dqkg(hipStream_t st, int B, int N, int H, const float* q,
                                const float* k, const float* b, const float* w, const float* v,
                                const float* gc, const float* A, const float* h_pre,
                                const float* v_new, const float* dout, const float* dv,
                                const float* dh_next, float scale, float* dq, float* dk,
                                float* db, float* dw, float* dv_raw, float* dgc, float* dakk,
                                char* ws, size_t* need);
template <int D>
hipError_t launch_stage_intra(hipStream_t st, int B, int T_len, int H, const float* daqk,
                              const float* dakk, const float* q, const float* k, const float* b,
                              const float* g, float scale, float* dq, float* dk, float* db,
                              float* dgc, char* ws, size_t* need);
template <typename TG, int D, typename TI>
hipError_t launch_stage_scores(hipStream_t st, int B, int T_len, int H, const void* q,
                               const void* k, const void* b, const void* g, float scale,
                               float* aqk, float* akk);
hipError_t launch_stage_solve(hipStream_t st, size_t nchunks, const float* akk, float* a_out);
template <typename TG, int D, typename TI>
hipError_t launch_stage_wy(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                           const void* v, const void* w, const void* b, const void* g,
                           const float* A, float* w_pseudo, float* u, float* kg, float* qg,
                           float* gc_last);
template <int D>
hipError_t launch_stage_combine(hipStream_t st, int B, int N, int H, const float* aqk,
                                const float* w_pseudo, const float* u, const float* kg,
                                const float* qg, const float* gc_last, const float* h0,
                                float scale, float* out, float* h_final, float* h_pre_all,
                                float* v_new_all, char* ws);

template <typename T, typename TG, int D>
hipError_t launch_decode(hipStream_t st, int B, int H, const void* q, const void* k,
                         const void* v, const void* w, const void* b, const void* g,
                         float scale, const float* h_in, float* h_out, float* out);

// Workspace element size: the MFMA operand type (float32 for GDN2_BF16_F32).
static size_t elem_size(int dtype) { return dtype == GDN2_BF16 ? 2 : 4; }

// Tag of GDN2_BF16_F32 in the dispatch: float32 tiles and arithmetic, bfloat16
// inputs and gradients.  Tile<X> / Stor<X> give the launchers' T and TI.
struct Bf16F32 {};
template <typename X> struct Tile { using type = X; };
template <> struct Tile<Bf16F32> { using type = float; };
template <typename X> struct Stor { using type = X; };
template <> struct Stor<Bf16F32> { using type = bf16_t; };

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static int check_ptrs(std::initializer_list<const void*> ps) {
  for (const void* p : ps) {
    if (!p) return GDN2_ERR_NULL;
    if (!aligned16(p)) return GDN2_ERR_ALIGN;
  }
  return GDN2_OK;
}
static int check_opt(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && !aligned16(p)) return GDN2_ERR_ALIGN;
  return GDN2_OK;
}

// Chunks per sequence, a short last chunk included (64-bit sum: T may be INT_MAX).
static int chunks_per_seq(int T, int BT) {
  return BT > 0 ? (int)(((long long)T + BT - 1) / BT) : 0;
}
static size_t nchunks(int B, int T, int H, int BT) {
  return (size_t)B * H * (size_t)chunks_per_seq(T, BT);
}

// gdn2_validate, with T % BT != 0 accepted when flags has GDN2_FWD_PARTIAL_CHUNK.
static int validate_fwd(int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
                        int flags) {
  if ((flags & GDN2_FWD_PARTIAL_CHUNK) && T > 0 && BT > 0 && T % BT != 0) {
    const int rc = gdn2_validate(B, T, H, D, BT, in_dtype, g_dtype);
    if (rc != GDN2_ERR_SEQ_LEN) return rc;
    // the same checks on the rounded-up length (the size limit included)
    return (long long)chunks_per_seq(T, BT) * BT > 0x7fffffffLL
               ? GDN2_ERR_SHAPE
               : gdn2_validate(B, chunks_per_seq(T, BT) * BT, H, D, BT, in_dtype, g_dtype);
  }
  return gdn2_validate(B, T, H, D, BT, in_dtype, g_dtype);
}

// Dispatch on (in dtype, g dtype, BT, D).
template <template <typename, typename, int, int> class F, typename... A>
static int dispatch(int in_dtype, int g_dtype, int BT, int D, A... args) {
#define GDN2_CASE(T, TG, BT_, D_)                                                   \
  if (BT == BT_ && D == D_) return F<T, TG, BT_, D_>::run(args...);
  if (in_dtype == GDN2_F32 && g_dtype == GDN2_F32) {
    GDN2_CASE(float, float, 64, 64)
    GDN2_CASE(float, float, 64, 128)
    GDN2_CASE(float, float, 64, 256)
  } else if (in_dtype == GDN2_BF16 && g_dtype == GDN2_F32) {
    GDN2_CASE(bf16_t, float, 64, 64)
    GDN2_CASE(bf16_t, float, 64, 128)
    GDN2_CASE(bf16_t, float, 128, 64)
    GDN2_CASE(bf16_t, float, 128, 128)
    GDN2_CASE(bf16_t, float, 64, 256)
  } else if (in_dtype == GDN2_BF16 && g_dtype == GDN2_BF16) {
    GDN2_CASE(bf16_t, bf16_t, 64, 64)
    GDN2_CASE(bf16_t, bf16_t, 64, 128)
    GDN2_CASE(bf16_t, bf16_t, 128, 64)
    GDN2_CASE(bf16_t, bf16_t, 128, 128)
    GDN2_CASE(bf16_t, bf16_t, 64, 256)
  } else if (in_dtype == GDN2_BF16_F32 && g_dtype == GDN2_F32) {
    GDN2_CASE(Bf16F32, float, 64, 64)
    GDN2_CASE(Bf16F32, float, 64, 128)
    GDN2_CASE(Bf16F32, float, 64, 256)
  } else if (in_dtype == GDN2_BF16_F32 && g_dtype == GDN2_BF16) {
    GDN2_CASE(Bf16F32, bf16_t, 64, 64)
    GDN2_CASE(Bf16F32, bf16_t, 64, 128)
    GDN2_CASE(Bf16F32, bf16_t, 64, 256)
  }
#undef GDN2_CASE
  return GDN2_ERR_CHUNK;
}

template <typename T, typename TG, int BT, int D>
struct FwdRun {
  static int run(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                 const void* v, const void* w, const void* b, const void* g, const float* h0,
                 float scale, float* out, float* h_final, char* ws, float* a_dbg,
                 int flags, const Varlen* vl) {
    hipError_t e = launch_fwd<typename Tile<T>::type, TG, BT, D, typename Stor<T>::type>(
        st, B, T_len, H, q, k, v, w, b, g, h0, scale, out, h_final, ws, a_dbg, flags, vl);
    return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
  }
};

template <typename T, typename TG, int BT, int D>
struct BwdRun {
  static int run(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                 const void* v, const void* w, const void* b, const void* g, const float* h0,
                 float scale, const float* dout, const float* dh_final, void* dq, void* dk,
                 void* dv, void* dw, void* db, void* dg, float* dh0, const char* fws,
                 char* ws, const int* cu_chunks, int nseq) {
    if constexpr (std::is_same_v<T, bf16_t>) {
      return GDN2_ERR_DTYPE;  // bfloat16 residuals: rejected by the entry points
    } else if constexpr (D > 128 && BT != 64) {
      return GDN2_ERR_CHUNK;  // D = 256 runs at chunk 64 only
    } else {
      hipError_t e = launch_bwd<typename Tile<T>::type, TG, BT, D, typename Stor<T>::type>(
          st, B, T_len, H, q, k, v, w, b, g, h0, scale, dout, dh_final, dq, dk, dv, dw, db, dg,
          dh0, fws, ws, cu_chunks, nseq);
      return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
    }
  }
};

// The stage entry points (the reference's kernels A-D one at a time): float32
// tiles at chunk 64; bfloat16 inputs are computed in float32 (GDN2_BF16_F32).
static int validate_stage(int B, int T, int H, int D, int BT, int in_dtype, int g_dtype) {
  if (BT != 64) return GDN2_ERR_CHUNK;
  return gdn2_validate(B, T, H, D, BT, in_dtype == GDN2_BF16 ? GDN2_BF16_F32 : in_dtype,
                       g_dtype);
}

// Dispatch of a stage launcher on (g storage type, D, input storage type).
template <template <typename, int, typename> class F, typename... A>
static int dispatch_stage(int in_dtype, int g_dtype, int D, A... args) {
#define GDN2_SCASE(TG, D_, TI) \
  if (D == D_) return F<TG, D_, TI>::run(args...);
  if (in_dtype == GDN2_F32) {
    GDN2_SCASE(float, 64, float)
    GDN2_SCASE(float, 128, float)
    GDN2_SCASE(float, 256, float)
  } else if (g_dtype == GDN2_F32) {
    GDN2_SCASE(float, 64, bf16_t)
    GDN2_SCASE(float, 128, bf16_t)
    GDN2_SCASE(float, 256, bf16_t)
  } else {
    GDN2_SCASE(bf16_t, 64, bf16_t)
    GDN2_SCASE(bf16_t, 128, bf16_t)
    GDN2_SCASE(bf16_t, 256, bf16_t)
  }
#undef GDN2_SCASE
  return GDN2_ERR_HEAD_DIM;
}

template <typename TG, int D, typename TI>
struct ScoresRun {
  static int run(hipStream_t st, int B, int T, int H, const void* q, const void* k,
                 const void* b, const void* g, float scale, float* aqk, float* akk) {
    hipError_t e = launch_stage_scores<TG, D, TI>(st, B, T, H, q, k, b, g, scale, aqk, akk);
    return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
  }
};

template <typename TG, int D, typename TI>
struct WyRun {
  static int run(hipStream_t st, int B, int T, int H, const void* q, const void* k,
                 const void* v, const void* w, const void* b, const void* g, const float* A,
                 float* w_pseudo, float* u, float* kg, float* qg, float* gc_last) {
    hipError_t e = launch_stage_wy<TG, D, TI>(st, B, T, H, q, k, v, w, b, g, A, w_pseudo, u, kg,
                                              qg, gc_last);
    return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
  }
};

template <typename T, typename TG, int D>
static int run_decode(hipStream_t st, int B, int H, const void* q, const void* k, const void* v,
                      const void* w, const void* b, const void* g, float scale,
                      const float* h_in, float* h_out, float* out) {
  hipError_t e = launch_decode<T, TG, D>(st, B, H, q, k, v, w, b, g, scale, h_in, h_out, out);
  return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

}  // namespace gdn2

namespace gdn2 {
thread_local LaunchEvents g_launch_events;
}

using namespace gdn2;

namespace {
// Clears the per-thread timing request when an entry point returns.
struct EventScope {
  ~EventScope() { g_launch_events = LaunchEvents{}; }
};
}  // namespace

extern "C" {

const char* gdn2_version(void) { return "0.1.0"; }

int gdn2_set_clip(float clip) {
  if (!(clip > 0.f) || !(clip <= 3.4e38f)) return GDN2_ERR_SHAPE;   // NaN, <= 0, inf
  const hipError_t e[] = {set_clip_fwd(clip), set_clip_bwd(clip), set_clip_decode(clip),
                          set_clip_stage(clip)};
  for (const hipError_t x : e)
    if (x != hipSuccess) return GDN2_ERR_LAUNCH;
  return GDN2_OK;
}

int gdn2_set_launch_events(void* const* events, int n) {
  g_launch_events = LaunchEvents{events, n > 0 ? n : 0, 0};
  return 0;
}

const char* gdn2_strerror(int code) {
  switch (code) {
    case GDN2_OK: return "ok";
    case GDN2_ERR_HEAD_DIM:
      return "head dim D must be 64, 128 or 256";
    case GDN2_ERR_SEQ_LEN: return "sequence length T must be divisible by the chunk size BT";
    case GDN2_ERR_CHUNK:
      return "chunk size BT must be 64 or 128 (128 needs GDN2_BF16 inputs and D <= 128)";
    case GDN2_ERR_DTYPE: return "unsupported dtype (inputs: GDN2_F32, GDN2_BF16 or GDN2_BF16_F32, the backward GDN2_F32 or GDN2_BF16_F32; g: float32, or bfloat16 with bfloat16 inputs)";
    case GDN2_ERR_NULL: return "required pointer is NULL";
    case GDN2_ERR_ALIGN: return "pointer is not 16-byte aligned";
    case GDN2_ERR_WORKSPACE: return "workspace too small";
    case GDN2_ERR_SHAPE: return "invalid shape (B and H must be >= 1, T >= 0)";
    case GDN2_ERR_LAUNCH: return "HIP kernel launch failed";
    case GDN2_ERR_FLAGS: return "invalid flags (GDN2_FWD_RAW_INPUTS cannot be combined with GDN2_FWD_SAVE_A; gdn2_fwd_noalloc takes no GDN2_FWD_SAVE_A)";
    case GDN2_ERR_SCRATCH:
      return "workload too large for gdn2_fwd_noalloc's fixed scratch (GDN2_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown error";
  }
}

int gdn2_validate(int B, int T, int H, int D, int BT, int in_dtype, int g_dtype) {
  if (B < 1 || H < 1 || T < 0) return GDN2_ERR_SHAPE;
  if (in_dtype != GDN2_F32 && in_dtype != GDN2_BF16 && in_dtype != GDN2_BF16_F32)
    return GDN2_ERR_DTYPE;
  if (g_dtype != GDN2_F32 && g_dtype != GDN2_BF16) return GDN2_ERR_DTYPE;
  if (in_dtype == GDN2_F32 && g_dtype != GDN2_F32) return GDN2_ERR_DTYPE;
  if (D != 64 && D != 128 && D != 256) return GDN2_ERR_HEAD_DIM;
  if (BT != 64 && BT != 128) return GDN2_ERR_CHUNK;
  if (BT == 128 && (in_dtype != GDN2_BF16 || D == 256)) return GDN2_ERR_CHUNK;
  if (T % BT != 0) return GDN2_ERR_SEQ_LEN;
  if ((double)B * T * H * D > 9.0e15) return GDN2_ERR_SHAPE;
  // launch grids: up to 8 workgroups per chunk (or per (b,h) and 16 columns of
  // the state), counted in 31 bits
  if ((double)B * H * ((double)T / BT + 1.0) * (D / 16) > 2147483647.0) return GDN2_ERR_SHAPE;
  return GDN2_OK;
}

// Forward workspace for the segment count that `flags` selects (automatic
// when its segment field is 0).  An inference call whose scan forms the outputs
// itself writes no h^T / v_new^T tiles, and its workspace has none, unless the
// call is the debug path (`debug`: the residual tiles are kept for inspection).
static size_t fwd_ws_need(int B, int T, int H, int D, int BT, int in_dtype, int flags,
                          bool debug = false) {
  const int N = chunks_per_seq(T, BT);
  const int es = (int)elem_size(in_dtype);
  const bool fused = state_out_waves_of(es, BT, D) > 0 && !(flags & GDN2_FWD_SAVE_A);
  const int S = state_segments((long long)B * H, N, D, es, (flags >> 8) & 0xff,
                               fused ? 32 : seg_pass_cols(es, D));
  return fwd_layout(nchunks(B, T, H, BT), BT, D, elem_size(in_dtype),
                    S > 1 ? (size_t)B * H * S : 0, !(flags & kFwdNoARegion),
                    !fused || debug).total;
}

size_t gdn2_fwd_workspace_bytes_ex(int B, int T, int H, int D, int BT, int in_dtype, int flags) {
  if (validate_fwd(B, T, H, D, BT, in_dtype, in_dtype, flags) != GDN2_OK &&
      validate_fwd(B, T, H, D, BT, in_dtype, GDN2_F32, flags) != GDN2_OK)
    return 0;
  return fwd_ws_need(B, T, H, D, BT, in_dtype, flags);
}

size_t gdn2_fwd_workspace_bytes(int B, int T, int H, int D, int BT, int in_dtype) {
  return gdn2_fwd_workspace_bytes_ex(B, T, H, D, BT, in_dtype, 0);
}

}  // extern "C"

namespace gdn2 {
// The forward behind gdn2_fwd, gdn2_fwd_debug and gdn2_fwd_noalloc; `flags` may
// carry kFwdNoARegion here (the public entry points clear it).
int fwd_entry(void* stream, int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
              const void* q, const void* k, const void* v, const void* w, const void* b,
              const void* g, const float* h0, float scale, float* out, float* h_final,
              void* ws, size_t ws_bytes, float* a_dbg, int flags) {
  EventScope scope;
  int rc = validate_fwd(B, T, H, D, BT, in_dtype, g_dtype, flags);
  if (rc) return rc;
  if ((flags & GDN2_FWD_RAW_INPUTS) && (flags & GDN2_FWD_SAVE_A)) return GDN2_ERR_FLAGS;
  if (T > 0 && (rc = check_ptrs({q, k, v, w, b, g, out}))) return rc;
  if ((rc = check_ptrs({h_final}))) return rc;
  if ((rc = check_opt({h0, a_dbg}))) return rc;
  const size_t need = fwd_ws_need(B, T, H, D, BT, in_dtype, flags, a_dbg != nullptr);
  if (need > 0 && (rc = check_ptrs({ws}))) return rc;
  if (ws_bytes < need) return GDN2_ERR_WORKSPACE;
  return dispatch<FwdRun>(in_dtype, g_dtype, BT, D, (hipStream_t)stream, B, T, H, q, k, v, w,
                          b, g, h0, scale, out, h_final, (char*)ws, a_dbg, flags,
                          (const Varlen*)nullptr);
}

// Workspace bytes of the forward for `flags` (kFwdNoARegion included), or 0 for
// shapes the forward rejects.
size_t fwd_workspace_need(int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
                          int flags) {
  if (validate_fwd(B, T, H, D, BT, in_dtype, g_dtype, flags) != GDN2_OK) return 0;
  return fwd_ws_need(B, T, H, D, BT, in_dtype, flags);
}
}  // namespace gdn2

extern "C" {

int gdn2_fwd(void* stream, int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
             const void* q, const void* k, const void* v, const void* w, const void* b,
             const void* g, const float* h0, float scale, float* out, float* h_final,
             void* ws, size_t ws_bytes, int flags) {
  return fwd_entry(stream, B, T, H, D, BT, in_dtype, g_dtype, q, k, v, w, b, g, h0, scale,
                   out, h_final, ws, ws_bytes, nullptr, flags & ~kFwdNoARegion);
}

int gdn2_fwd_debug(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                   int g_dtype, const void* q, const void* k, const void* v, const void* w,
                   const void* b, const void* g, const float* h0, float scale, float* out,
                   float* h_final, void* ws, size_t ws_bytes, float* a_out) {
  if (!a_out && T > 0) return GDN2_ERR_NULL;
  return fwd_entry(stream, B, T, H, D, BT, in_dtype, g_dtype, q, k, v, w, b, g, h0, scale,
                   out, h_final, ws, ws_bytes, a_out, GDN2_FWD_PARTIAL_CHUNK);
}

size_t gdn2_bwd_workspace_bytes(int B, int T, int H, int D, int BT, int in_dtype) {
  if (in_dtype == GDN2_BF16) return 0;
  if (gdn2_validate(B, T, H, D, BT, in_dtype, in_dtype) != GDN2_OK &&
      gdn2_validate(B, T, H, D, BT, in_dtype, GDN2_F32) != GDN2_OK)
    return 0;
  return bwd_ws_bytes(nchunks(B, T, H, BT), BT, D, elem_size(in_dtype));
}

int gdn2_bwd(void* stream, int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
             const void* q, const void* k, const void* v, const void* w, const void* b,
             const void* g, const float* h0, float scale, const float* dout,
             const float* dh_final, void* dq, void* dk, void* dv, void* dw, void* db, void* dg,
             float* dh0, const void* fwd_ws, size_t fwd_ws_bytes, void* ws,
             size_t ws_bytes) {
  EventScope scope;
  int rc = gdn2_validate(B, T, H, D, BT, in_dtype, g_dtype);
  if (rc) return rc;
  if (in_dtype == GDN2_BF16) return GDN2_ERR_DTYPE;  // bfloat16 residuals: see gdn2.h
  if (T > 0 && (rc = check_ptrs({q, k, v, w, b, g, dout, dq, dk, dv, dw, db, dg}))) return rc;
  if ((rc = check_ptrs({dh0}))) return rc;
  if ((rc = check_opt({h0, dh_final}))) return rc;
  if (BT != 64) return GDN2_ERR_CHUNK;  // the backward kernels tile 64-token chunks
  const size_t nc = nchunks(B, T, H, BT);
  const size_t fneed = fwd_layout(nc, BT, D, elem_size(in_dtype)).total;
  const size_t bneed = bwd_ws_bytes(nc, BT, D, elem_size(in_dtype));
  if (fneed > 0 && (rc = check_ptrs({fwd_ws}))) return rc;
  if (bneed > 0 && (rc = check_ptrs({ws}))) return rc;
  if (fwd_ws_bytes < fneed || ws_bytes < bneed) return GDN2_ERR_WORKSPACE;
  return dispatch<BwdRun>(in_dtype, g_dtype, BT, D, (hipStream_t)stream, B, T, H, q, k, v, w,
                          b, g, h0, scale, dout, dh_final, dq, dk, dv, dw, db, dg, dh0,
                          (const char*)fwd_ws, (char*)ws, (const int*)nullptr, 0);
}

size_t gdn2_bwd_varlen_workspace_bytes(int total_chunks, int H, int D, int BT, int in_dtype) {
  if (total_chunks < 0 || (double)total_chunks * BT > 2.0e9) return 0;
  return gdn2_bwd_workspace_bytes(1, total_chunks * BT, H, D, BT, in_dtype);
}

int gdn2_bwd_varlen(void* stream, int num_seqs, const int* cu_chunks, int total_chunks, int H,
                    int D, int BT, int in_dtype, int g_dtype, const void* q, const void* k,
                    const void* v, const void* w, const void* b, const void* g, const float* h0,
                    float scale, const float* dout, const float* dh_final, void* dq, void* dk,
                    void* dv, void* dw, void* db, void* dg, float* dh0, const void* fwd_ws,
                    size_t fwd_ws_bytes, void* ws, size_t ws_bytes) {
  EventScope scope;
  if (num_seqs < 1 || total_chunks < 0 || (double)total_chunks * BT > 2.0e9 ||
      (double)num_seqs * H * (D / 16) > 2147483647.0)
    return GDN2_ERR_SHAPE;
  const int T = total_chunks * BT;
  int rc = gdn2_validate(1, T, H, D, BT, in_dtype, g_dtype);
  if (rc) return rc;
  if (in_dtype == GDN2_BF16) return GDN2_ERR_DTYPE;  // bfloat16 residuals: see gdn2.h
  if (BT != 64) return GDN2_ERR_CHUNK;
  if (T > 0 && (rc = check_ptrs({q, k, v, w, b, g, dout, dq, dk, dv, dw, db, dg}))) return rc;
  if ((rc = check_ptrs({dh0, cu_chunks}))) return rc;
  if ((rc = check_opt({h0, dh_final}))) return rc;
  const size_t nc = nchunks(1, T, H, BT);
  const size_t fneed = fwd_layout(nc, BT, D, elem_size(in_dtype)).total;
  const size_t bneed = bwd_ws_bytes(nc, BT, D, elem_size(in_dtype));
  if (fneed > 0 && (rc = check_ptrs({fwd_ws}))) return rc;
  if (bneed > 0 && (rc = check_ptrs({ws}))) return rc;
  if (fwd_ws_bytes < fneed || ws_bytes < bneed) return GDN2_ERR_WORKSPACE;
  return dispatch<BwdRun>(in_dtype, g_dtype, BT, D, (hipStream_t)stream, 1, T, H, q, k, v, w,
                          b, g, h0, scale, dout, dh_final, dq, dk, dv, dw, db, dg, dh0,
                          (const char*)fwd_ws, (char*)ws, cu_chunks, num_seqs);
}

size_t gdn2_fwd_varlen_workspace_bytes(int total_chunks, int H, int D, int BT, int in_dtype) {
  if (total_chunks < 0 || (double)total_chunks * BT > 2.0e9) return 0;
  if (gdn2_validate(1, total_chunks * BT, H, D, BT, in_dtype, GDN2_F32) != GDN2_OK) return 0;
  return fwd_layout((size_t)H * total_chunks, BT, D, elem_size(in_dtype)).total;
}

int gdn2_fwd_varlen(void* stream, int num_seqs, const int* cu_chunks, const int* chunk_start,
                    int total_chunks, int T, int H, int D, int BT, int in_dtype, int g_dtype,
                    const void* q, const void* k, const void* v, const void* w, const void* b,
                    const void* g, const float* h0, float scale, float* out, float* h_final,
                    void* ws, size_t ws_bytes, int flags) {
  EventScope scope;
  if (num_seqs < 1 || total_chunks < 0 || T < 0 || T > total_chunks * (long long)BT ||
      (double)total_chunks * BT > 2.0e9 || (double)num_seqs * H * (D / 16) > 2147483647.0)
    return GDN2_ERR_SHAPE;
  if (T < total_chunks) return GDN2_ERR_SEQ_LEN;  // every chunk holds at least one token
  int rc = gdn2_validate(1, BT > 0 ? total_chunks * BT : 0, H, D, BT, in_dtype, g_dtype);
  if (rc) return rc;
  if ((flags & GDN2_FWD_SAVE_A) && (flags & GDN2_FWD_RAW_INPUTS)) return GDN2_ERR_FLAGS;
  if (T > 0 && (rc = check_ptrs({q, k, v, w, b, g, out}))) return rc;
  if ((rc = check_ptrs({h_final, cu_chunks}))) return rc;
  if (total_chunks > 0 && (rc = check_ptrs({chunk_start}))) return rc;
  if ((rc = check_opt({h0}))) return rc;
  const size_t need = gdn2_fwd_varlen_workspace_bytes(total_chunks, H, D, BT, in_dtype);
  if (need > 0 && (rc = check_ptrs({ws}))) return rc;
  if (ws_bytes < need) return GDN2_ERR_WORKSPACE;
  const Varlen vl{cu_chunks, chunk_start, num_seqs, total_chunks};
  return dispatch<FwdRun>(in_dtype, g_dtype, BT, D, (hipStream_t)stream, 1, T, H, q, k, v, w,
                          b, g, h0, scale, out, h_final, (char*)ws, (float*)nullptr,
                          flags & (GDN2_FWD_RAW_INPUTS | GDN2_FWD_SAVE_A), &vl);
}

int gdn2_chunk_scores(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                      int g_dtype, const void* q, const void* k, const void* b,
                      const void* g, float scale, float* aqk, float* akk) {
  EventScope scope;
  int rc = validate_stage(B, T, H, D, BT, in_dtype, g_dtype);
  if (rc) return rc;
  if (T == 0) return GDN2_OK;   // no chunks
  if ((rc = check_ptrs({q, k, b, g, aqk, akk}))) return rc;
  return dispatch_stage<ScoresRun>(in_dtype, g_dtype, D, (hipStream_t)stream, B, T, H, q, k, b,
                                   g, scale, aqk, akk);
}

int gdn2_wy_solve(void* stream, long long nchunks, int BT, const float* akk, float* a) {
  EventScope scope;
  if (BT != 64) return GDN2_ERR_CHUNK;
  if (nchunks < 0 || nchunks > 0x7fffffffLL) return GDN2_ERR_SHAPE;
  if (nchunks == 0) return GDN2_OK;
  int rc = check_ptrs({akk, a});
  if (rc) return rc;
  return launch_stage_solve((hipStream_t)stream, (size_t)nchunks, akk, a) == hipSuccess
             ? GDN2_OK
             : GDN2_ERR_LAUNCH;
}

int gdn2_recompute_wy(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                      int g_dtype, const void* q, const void* k, const void* v,
                      const void* w, const void* b, const void* g, const float* a,
                      float* w_pseudo, float* u, float* kg, float* qg, float* gc_last) {
  EventScope scope;
  int rc = validate_stage(B, T, H, D, BT, in_dtype, g_dtype);
  if (rc) return rc;
  if (T == 0) return GDN2_OK;   // no chunks
  if ((rc = check_ptrs({q, k, v, w, b, g, a, w_pseudo, u, kg, qg, gc_last}))) return rc;
  return dispatch_stage<WyRun>(in_dtype, g_dtype, D, (hipStream_t)stream, B, T, H, q, k, v, w,
                               b, g, a, w_pseudo, u, kg, qg, gc_last);
}

// gdn2_chunk_combine's shape checks: N chunks of 64 tokens, and the transposes
// of the D x D state tiles (one workgroup per 32 x 32 tile) within a 31-bit grid.
static int validate_combine(int B, int N, int H, int D, int BT) {
  if (N < 0 || (long long)N * 64 > 0x7fffffffLL) return GDN2_ERR_SHAPE;
  const int rc = validate_stage(B, N * 64, H, D, BT, GDN2_F32, GDN2_F32);
  if (rc) return rc;
  if ((double)B * H * N * (D / 32) * (D / 32) > 2147483647.0) return GDN2_ERR_SHAPE;
  return GDN2_OK;
}

size_t gdn2_chunk_combine_workspace_bytes(int B, int N, int H, int D, int BT) {
  if (validate_combine(B, N, H, D, BT) != GDN2_OK) return 0;
  return combine_layout(nchunks(B, N * 64, H, 64), 64, D).total;
}

int gdn2_chunk_combine(void* stream, int B, int N, int H, int D, int BT, const float* aqk,
                       const float* w_pseudo, const float* u, const float* kg,
                       const float* qg, const float* gc_last, const float* h0, float scale,
                       float* out, float* h_final, float* h_pre_all, float* v_new_all,
                       void* ws, size_t ws_bytes) {
  EventScope scope;
  int rc = validate_combine(B, N, H, D, BT);
  if (rc) return rc;
  if (N > 0 && (rc = check_ptrs({aqk, w_pseudo, u, kg, qg, gc_last, out}))) return rc;
  if ((rc = check_ptrs({h_final}))) return rc;
  if ((rc = check_opt({h0, h_pre_all, v_new_all}))) return rc;
  const size_t need = combine_layout(nchunks(B, N * 64, H, 64), 64, D).total;
  if (need > 0 && (rc = check_ptrs({ws}))) return rc;
  if (ws_bytes < need) return GDN2_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (D == 64)
    e = launch_stage_combine<64>(st, B, N, H, aqk, w_pseudo, u, kg, qg, gc_last, h0, scale, out,
                                 h_final, h_pre_all, v_new_all, (char*)ws);
  else if (D == 128)
    e = launch_stage_combine<128>(st, B, N, H, aqk, w_pseudo, u, kg, qg, gc_last, h0, scale, out,
                                  h_final, h_pre_all, v_new_all, (char*)ws);
  else
    e = launch_stage_combine<256>(st, B, N, H, aqk, w_pseudo, u, kg, qg, gc_last, h0, scale, out,
                                  h_final, h_pre_all, v_new_all, (char*)ws);
  return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

// ---- backward stages ------------------------------------------------------------
// Shapes of the backward stage entry points: those of gdn2_chunk_combine (float32,
// chunk 64, N chunks of 64 tokens per sequence, the D x D tile transposes within
// a 31-bit grid, the largest of their grids).
static int validate_bstage(int B, int N, int H, int D, int BT) {
  return validate_combine(B, N, H, D, BT);
}

// Dispatch of a backward stage launcher on D.
#define GDN2_BSTAGE_CALL(fn, ...)                                   \
  (D == 64 ? fn<64>(__VA_ARGS__) : D == 128 ? fn<128>(__VA_ARGS__) \
                                            : fn<256>(__VA_ARGS__))

size_t gdn2_bwd_stage_workspace_bytes(int stage, int B, int N, int H, int D, int BT) {
  if (validate_bstage(B, N, H, D, BT) != GDN2_OK) return 0;
  size_t need = 0;
  hipStream_t st = nullptr;
  switch (stage) {
    case GDN2_STAGE_DHU:
      GDN2_BSTAGE_CALL(launch_stage_dhu, st, B, N, H, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, 1.f, nullptr, nullptr, nullptr, nullptr, nullptr,
                       &need);
      break;
    case GDN2_STAGE_DAV:
      GDN2_BSTAGE_CALL(launch_stage_dav, st, B, N, H, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, &need);
      break;
    case GDN2_STAGE_WY:
      GDN2_BSTAGE_CALL(launch_stage_wy_dqkg, st, B, N, H, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                       1.f, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                       nullptr, &need);
      break;
    case GDN2_STAGE_INTRA:
      GDN2_BSTAGE_CALL(launch_stage_intra, st, B, N * 64, H, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, 1.f, nullptr, nullptr, nullptr, nullptr, nullptr,
                       &need);
      break;
    default:
      return 0;
  }
  return need;
}

// The workspace check shared by the backward stage entry points.
static int check_bstage_ws(int stage, int B, int N, int H, int D, int BT, const void* ws,
                           size_t ws_bytes) {
  const size_t need = gdn2_bwd_stage_workspace_bytes(stage, B, N, H, D, BT);
  if (need > 0 && !ws) return GDN2_ERR_NULL;
  if (need > 0 && ((uintptr_t)ws & 15u)) return GDN2_ERR_ALIGN;
  return ws_bytes < need ? GDN2_ERR_WORKSPACE : GDN2_OK;
}

int gdn2_bwd_dhu(void* stream, int B, int N, int H, int D, int BT, const float* dout,
                 const float* dv_partial, const float* w_pseudo, const float* qg,
                 const float* kg, const float* gc_last, float scale, const float* dht,
                 float* dh_all, float* dh0, float* dv_all, void* ws, size_t ws_bytes) {
  EventScope scope;
  int rc = validate_bstage(B, N, H, D, BT);
  if (rc) return rc;
  if (N > 0 && (rc = check_ptrs({dout, dv_partial, w_pseudo, qg, kg, gc_last, dh_all, dv_all})))
    return rc;
  if ((rc = check_ptrs({dh0}))) return rc;
  if ((rc = check_opt({dht}))) return rc;
  if ((rc = check_bstage_ws(GDN2_STAGE_DHU, B, N, H, D, BT, ws, ws_bytes))) return rc;
  size_t unused = 0;
  const hipError_t e = GDN2_BSTAGE_CALL(launch_stage_dhu, (hipStream_t)stream, B, N, H, dout,
                                        dv_partial, w_pseudo, qg, kg, gc_last, scale, dht,
                                        dh_all, dh0, dv_all, (char*)ws, &unused);
  return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_bwd_dav(void* stream, int B, int N, int H, int D, int BT, const float* aqk,
                 const float* v_new, const float* dout, float* daqk, float* dv_new, void* ws,
                 size_t ws_bytes) {
  EventScope scope;
  int rc = validate_bstage(B, N, H, D, BT);
  if (rc) return rc;
  if (N == 0) return GDN2_OK;
  if ((rc = check_ptrs({aqk, v_new, dout, daqk, dv_new}))) return rc;
  if ((rc = check_bstage_ws(GDN2_STAGE_DAV, B, N, H, D, BT, ws, ws_bytes))) return rc;
  size_t unused = 0;
  const hipError_t e = GDN2_BSTAGE_CALL(launch_stage_dav, (hipStream_t)stream, B, N, H, aqk,
                                        v_new, dout, daqk, dv_new, (char*)ws, &unused);
  return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_bwd_wy_dqkg(void* stream, int B, int N, int H, int D, int BT, const float* q,
                     const float* k, const float* b, const float* w, const float* v,
                     const float* gc, const float* a, const float* h_pre_all,
                     const float* v_new_all, const float* dout, const float* dv,
                     const float* dh_next_all, float scale, float* dq, float* dk, float* db,
                     float* dw, float* dv_raw, float* dgc, float* dakk, void* ws,
                     size_t ws_bytes) {
  EventScope scope;
  int rc = validate_bstage(B, N, H, D, BT);
  if (rc) return rc;
  if (N == 0) return GDN2_OK;
  if ((rc = check_ptrs({q, k, b, w, v, gc, a, h_pre_all, v_new_all, dout, dv, dh_next_all})))
    return rc;
  if ((rc = check_ptrs({dq, dk, db, dw, dv_raw, dgc, dakk}))) return rc;
  if ((rc = check_bstage_ws(GDN2_STAGE_WY, B, N, H, D, BT, ws, ws_bytes))) return rc;
  size_t unused = 0;
  const hipError_t e = GDN2_BSTAGE_CALL(
      launch_stage_wy_dqkg, (hipStream_t)stream, B, N, H, q, k, b, w, v, gc, a, h_pre_all,
      v_new_all, dout, dv, dh_next_all, scale, dq, dk, db, dw, dv_raw, dgc, dakk, (char*)ws,
      &unused);
  return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_bwd_intra(void* stream, int B, int T, int H, int D, int BT, const float* daqk,
                   const float* dakk, const float* q, const float* k, const float* b,
                   const float* g, float scale, float* dq, float* dk, float* db, float* dgc,
                   void* ws, size_t ws_bytes) {
  EventScope scope;
  if (T < 0 || BT != 64) return BT != 64 ? GDN2_ERR_CHUNK : GDN2_ERR_SHAPE;
  if (T % 64 != 0) return GDN2_ERR_SEQ_LEN;
  const int N = T / 64;
  int rc = validate_bstage(B, N, H, D, BT);
  if (rc) return rc;
  if (N == 0) return GDN2_OK;
  if ((rc = check_ptrs({daqk, dakk, q, k, b, g, dq, dk, db, dgc}))) return rc;
  if ((rc = check_bstage_ws(GDN2_STAGE_INTRA, B, N, H, D, BT, ws, ws_bytes))) return rc;
  size_t unused = 0;
  const hipError_t e = GDN2_BSTAGE_CALL(launch_stage_intra, (hipStream_t)stream, B, T, H, daqk,
                                        dakk, q, k, b, g, scale, dq, dk, db, dgc, (char*)ws,
                                        &unused);
  return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_bwd_reverse_cumsum(void* stream, long long tiles, int BT, int D, const float* dgc,
                            float* dg) {
  EventScope scope;
  if (tiles < 0 || BT < 1 || D < 1 || BT > 4096 || D > 65536) return GDN2_ERR_SHAPE;
  if ((double)tiles * BT * D > 9.0e15) return GDN2_ERR_SHAPE;
  if (tiles == 0) return GDN2_OK;
  if (!dgc || !dg) return GDN2_ERR_NULL;
  if (((uintptr_t)dgc & 3u) || ((uintptr_t)dg & 3u)) return GDN2_ERR_ALIGN;
  reverse_cumsum((hipStream_t)stream, dgc, dg, (size_t)tiles, BT, D);
  return hipGetLastError() == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}
#undef GDN2_BSTAGE_CALL

int gdn2_decode(void* stream, int B, int H, int D, int in_dtype, int g_dtype, const void* q,
                const void* k, const void* v, const void* w, const void* b, const void* g,
                float scale, const float* h_in, float* h_out, float* out) {
  EventScope scope;
  int rc = gdn2_validate(B, 0, H, D, 64, in_dtype, g_dtype);
  if (rc) return rc;
  if ((rc = check_ptrs({q, k, v, w, b, g, h_out, out}))) return rc;
  if ((rc = check_opt({h_in}))) return rc;
  hipStream_t st = (hipStream_t)stream;
#define GDN2_DEC(T, TG, D_) \
  if (D == D_) return run_decode<T, TG, D_>(st, B, H, q, k, v, w, b, g, scale, h_in, h_out, out);
  if (in_dtype == GDN2_F32) {
    GDN2_DEC(float, float, 64)
    GDN2_DEC(float, float, 128)
    GDN2_DEC(float, float, 256)
  } else if (g_dtype == GDN2_F32) {   // GDN2_BF16 or GDN2_BF16_F32: the step is float32
    GDN2_DEC(bf16_t, float, 64)
    GDN2_DEC(bf16_t, float, 128)
    GDN2_DEC(bf16_t, float, 256)
  } else {
    GDN2_DEC(bf16_t, bf16_t, 64)
    GDN2_DEC(bf16_t, bf16_t, 128)
    GDN2_DEC(bf16_t, bf16_t, 256)
  }
#undef GDN2_DEC
  return GDN2_ERR_HEAD_DIM;
}

}  // extern "C"
