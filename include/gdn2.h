/*
 * gdn2.h -- C ABI of the MI355X (gfx950) GDN-2 chunked linear-attention library
 * (libgdn2_hip.so).
 *
 * The library replaces the device side of the reference's Python API:
 *   gdn2_pallas_forward(q,k,v,w,b,g,scale,h0=None)          gdn2_fwd.py:400-424
 *   gdn2_pallas_forward_trainable(q,k,v,w,b,g,scale,h0=None) gdn2_pipeline.py:143-159
 * whose forward is kernels A-D (gdn2_fwd.py:142-397) and whose custom_vjp
 * backward is B1-B5 (gdn2_bwd.py:32-375, assembled at gdn2_pipeline.py:70-137).
 *
 * Conventions
 *  - Tensors are dense row-major.  q,k,v,w,b,g,out and all gradients are
 *    (B, T, H, D); states h0, h_final, dh_final, dh0 are (B, H, D, D) indexed
 *    [b][h][dk][dv] (gdn2_fwd.py:342,355-357).  out, h_final, dh0 are float32
 *    (gdn2_fwd.py:163-165,342); gradients come back in the input dtype
 *    (gdn2_pipeline.py:129-135).
 *  - Every pointer is caller-owned device memory, 16-byte aligned.  No entry
 *    point allocates: the caller sizes the workspace with the *_workspace_bytes
 *    functions.  Work is enqueued on `stream` (a hipStream_t; NULL = default
 *    stream) and the call returns without synchronising.
 *  - Return value 0 on success, a negative GDN2_ERR_* code otherwise;
 *    gdn2_strerror() names it.  Invalid shapes are rejected before any launch.
 *  - No mutable global state beyond the per-thread timing request of
 *    gdn2_set_launch_events and the clip bound of gdn2_set_clip: calls on
 *    different streams may run concurrently provided their workspaces do not
 *    overlap.
 */
#ifndef GDN2_H_
#define GDN2_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (in_dtype applies to q,k,v,w,b and the gradients). */
#define GDN2_F32  0
#define GDN2_BF16 1  /* bfloat16 data and bfloat16 MFMA operands (inference) */
/* bfloat16 q,k,v,w,b and gradients, float32 arithmetic, residuals and MFMA
 * operands: the float32 path on bfloat16 inputs, as the reference's training
 * path upcasts every input before any arithmetic (gdn2_fwd.py:100-103,
 * gdn2_bwd.py:130-142) -- without float32 copies of the inputs or gradients.
 * Chunk 64 only; the workspace is sized as for GDN2_F32. */
#define GDN2_BF16_F32 2

/* Error codes. */
#define GDN2_OK                0
#define GDN2_ERR_HEAD_DIM     -1  /* D not in {64,128,256};
                                     ref asserts D==128, gdn2_fwd.py:145, gdn2_bwd.py:348 */
#define GDN2_ERR_SEQ_LEN      -2  /* T % BT != 0; ref asserts, gdn2_fwd.py:146 */
#define GDN2_ERR_CHUNK        -3  /* BT not in {64,128}, or BT=128 with float32 arithmetic or D=256 */
#define GDN2_ERR_DTYPE        -4  /* unknown dtype code; GDN2_BF16 in the backward */
#define GDN2_ERR_NULL         -5  /* required pointer is NULL */
#define GDN2_ERR_ALIGN        -6  /* pointer not 16-byte aligned */
#define GDN2_ERR_WORKSPACE    -7  /* workspace smaller than *_workspace_bytes() */
#define GDN2_ERR_SHAPE        -8  /* B<1, H<1, T<0, or sizes overflow (elements,
                                     or workgroups of a launch past 2^31) */
#define GDN2_ERR_LAUNCH       -9  /* HIP launch failure */
#define GDN2_ERR_FLAGS       -10  /* invalid flag combination */
#define GDN2_ERR_SCRATCH     -11  /* gdn2_fwd_noalloc: workload needs more than its scratch */

/* Library version string, e.g. "0.1.0". */
const char* gdn2_version(void);

/* Static description of an error code (never NULL). */
const char* gdn2_strerror(int code);

/* Host-only shape/dtype check (no GPU needed).  Mirrors the reference's
 * trace-time assertions gdn2_fwd.py:145-146 and gdn2_bwd.py:348-349. */
int gdn2_validate(int B, int T, int H, int D, int BT, int in_dtype, int g_dtype);

/* Bytes of workspace gdn2_fwd needs for an inference call (flags 0).  With
 * GDN2_FWD_SAVE_A (gdn2_fwd_workspace_bytes_ex) the workspace holds the
 * per-chunk residuals (WY factors, chunk states, v_new) that gdn2_bwd reads;
 * after an inference call its contents are unspecified.  Where the state scan
 * forms the outputs itself (bfloat16 inputs at D = 128 and 256, float32 at
 * D = 64), the chunk states and v_new never leave the GPU's on-chip memory and
 * the inference workspace has no room for them. */
size_t gdn2_fwd_workspace_bytes(int B, int T, int H, int D, int BT, int in_dtype);

/* gdn2_fwd flags. */
#define GDN2_FWD_SAVE_A 1  /* also keep A = (I + Akk)^{-1} in ws, needed by gdn2_bwd */
/* q,k,w,b,g are given before their activations, which the forward applies as it
 * reads them: q,k <- q,k / max(|.|_2, 1e-12) over D, w,b <- sigmoid, g <-
 * -softplus(g) -- the caller's preparation step of BASELINE's input
 * distributions, fused into the forward.  Inference only: not with
 * GDN2_FWD_SAVE_A (the backward reads the activated inputs). */
#define GDN2_FWD_RAW_INPUTS 2
/* Segments of the state scan (bits 8-15; 0 = automatic).  Long sequences with
 * few (b,h) pairs split the serial chunk recurrence into S segments scanned in
 * parallel and chained by their affine transitions (the sequence-parallel
 * design of the reference's kernel D, gdn2_fwd.py:338-366).  The chaining is
 * exact while the +-CLIP clip of the carried state (gdn2_fwd.py:358) does not
 * bind; the segmented passes flag any state clip that binds, and a flagged call
 * reruns the scan serially on the device (no host round trip), so the result
 * is the serial one either way.  n is clamped to [1, T/BT]; a forced count
 * needs gdn2_fwd_workspace_bytes_ex's workspace. */
#define GDN2_FWD_SEGMENTS(n) (((n) & 0xff) << 8)
/* Accept T % BT != 0: the last chunk of each sequence holds T % BT tokens and
 * is padded inside the kernels with neutral tokens (k = q = 0, g = 0; the state
 * passes through them unchanged), so out and h_final equal the forward over the
 * T real tokens.  Without this flag T % BT != 0 is GDN2_ERR_SEQ_LEN, as the
 * reference asserts (gdn2_fwd.py:146).  gdn2_fwd_workspace_bytes_ex with the
 * same flag sizes the workspace.  Not for gdn2_bwd (its inputs are whole
 * chunks: a caller pads with zero tokens, which leaves every result unchanged). */
#define GDN2_FWD_PARTIAL_CHUNK 4

/* As gdn2_fwd_workspace_bytes, for the segment count `flags` selects.  No
 * counterpart in the reference (its scan is serial); used to force a count. */
size_t gdn2_fwd_workspace_bytes_ex(int B, int T, int H, int D, int BT, int in_dtype, int flags);

/* Forward: replaces gdn2_pallas_forward (gdn2_fwd.py:400-424), kernels A-D.
 * h0 may be NULL (zero initial state, gdn2_fwd.py:403-404).  out (B,T,H,D)
 * and h_final (B,H,D,D) are float32.  flags: 0 for inference, GDN2_FWD_SAVE_A
 * when gdn2_bwd will consume ws (the trainable forward, gdn2_pipeline.py:64-67).
 * Inference with bfloat16 inputs at D = 128 and 256 (and float32 at D = 64)
 * runs two kernels: the state scan forms the outputs itself. */
int gdn2_fwd(void* stream, int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
             const void* q, const void* k, const void* v, const void* w, const void* b,
             const void* g, const float* h0, float scale, float* out, float* h_final,
             void* ws, size_t ws_bytes, int flags);

/* Test hook: as gdn2_fwd, and additionally writes A = (I + Akk)^{-1}
 * (kernel B's output, gdn2_fwd.py:246-260) as float32 (B,H,N,BT,BT) to a_out.
 * The workspace keeps every residual tile (h_c and v_new included), so it
 * takes gdn2_fwd_workspace_bytes_ex(..., GDN2_FWD_SAVE_A) bytes (or
 * GDN2_FWD_SAVE_A | GDN2_FWD_PARTIAL_CHUNK when T % BT != 0). */
int gdn2_fwd_debug(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                   int g_dtype, const void* q, const void* k, const void* v,
                   const void* w, const void* b, const void* g, const float* h0,
                   float scale, float* out, float* h_final, void* ws, size_t ws_bytes,
                   float* a_out);

/* Timing hook.  For the next gdn2_fwd / gdn2_fwd_debug / gdn2_bwd call made
 * on the calling host thread, record events[0] (hipEvent_t) on the call's
 * stream before its first kernel and events[i] after its i-th kernel stage,
 * for i < n.  The request is consumed by that call (also when it fails).
 * gdn2_fwd has 3 stages (fwd_prep, the state scan, fwd_out); where the scan
 * forms the outputs the third stage launches nothing.  Returns 0. */
int gdn2_set_launch_events(void* const* events, int n);

/* Saturation bound of every stage sanitize (x -> clip(nan_to_num(x)) to
 * [-clip, clip]), the reference's module constant CLIP (gdn2_fwd.py:33, 1e4 by
 * default), which its README overrides after import (README.md:87-92), for
 * every kernel this library launches on the current device from now on.
 * Synchronous (a copy into constant memory): call it with none of this
 * library's work in flight on the device and outside graph capture.  Returns
 * GDN2_ERR_SHAPE for a bound that is not finite and positive. */
int gdn2_set_clip(float clip);

/* Bytes of workspace gdn2_bwd needs in addition to the forward workspace. */
size_t gdn2_bwd_workspace_bytes(int B, int T, int H, int D, int BT, int in_dtype);

/* Backward: replaces _gdn2_core_bwd (gdn2_pipeline.py:70-137), kernels B1-B5.
 * fwd_ws must hold the residuals of a gdn2_fwd call with GDN2_FWD_SAVE_A on
 * the same inputs, h0 and scale (the reference recomputes them,
 * gdn2_pipeline.py:77-83; a caller that kept no residuals re-runs gdn2_fwd
 * first).  BT must be 64.  dh_final and h0 may be NULL (zero).  dq,dk,dv,dw,db
 * are in_dtype, dg is g_dtype, dh0 is float32 (B,H,D,D); all gradients are
 * sanitized as gdn2_pipeline.py:129-135.  in_dtype is GDN2_F32 or GDN2_BF16_F32:
 * the arithmetic and the residuals in fwd_ws are float32, as the reference
 * upcasts every input before any arithmetic (gdn2_fwd.py:100-103,
 * gdn2_bwd.py:130-142; gdn2_pipeline.py:129-135); GDN2_BF16_F32 reads bfloat16
 * inputs and writes bfloat16 gradients.  in_dtype = GDN2_BF16 (bfloat16
 * residuals, whose rounding puts gradients contracted against a unit dh_final
 * outside the bfloat16 tolerance) is GDN2_ERR_DTYPE, and
 * gdn2_bwd_workspace_bytes returns 0 for it.
 * Launches 4 kernels at D <= 128 (see gdn2_set_launch_events); at D = 256 the
 * per-chunk products run as separate launches (the launch marks still bracket
 * the same four stages). */
int gdn2_bwd(void* stream, int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
             const void* q, const void* k, const void* v, const void* w, const void* b,
             const void* g, const float* h0, float scale, const float* dout,
             const float* dh_final, void* dq, void* dk, void* dv, void* dw, void* db,
             void* dg, float* dh0, const void* fwd_ws, size_t fwd_ws_bytes, void* ws,
             size_t ws_bytes);

/* Variable-length batch.  No reference counterpart: the reference takes
 * equal-length sequences with T % BT == 0 (gdn2_fwd.py:145-146).  num_seqs
 * sequences are packed along T in (1,T,H,D) inputs; each is chunked on its
 * own -- its last chunk may be short and is padded inside the kernels with
 * neutral tokens -- and scanned from its own h0[s] ((num_seqs,H,D,D), may be
 * NULL) to h_final[s] ((num_seqs,H,D,D)).  Device tables (int32):
 * cu_chunks[num_seqs+1], sequence s owning chunks [cu_chunks[s],
 * cu_chunks[s+1]) of the packed chunk list; chunk_start[total_chunks+1], the
 * first token row of each chunk, chunk_start[total_chunks] = T.  Table values
 * are clamped in the kernels (no access outside the buffers).  flags: 0,
 * GDN2_FWD_RAW_INPUTS, or GDN2_FWD_SAVE_A when gdn2_bwd_varlen will consume ws. */
size_t gdn2_fwd_varlen_workspace_bytes(int total_chunks, int H, int D, int BT, int in_dtype);
int gdn2_fwd_varlen(void* stream, int num_seqs, const int* cu_chunks, const int* chunk_start,
                    int total_chunks, int T, int H, int D, int BT, int in_dtype, int g_dtype,
                    const void* q, const void* k, const void* v, const void* w, const void* b,
                    const void* g, const float* h0, float scale, float* out, float* h_final,
                    void* ws, size_t ws_bytes, int flags);

/* Backward of a variable-length batch.  No reference counterpart (see
 * gdn2_fwd_varlen).  Every sequence must occupy whole chunks: the packed
 * inputs are (1, total_chunks*BT, H, D), sequence s owning chunks
 * [cu_chunks[s], cu_chunks[s+1]); a caller pads each sequence with zero tokens
 * (neutral: its results and gradients are unchanged).  fwd_ws holds the
 * residuals of gdn2_fwd_varlen with GDN2_FWD_SAVE_A on the same inputs, with
 * chunk_start[c] = c*BT.  dh_final and dh0 are (num_seqs,H,D,D) float32
 * (dh_final may be NULL); gradients as gdn2_bwd.  BT must be 64. */
size_t gdn2_bwd_varlen_workspace_bytes(int total_chunks, int H, int D, int BT, int in_dtype);
int gdn2_bwd_varlen(void* stream, int num_seqs, const int* cu_chunks, int total_chunks, int H,
                    int D, int BT, int in_dtype, int g_dtype, const void* q, const void* k,
                    const void* v, const void* w, const void* b, const void* g, const float* h0,
                    float scale, const float* dout, const float* dh_final, void* dq, void* dk,
                    void* dv, void* dw, void* db, void* dg, float* dh0, const void* fwd_ws,
                    size_t fwd_ws_bytes, void* ws, size_t ws_bytes);

/* Forward that allocates nothing: gdn2_fwd's kernels with the workspace in a
 * fixed device array of the library (GDN2_NOALLOC_SCRATCH_BYTES per GPU, held
 * until the process ends).  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Arguments as gdn2_fwd
 * without ws / ws_bytes; flags: GDN2_FWD_RAW_INPUTS, GDN2_FWD_PARTIAL_CHUNK,
 * GDN2_FWD_SEGMENTS(n) -- GDN2_FWD_SAVE_A is GDN2_ERR_FLAGS (the residuals would
 * not survive the next call).  A workload whose inference workspace exceeds the
 * scratch returns GDN2_ERR_SCRATCH before any launch (128 MiB: about 97 k
 * token-heads B*T*H for bfloat16 inputs at chunk 128 and D = 128, e.g.
 * B = 1, T = 8192, H = 11).
 * All calls on one GPU share its scratch: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller. */
#define GDN2_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int gdn2_fwd_noalloc(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                     int g_dtype, const void* q, const void* k, const void* v, const void* w,
                     const void* b, const void* g, const float* h0, float scale, float* out,
                     float* h_final, int flags);

/* Single-token recurrent step on the (B,H,D,D) float32 state, for serving:
 * the reference has no decode entry; this is gdn2_pallas_forward with T = 1
 * (gdn2_fwd.py:400-424), i.e. one chunk of one token, on the state layout of
 * h0 / h_final (gdn2_fwd.py:342).  q,k,v,w,b,g are (B,H,D) (one token of the
 * (B,T,H,D) inputs); h_in may be NULL (zero state) and may equal h_out (update
 * in place); out (B,H,D) float32.  Dtypes as gdn2_fwd; no chunk size applies.
 * One kernel (see gdn2_set_launch_events). */
int gdn2_decode(void* stream, int B, int H, int D, int in_dtype, int g_dtype, const void* q,
                const void* k, const void* v, const void* w, const void* b, const void* g,
                float scale, const float* h_in, float* h_out, float* out);

/* ---- The forward's stages one at a time ------------------------------------
 * The reference's module-level kernels, for callers that run or inspect them
 * separately.  Float32 arithmetic and float32 outputs in the reference's
 * (B,H,N,BT,.) layouts; chunk 64 only (GDN2_ERR_CHUNK otherwise); in_dtype
 * GDN2_F32, or GDN2_BF16 / GDN2_BF16_F32 for bfloat16 inputs (computed in float32,
 * as the reference upcasts, gdn2_fwd.py:100-103,266-272); T % 64 == 0.
 * gdn2_fwd runs the same mathematics fused. */

/* Kernel A: replaces build_chunk_scores_pallas (gdn2_fwd.py:142-170).  q,k,b,g
 * (B,T,H,D); aqk = scale * causal scores, akk = strictly lower (b k) k scores,
 * each (B,H,N,64,64) float32, zero above the diagonal. */
int gdn2_chunk_scores(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                      int g_dtype, const void* q, const void* k, const void* b,
                      const void* g, float scale, float* aqk, float* akk);

/* Kernel B: replaces wy_solve_pallas (gdn2_fwd.py:246-260).  a = (I + akk)^{-1}
 * for nchunks tiles of 64 x 64 float32 ([nchunks][64][64]); only the strictly
 * lower part of akk is read. */
int gdn2_wy_solve(void* stream, long long nchunks, int BT, const float* akk, float* a);

/* Kernel C: replaces recompute_wy_pallas (gdn2_fwd.py:298-330).  Inputs
 * (B,T,H,D) and a given a (B,H,N,64,64); w_pseudo = a (b k e^gc), u = a (w v),
 * kg, qg (B,H,N,64,D) and gc_last (B,H,N,D), float32. */
int gdn2_recompute_wy(void* stream, int B, int T, int H, int D, int BT, int in_dtype,
                      int g_dtype, const void* q, const void* k, const void* v,
                      const void* w, const void* b, const void* g, const float* a,
                      float* w_pseudo, float* u, float* kg, float* qg, float* gc_last);

/* Workspace bytes of gdn2_chunk_combine (N chunks per sequence). */
size_t gdn2_chunk_combine_workspace_bytes(int B, int N, int H, int D, int BT);

/* Kernel D: replaces gdn2_inter_chunk_combine and
 * gdn2_inter_chunk_combine_with_state (gdn2_fwd.py:338-397).  Per-chunk float32
 * tiles as kernels A and C give them: aqk (B,H,N,64,64), w_pseudo, u, kg, qg
 * (B,H,N,64,D), gc_last (B,H,N,D); h0 may be NULL.  out is (B, N*64, H, D) (the
 * token layout of gdn2_fwd; the reference returns it per chunk), h_final
 * (B,H,D,D).  h_pre_all (B,H,N,D,D), the state entering each chunk, and
 * v_new_all (B,H,N,64,D) are written when not NULL. */
int gdn2_chunk_combine(void* stream, int B, int N, int H, int D, int BT, const float* aqk,
                       const float* w_pseudo, const float* u, const float* kg,
                       const float* qg, const float* gc_last, const float* h0, float scale,
                       float* out, float* h_final, float* h_pre_all, float* v_new_all,
                       void* ws, size_t ws_bytes);

/* ---- The backward's stages one at a time -----------------------------------
 * The reference's backward module functions (gdn2_bwd.py:32-342), float32 on
 * the reference's chunk layouts (B,H,N,64,.), chunk 64 (GDN2_ERR_CHUNK
 * otherwise), D in {64, 128, 256}.  Each takes a device workspace of
 * gdn2_bwd_stage_workspace_bytes(stage, ...) bytes for its layout copies (none
 * for the reverse cumsum).  gdn2_bwd runs the same mathematics fused. */
#define GDN2_STAGE_DHU 1   /* gdn2_bwd_dhu */
#define GDN2_STAGE_DAV 2   /* gdn2_bwd_dav */
#define GDN2_STAGE_WY 3    /* gdn2_bwd_wy_dqkg */
#define GDN2_STAGE_INTRA 4 /* gdn2_bwd_intra */
size_t gdn2_bwd_stage_workspace_bytes(int stage, int B, int N, int H, int D, int BT);

/* B1: replaces gdn2_dhu_backward (gdn2_bwd.py:45-80).  do, dv_partial,
 * w_pseudo, qg, kg (B,H,N,64,D), gc_last (B,H,N,D), dht (B,H,D,D) or NULL.
 * dh_all (B,H,N,D,D): the gradient of the state entering each chunk (dh_all[0]
 * = dh0); dh0 (B,H,D,D); dv_all (B,H,N,64,D). */
int gdn2_bwd_dhu(void* stream, int B, int N, int H, int D, int BT, const float* dout,
                 const float* dv_partial, const float* w_pseudo, const float* qg,
                 const float* kg, const float* gc_last, float scale, const float* dht,
                 float* dh_all, float* dh0, float* dv_all, void* ws, size_t ws_bytes);

/* B2: replaces dav_backward_pallas (gdn2_bwd.py:99-122).  aqk (B,H,N,64,64),
 * taken as causal (kernel A's output); v_new, do (B,H,N,64,D).  daqk (B,H,N,64,64),
 * dv_new = aqk^T do (B,H,N,64,D). */
int gdn2_bwd_dav(void* stream, int B, int N, int H, int D, int BT, const float* aqk,
                 const float* v_new, const float* dout, float* daqk, float* dv_new, void* ws,
                 size_t ws_bytes);

/* B3: replaces wy_dqkg_backward_pallas (gdn2_bwd.py:213-244).  q, k, b, w, v,
 * gc (the in-chunk cumsum of g), v_new_all, do, dv (B,H,N,64,D); a (B,H,N,64,64);
 * h_pre_all, dh_next_all (B,H,N,D,D).  dq, dk, db, dw, dv_raw, dgc (B,H,N,64,D),
 * dakk (B,H,N,64,64). */
int gdn2_bwd_wy_dqkg(void* stream, int B, int N, int H, int D, int BT, const float* q,
                     const float* k, const float* b, const float* w, const float* v,
                     const float* gc, const float* a, const float* h_pre_all,
                     const float* v_new_all, const float* dout, const float* dv,
                     const float* dh_next_all, float scale, float* dq, float* dk, float* db,
                     float* dw, float* dv_raw, float* dgc, float* dakk, void* ws,
                     size_t ws_bytes);

/* B4: replaces intra_backward_pallas (gdn2_bwd.py:342-375).  daqk, dakk
 * (B,H,N,64,64); q, k, b, g (B,T,H,D) as the reference takes them.  dq, dk, db,
 * dgc (B,H,N,64,D), the sub-block pair clipping of gdn2_bwd.py:287-328 included. */
int gdn2_bwd_intra(void* stream, int B, int T, int H, int D, int BT, const float* daqk,
                   const float* dakk, const float* q, const float* k, const float* b,
                   const float* g, float scale, float* dq, float* dk, float* db, float* dgc,
                   void* ws, size_t ws_bytes);

/* B5: replaces reverse_cumsum_bwd (gdn2_bwd.py:32-41).  For `tiles` tiles of BT
 * rows by D columns: dg[i] = sanitize(sum_{j >= i} dgc[j]), row-wise. */
int gdn2_bwd_reverse_cumsum(void* stream, long long tiles, int BT, int D, const float* dgc,
                            float* dg);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_H_ */
