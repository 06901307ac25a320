// Layout kernels of the stage entry points (the reference's kernels A-D and
// B1-B5 called one at a time, on the reference's (B,H,N,BT,.) chunk layouts):
// host launchers, defined in gdn2_stage.hip.  All float32, stream-ordered, no
// allocation.
#pragma once

#include <hip/hip_runtime.h>

#include <stddef.h>

namespace gdn2 {

// dst[m][c][r] = src[m][r][c] for n matrices of R x C (R, C multiples of 32).
void transpose_all(hipStream_t st, const float* src, float* dst, size_t n, int R, int C);

// For groups of N matrices of R x C: dst[g][i+1] = src[g][i]^T for i < N-1 (the
// state entering chunk i+1 from the one leaving chunk i); dst[g][0] is left alone.
void transpose_shift(hipStream_t st, const float* src, float* dst, size_t groups, int N, int R,
                     int C);

// Rows of D floats between the chunk layout (B,H,N,BT,D) and the token layout
// (B,N*BT,H,D): to_tokens = true moves chunk rows to token rows.  With `diff`
// (to_tokens only) each chunk's rows are turned from the in-chunk cumsum gc into
// g (row 0 as is, row t the difference gc[t] - gc[t-1]).
void chunk_rows_permute(hipStream_t st, const float* src, float* dst, int B, int H, int N,
                        int BT, int D, bool to_tokens, bool diff);

// B5 (gdn2_bwd.py:32-41): dg[i] = sanitize(sum_{j >= i} dgc[j]) within each of
// `tiles` tiles of BT rows x D columns.
void reverse_cumsum(hipStream_t st, const float* dgc, float* dg, size_t tiles, int BT, int D);

// dst[i] = sanitize(src[i]) for n floats; src == nullptr writes zeros.
void sanitized_copy(hipStream_t st, const float* src, float* dst, size_t n);

// Rows of float32 tiles into the split pair layout of the float32 scans
// (gdn2_common.h): `runs` runs of 32 floats, src == dst allowed (each run is
// read whole before it is written).
void split_runs(hipStream_t st, const float* src, float* dst, size_t runs);

}  // namespace gdn2
