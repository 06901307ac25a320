// Workspace layout shared by the host API and the kernels.
//
// Every per-chunk tensor is stored chunk-major: chunk id cid = (b*H + h)*N + c,
// then the tile.  Tiles are laid out so that each consumer reads 16-byte rows:
//   W    [cid][BT][D]   T     w_pseudo = A (b k e^gc)        (gdn2_fwd.py:278-279)
//   UT   [cid][D][BT]   T     u^T, u = A (w v)               (gdn2_fwd.py:280)
//   KgT  [cid][D][BT]   T     kg^T, kg = k e^(gc_last - gc)  (gdn2_fwd.py:285)
//   Qg   [cid][BT][D]   T     qg = q e^gc                    (gdn2_fwd.py:286)
//   Aqk  [cid][BT][BT]  T     intra-chunk scores, lower blocks only (gdn2_fwd.py:127)
//   GL   [cid][D]       f32   gc_last                        (gdn2_fwd.py:284)
//   HT   [cid][D][D]    T     h_c^T: state entering chunk c, [dv][dk] (gdn2_fwd.py:391)
//   VnT  [cid][D][BT]   T     v_new^T                         (gdn2_fwd.py:350)
//   A    [cid][BT][BT]  f32   (I + Akk)^{-1}, written only for the backward
//                             (GDN2_FWD_SAVE_A)               (gdn2_fwd.py:246-260)
// T is float for float32 inputs and bfloat16 for bfloat16 inputs.  For
// bfloat16 the last dimension of W, UT, KgT, HT and VnT (the index the serial state
// pass contracts over or produces) is stored in chunk order kpos<T>() of
// gdn2_common.h: within each 32-column block, column 16*half + 4*lg + r sits at
// position 8*lg + 4*half + r.  float32 tiles are in natural order.
//
// Backward workspace (all f32, chunk-major, one region per name):
//   DAQK [BT][BT] dAqk (causal)      DVPT [D][BT] (Aqk^T do)^T    QDOT [D][D] (scale qg^T do)^T
//   DHT  [D][D]  dh_{c+1}^T           DVNT [D][BT] dv_new^T
//   DQG, DKG, DKBD [BT][D]            DAKK [BT][BT]
//   SDH  [D]      sum_e dh_{c+1}[d][e] h_c[d][e]
#pragma once

#include <stddef.h>

namespace gdn2 {

struct FwdLayout {
  size_t W, UT, KgT, Qg, Aqk, GL, HT, VnT, A, SEG, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Internal launch flag, never accepted from callers (the public entry points
// clear it): the workspace has no A region, because nothing will read the
// residuals (the no-allocation inference entry point, whose workspace is a
// fixed device array).
constexpr int kFwdNoARegion = 1 << 24;

// SEG (only with a segmented state scan, S > 1): per (b,h) and segment the end
// state from h = 0 and the transition M_seg ([bh][S][2][D][D] f32), then the
// segment entry states ([bh][S][D][D] f32), then the saturation flag (one int32
// in a 256-byte slot, the last of the workspace: set when a clip of the state
// bound in the segmented passes, see seg_flag_offset).  SEG comes last, so the
// offsets the backward reads do not depend on S.  Without `a_region` the A
// tiles take no space, without `states` the HT / VnT tiles (the inference scan
// that forms the outputs itself writes neither); later regions move up.
inline size_t seg_bytes(size_t seg_units, int D) {
  return seg_units ? seg_units * 3 * (size_t)D * D * 4 + 256 : 0;
}
inline FwdLayout fwd_layout(size_t nchunks, int BT, int D, size_t elem, size_t seg_units = 0,
                            bool a_region = true, bool states = true) {
  FwdLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
  L.W = take(nchunks * BT * D * elem);
  L.UT = take(nchunks * D * BT * elem);
  L.KgT = take(nchunks * D * BT * elem);
  L.Qg = take(nchunks * BT * D * elem);
  L.Aqk = take(nchunks * BT * BT * elem);
  L.GL = take(nchunks * D * 4);
  L.HT = take(states ? nchunks * D * D * elem : 0);
  L.VnT = take(states ? nchunks * D * BT * elem : 0);
  L.A = take(a_region ? nchunks * BT * BT * 4 : 0);
  L.SEG = take(seg_bytes(seg_units, D));
  L.total = off;
  return L;
}
// Workspace of the stage entry point gdn2_chunk_combine (float32 tiles): u^T
// and kg^T, the scan's [D][BT] copies of the caller's u and kg, W in the scan's
// split pair layout, and the h^T / v_new^T tiles the scan writes for the output
// pass.
struct CombineLayout {
  size_t UT, KgT, W, HT, VnT, total;
};
inline CombineLayout combine_layout(size_t nchunks, int BT, int D) {
  CombineLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
  L.UT = take(nchunks * D * BT * 4);
  L.KgT = take(nchunks * D * BT * 4);
  L.W = take(nchunks * BT * D * 4);
  L.HT = take(nchunks * (size_t)D * D * 4);
  L.VnT = take(nchunks * D * BT * 4);
  L.total = off;
  return L;
}

// Byte offset of the saturation flag inside SEG (S > 1).
inline size_t seg_flag_offset(size_t seg_units, int D) {
  return seg_units * 3 * (size_t)D * D * 4;
}

// A variable-length batch (B = 1, sequences packed along T): sequence s owns
// chunks [cu_chunks[s], cu_chunks[s+1]) of the packed chunk list, and chunk c
// starts at token row cstart[c] (cstart[total_chunks] = T); a sequence's last
// chunk may be short.  Both tables live in device memory.
struct Varlen {
  const int* cu_chunks;
  const int* cstart;
  int nseq;
  int total_chunks;
};

// Workgroup id -> (unit, part) for kernels that run NS workgroups per unit (a
// chunk's column slices or channel panels), so that a unit's workgroups share an
// XCD and its L2: workgroups are dealt to the 8 XCDs in turn (id mod 8), so ids
// x, x + 8, ..., x + 8 (NS - 1) take the NS parts of one unit.  Whole groups of
// 8 NS ids are mapped that way, the ids past them unit-major.  A bijection from
// [0, nwg) onto [0, nwg / NS) x [0, NS) for nwg a multiple of NS.
struct UnitPart {
  int unit, part;
};
constexpr UnitPart xcd_split(int id, int nwg, int NS) {
  const int full = nwg / (8 * NS) * (8 * NS);
  if (id < full) return UnitPart{(id / 8 / NS) * 8 + id % 8, (id / 8) % NS};
  return UnitPart{id / NS, id % NS};
}

// Table clamps of a variable-length batch.  The kernels read their chunk
// tables through these two functions only, so a malformed table can give wrong
// numbers but never an access outside the buffers.  They are constexpr, which
// makes them callable from device code and from a plain host compiler (the CPU
// test of the clamps compiles this header with g++).
//
// First token row of chunk c and its number of real tokens: from the chunk
// table of a variable-length batch (row0 in [0, T_len), valid in [0, BT] with
// row0 + valid <= T_len; valid = 0 points at row 0), else c*BT within batch
// element bb, with min(BT, T_len - c*BT) real tokens.
struct ChunkRows {
  size_t row0;
  int valid;
};
constexpr ChunkRows chunk_rows(const int* cstart, int c, int bb, int T_len, int BT) {
  if (!cstart) {  // equal sequences of T_len tokens; the last chunk may be short
    const int rest = T_len - c * BT;
    return ChunkRows{(size_t)bb * T_len + (size_t)c * BT, rest < BT ? rest : BT};
  }
  const int r0 = cstart[c];
  if (r0 < 0 || r0 >= T_len) return ChunkRows{0, 0};  // no real rows: point at row 0
  long long v = (long long)cstart[c + 1] - r0;
  v = v < BT ? v : BT;
  v = v < T_len - r0 ? v : T_len - r0;
  if (v <= 0) return ChunkRows{0, 0};
  return ChunkRows{(size_t)r0, (int)v};
}

// Chunks [c0, c0 + n) of sequence s in a list of N chunks, from the sequence
// table cu (cu[s], cu[s+1]) clamped to [0, N].
struct SeqChunks {
  int c0, n;
};
constexpr SeqChunks seq_chunks(const int* cu, int s, int N) {
  int c0 = cu[s];
  c0 = c0 < 0 ? 0 : (c0 > N ? N : c0);
  long long n = (long long)cu[s + 1] - c0;
  n = n < N - c0 ? n : N - c0;
  return SeqChunks{c0, n > 0 ? (int)n : 0};
}

// Columns of a segmented-pass workgroup: 64 for bfloat16 tiles at D >= 128, else 32.
constexpr int seg_pass_cols(int esize, int D) { return esize == 2 && D >= 128 ? 64 : 32; }

// Shape of the forward state-scan variants (fwd_state in gdn2_fwd.hip), here so
// that the host's workspace size follows the same choices.  Tile buffers: two
// when W and kg^T of two chunks fit LDS.  K-split: two compute waves per
// column slice for float32, and for bfloat16 where the W tile holds the
// exchanged partials.
constexpr int state_bufs_of(int esize, int BT, int D) {
  return 4 * BT * D * esize <= 132 * 1024 ? 2 : 1;
}
constexpr int state_ksplit_of(int esize, int BT, int D) {
  return esize == 4 ? 2 : (4 * (BT / 16) * 1024 <= BT * D * 2 ? 2 : 1);
}
// Output waves of the inference scan (32 value columns per workgroup), which
// then forms the outputs itself, or 0 where a separate output pass runs: no
// K-split (bfloat16 at D = 64), a single tile buffer, or more LDS than 160 KB
// (float32 at D >= 128).  The LDS count mirrors fwd_state's arrays.
constexpr int state_out_waves_of(int esize, int BT, int D) {
  const int NW = 2, PADT = 16 / esize;
  const int tiles = 2 * 2 * BT * D * esize;                          // W, kg^T x 2
  const int ub = NW * (esize == 4 ? BT / 16 : BT / 32) * 1024;       // u^T gather
  const int xs = esize == 4 ? 2 * NW * (BT / 16) * 1024 : 0;        // K-split partials
  const int fo = 16 * NW * (D + BT + 2 * PADT) * esize;             // staged h, v_new
  const int lds = tiles + ub + xs + fo + 2 * D * 4 + 256;
  return (state_ksplit_of(esize, BT, D) == 2 && state_bufs_of(esize, BT, D) == 2 &&
          lds <= 160 * 1024) ? BT / 32 : 0;
}

// Segments of the forward state scan for BH (b,h) pairs of N chunks with
// `esize`-byte tiles, whose final pass runs workgroups of `final_cols` value
// columns (seg_pass_cols, or 32 for the inference scan with output waves).
// Automatic choice: as many as fill a 256-CU device in the final pass (BH *
// D/final_cols workgroups per segment), each at least 16 chunks, and only when
// that gives 4 or more (the segmented scan costs about 3/S of the serial chain
// plus a small combine).  `forced` (1..255) overrides it.  The result is
// adjusted so that no segment is empty.  Depends on shapes and flags only, so
// the workspace size is known without a device.
inline int state_segments(long long BH, int N, int D, int esize, int forced, int final_cols) {
  if (N <= 1) return 1;
  long long s;
  if (forced > 0) {
    s = forced;
  } else {
    const long long slices = BH * (D / final_cols);
    s = slices > 0 ? 256 / slices : 1;
    if (s > N / 16) s = N / 16;
    if (s < 4) s = 1;
  }
  if (s > N) s = N;
  if (s < 1) s = 1;
  const long long len = (N + s - 1) / s;
  return (int)((N + len - 1) / (len > 0 ? len : 1));
}

}  // namespace gdn2

namespace gdn2 {

enum BwdBuf {
  B_DAQK, B_DVPT, B_QDOT, B_DHT, B_DVNT, B_DQG, B_DKG, B_DKBD, B_DAKK, B_SDH, B_COUNT
};

struct BwdLayout {
  size_t off[B_COUNT];
  size_t elems[B_COUNT];  // per chunk
  size_t total;
};

inline BwdLayout bwd_layout(size_t nchunks, int BT, int D) {
  BwdLayout L;
  const size_t tt = (size_t)BT * BT, td = (size_t)BT * D, dd = (size_t)D * D;
  const size_t per[B_COUNT] = {tt, td, dd, dd, td, td, td, td, tt, (size_t)D};
  size_t off = 0;
  for (int i = 0; i < B_COUNT; ++i) {
    L.off[i] = off;
    L.elems[i] = per[i];
    off = align256(off + nchunks * per[i] * 4);
  }
  L.total = off;
  return L;
}

}  // namespace gdn2
