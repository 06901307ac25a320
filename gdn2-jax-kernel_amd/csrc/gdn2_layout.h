// Workspace layout shared by the host API and the kernels.
//
// Every per-chunk tensor is stored chunk-major: chunk id cid = (b*H + h)*N + c,
// then the tile.  Tiles are laid out so that each consumer reads 16-byte rows:
//   W    [cid][BT][D]   T     w_pseudo = A (b k e^gc)        (gdn2_fwd.py:278-279)
//   UT   [cid][D][BT]   f32   u^T, u = A (w v)               (gdn2_fwd.py:280)
//   KgT  [cid][D][BT]   T     kg^T, kg = k e^(gc_last - gc)  (gdn2_fwd.py:285)
//   Qg   [cid][BT][D]   T     qg = q e^gc                    (gdn2_fwd.py:286)
//   Aqk  [cid][BT][BT]  T     intra-chunk scores, lower blocks only (gdn2_fwd.py:127)
//   GL   [cid][D]       f32   gc_last                        (gdn2_fwd.py:284)
//   HT   [cid][D][D]    T     h_c^T: state entering chunk c, [dv][dk] (gdn2_fwd.py:391)
//   VnT  [cid][D][BT]   T     v_new^T                         (gdn2_fwd.py:350)
// T is float for float32 inputs and bfloat16 for bfloat16 inputs.
#pragma once

#include <stddef.h>

namespace gdn2 {

struct FwdLayout {
  size_t W, UT, KgT, Qg, Aqk, GL, HT, VnT, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline FwdLayout fwd_layout(size_t nchunks, int BT, int D, size_t elem) {
  FwdLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
  L.W = take(nchunks * BT * D * elem);
  L.UT = take(nchunks * D * BT * 4);
  L.KgT = take(nchunks * D * BT * elem);
  L.Qg = take(nchunks * BT * D * elem);
  L.Aqk = take(nchunks * BT * BT * elem);
  L.GL = take(nchunks * D * 4);
  L.HT = take(nchunks * D * D * elem);
  L.VnT = take(nchunks * D * BT * elem);
  L.total = off;
  return L;
}

}  // namespace gdn2
