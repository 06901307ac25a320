// Host-side checks of libgdn2_hip's C ABI (include/gdn2.h), built without device
// code and run under AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_host_sanitizers.py: shape validation, workspace sizing and every
// rejection that happens before a launch, over a grid of shapes that includes
// the extremes of int.  No call here reaches a kernel launch or the GPU; the
// fake device pointers are never dereferenced.  Exit status 0 when every check
// holds (a sanitizer report aborts the run).
#include <climits>
#include <limits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>

#include "gdn2.h"

static int g_fail = 0;
#define CHECK(cond)                                                        \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
      ++g_fail;                                                            \
    }                                                                      \
  } while (0)

static bool known(int rc) { return rc <= 0 && rc >= GDN2_ERR_SCRATCH; }

int main() {
  const int Bs[] = {INT_MIN, -1, 0, 1, 3, 8, 1 << 20, INT_MAX};
  const int Ts[] = {INT_MIN, -64, -1, 0, 1, 63, 64, 100, 128, 8192, 131072, 1 << 30,
                    INT_MAX - 63, INT_MAX};
  const int Hs[] = {INT_MIN, 0, 1, 6, 1 << 16, INT_MAX};
  const int Ds[] = {-128, 0, 32, 64, 96, 128, 256, 512, INT_MAX};
  const int BTs[] = {INT_MIN, -64, 0, 1, 16, 64, 128, 256, INT_MAX};
  const int DTs[] = {-1, GDN2_F32, GDN2_BF16, GDN2_BF16_F32, 3, INT_MAX};
  const int flag_sets[] = {0, GDN2_FWD_SAVE_A, GDN2_FWD_PARTIAL_CHUNK,
                           GDN2_FWD_PARTIAL_CHUNK | GDN2_FWD_SAVE_A, GDN2_FWD_SEGMENTS(4),
                           GDN2_FWD_SEGMENTS(255) | GDN2_FWD_PARTIAL_CHUNK,
                           GDN2_FWD_RAW_INPUTS, INT_MAX, INT_MIN};
  long n = 0;
  for (int B : Bs)
    for (int T : Ts)
      for (int H : Hs)
        for (int D : Ds)
          for (int BT : BTs)
            for (int dt : DTs)
              for (int gdt : DTs) {
                const int rc = gdn2_validate(B, T, H, D, BT, dt, gdt);
                CHECK(known(rc));
                if (rc == GDN2_OK) {
                  CHECK(B >= 1 && H >= 1 && T >= 0 && T % BT == 0);
                  CHECK(D == 64 || D == 128 || D == 256);
                  CHECK(BT == 64 || (BT == 128 && dt == GDN2_BF16 && D <= 128));
                }
                ++n;
                if (gdt != GDN2_F32) continue;
                // the sizing functions take no g dtype: valid if either g type is
                const bool any_ok = rc == GDN2_OK ||
                                    gdn2_validate(B, T, H, D, BT, dt, dt) == GDN2_OK;
                for (int fl : flag_sets) {
                  const size_t ws = gdn2_fwd_workspace_bytes_ex(B, T, H, D, BT, dt, fl);
                  if (any_ok && T > 0 && !(fl & ~0xffff)) CHECK(ws > 0);
                  if (!any_ok && !(fl & GDN2_FWD_PARTIAL_CHUNK)) CHECK(ws == 0);
                }
                const size_t bws = gdn2_bwd_workspace_bytes(B, T, H, D, BT, dt);
                if (dt == GDN2_BF16) CHECK(bws == 0);
                if (!any_ok) CHECK(bws == 0);
                if (any_ok && T > 0 && dt != GDN2_BF16 && BT == 64) CHECK(bws > 0);
              }
  // grids that would not fit 31 bits are shape errors
  CHECK(gdn2_validate(INT_MAX, 64, INT_MAX, 64, 64, GDN2_F32, GDN2_F32) == GDN2_ERR_SHAPE);
  CHECK(gdn2_validate(1 << 16, 1 << 20, 64, 256, 64, GDN2_F32, GDN2_F32) == GDN2_ERR_SHAPE);
  CHECK(gdn2_validate(8, 8192, 6, 128, 128, GDN2_BF16, GDN2_F32) == GDN2_OK);
  // workspace sizes grow with T and with the kept residuals
  for (int D : {64, 128, 256}) {
    const int BT = 64;
    size_t prev = 0;
    for (int T = 64; T <= (1 << 20); T *= 2) {
      const size_t w = gdn2_fwd_workspace_bytes(2, T, 3, D, BT, GDN2_F32);
      CHECK(w > prev);
      CHECK(gdn2_fwd_workspace_bytes_ex(2, T, 3, D, BT, GDN2_F32, GDN2_FWD_SAVE_A) >= w);
      prev = w;
    }
  }

  // rejections before any launch: fake, aligned, never dereferenced pointers
  auto P = [](uintptr_t a) { return reinterpret_cast<void*>(a); };
  void* x[6];
  for (int i = 0; i < 6; ++i) x[i] = P(0x100000u * (i + 1));
  float* fo = static_cast<float*>(P(0x900000));
  float* fh = static_cast<float*>(P(0xa00000));
  const size_t big = (size_t)1 << 40;
  // shape errors first, then pointers, then the workspace
  CHECK(gdn2_fwd(nullptr, 1, 512, 2, 96, 64, GDN2_F32, GDN2_F32, x[0], x[1], x[2], x[3], x[4],
                 x[5], nullptr, 0.1f, fo, fh, P(0xb00000), big, 0) == GDN2_ERR_HEAD_DIM);
  CHECK(gdn2_fwd(nullptr, 1, 512, 2, 64, 64, GDN2_F32, GDN2_F32, nullptr, x[1], x[2], x[3],
                 x[4], x[5], nullptr, 0.1f, fo, fh, P(0xb00000), big, 0) == GDN2_ERR_NULL);
  CHECK(gdn2_fwd(nullptr, 1, 512, 2, 64, 64, GDN2_F32, GDN2_F32, P(0x100004), x[1], x[2], x[3],
                 x[4], x[5], nullptr, 0.1f, fo, fh, P(0xb00000), big, 0) == GDN2_ERR_ALIGN);
  CHECK(gdn2_fwd(nullptr, 1, 512, 2, 64, 64, GDN2_F32, GDN2_F32, x[0], x[1], x[2], x[3], x[4],
                 x[5], nullptr, 0.1f, fo, fh, P(0xb00000), 16, 0) == GDN2_ERR_WORKSPACE);
  CHECK(gdn2_fwd(nullptr, 1, 512, 2, 64, 64, GDN2_F32, GDN2_F32, x[0], x[1], x[2], x[3], x[4],
                 x[5], nullptr, 0.1f, fo, fh, P(0xb00000), big,
                 GDN2_FWD_RAW_INPUTS | GDN2_FWD_SAVE_A) == GDN2_ERR_FLAGS);
  CHECK(gdn2_fwd(nullptr, 1, INT_MAX, 2, 64, 64, GDN2_F32, GDN2_F32, x[0], x[1], x[2], x[3],
                 x[4], x[5], nullptr, 0.1f, fo, fh, P(0xb00000), big,
                 GDN2_FWD_PARTIAL_CHUNK) != GDN2_OK);
  CHECK(gdn2_fwd_debug(nullptr, 1, 512, 2, 64, 64, GDN2_F32, GDN2_F32, x[0], x[1], x[2], x[3],
                       x[4], x[5], nullptr, 0.1f, fo, fh, P(0xb00000), big,
                       nullptr) == GDN2_ERR_NULL);
  void* g6[6];
  for (int i = 0; i < 6; ++i) g6[i] = P(0xc00000u + 0x10000u * i);
  auto bwd = [&](int D, int BT, int dt, const float* dout, size_t fws, size_t bws) {
    return gdn2_bwd(nullptr, 1, 512, 2, D, BT, dt, GDN2_F32, x[0], x[1], x[2], x[3], x[4], x[5],
                    nullptr, 0.1f, dout, nullptr, g6[0], g6[1], g6[2], g6[3], g6[4], g6[5],
                    fh, P(0xd00000), fws, P(0xe00000), bws);
  };
  const float* dout = static_cast<const float*>(P(0xf00000));
  CHECK(bwd(96, 64, GDN2_F32, dout, big, big) == GDN2_ERR_HEAD_DIM);
  CHECK(bwd(64, 64, GDN2_BF16, dout, big, big) == GDN2_ERR_DTYPE);
  CHECK(bwd(64, 128, GDN2_BF16_F32, dout, big, big) == GDN2_ERR_CHUNK);
  CHECK(bwd(64, 64, GDN2_F32, nullptr, big, big) == GDN2_ERR_NULL);
  CHECK(bwd(64, 64, GDN2_F32, dout, 16, big) == GDN2_ERR_WORKSPACE);
  CHECK(bwd(64, 64, GDN2_F32, dout, big, 16) == GDN2_ERR_WORKSPACE);
  // variable length: bad tables and counts
  const int* cu = static_cast<const int*>(P(0x700000));
  const int* cs = static_cast<const int*>(P(0x710000));
  for (int total : {-1, 0, 4, INT_MAX / 64 + 1, INT_MAX}) {
    for (int nseq : {INT_MIN, 0, 1, 2}) {
      for (int T : {-1, 0, 1, 100, 256, INT_MAX}) {
        const int rc = gdn2_fwd_varlen(nullptr, nseq, cu, cs, total, T, 2, 64, 64, GDN2_F32,
                                       GDN2_F32, x[0], x[1], x[2], x[3], x[4], x[5], nullptr,
                                       0.1f, fo, fh, P(0xb00000), 16, 0);
        CHECK(rc != GDN2_OK && known(rc));
        const int rb = gdn2_bwd_varlen(nullptr, nseq, cu, total, 2, 64, 64, GDN2_F32, GDN2_F32,
                                       x[0], x[1], x[2], x[3], x[4], x[5], nullptr, 0.1f, dout,
                                       nullptr, g6[0], g6[1], g6[2], g6[3], g6[4], g6[5], fh,
                                       P(0xd00000), 16, P(0xe00000), 16);
        CHECK(known(rb) && (total == 0 || rb != GDN2_OK));
      }
    }
    CHECK(gdn2_fwd_varlen_workspace_bytes(total, 2, 64, 64, GDN2_F32) < ((size_t)1 << 50));
    CHECK(gdn2_bwd_varlen_workspace_bytes(total, 2, 64, 64, GDN2_F32) < ((size_t)1 << 50));
  }
  // decode and the no-allocation forward
  CHECK(gdn2_decode(nullptr, 2, 3, 96, GDN2_F32, GDN2_F32, x[0], x[1], x[2], x[3], x[4], x[5],
                    0.1f, nullptr, fh, fo) == GDN2_ERR_HEAD_DIM);
  CHECK(gdn2_decode(nullptr, INT_MAX, INT_MAX, 64, GDN2_F32, GDN2_F32, x[0], x[1], x[2],
                    x[3], x[4], x[5], 0.1f, nullptr, fh, fo) == GDN2_ERR_SHAPE);
  CHECK(gdn2_fwd_noalloc(nullptr, 1, 256, 1, 128, 128, GDN2_BF16, GDN2_F32, x[0], x[1], x[2],
                         x[3], x[4], x[5], nullptr, 0.1f, fo, fh,
                         GDN2_FWD_SAVE_A) == GDN2_ERR_FLAGS);
  CHECK(gdn2_fwd_noalloc(nullptr, 2, 32768, 16, 128, 128, GDN2_BF16, GDN2_F32, x[0], x[1], x[2],
                         x[3], x[4], x[5], nullptr, 0.1f, fo, fh, 0) == GDN2_ERR_SCRATCH);
  // the stage entry points (kernels A-D one at a time): chunk 64 only, shape and
  // dtype rules of the forward, 31-bit grids, then pointers and workspace
  float* fa = static_cast<float*>(P(0x600000));
  for (int B : Bs)
    for (int T : Ts)
      for (int D : Ds)
        for (int BT : {0, 64, 128}) {
          const int rs = gdn2_chunk_scores(nullptr, B, T, 3, D, BT, GDN2_BF16, GDN2_F32, x[0],
                                           x[1], x[4], x[5], 0.1f, fo, fh);
          CHECK(known(rs));
          if (BT != 64) CHECK(rs == GDN2_ERR_CHUNK);
          const int rw = gdn2_recompute_wy(nullptr, B, T, 3, D, BT, GDN2_F32, GDN2_F32, x[0],
                                           x[1], x[2], x[3], x[4], x[5], fa, fo, fo, fo, fo,
                                           fh);
          CHECK(known(rw));
          if (rs == GDN2_OK || rw == GDN2_OK) CHECK(BT == 64 && T % 64 == 0 && B >= 1);
          const int N = T / 64;
          if (N <= 0) continue;   // no chunks: the scan would launch for h_final
          const size_t cws = gdn2_chunk_combine_workspace_bytes(B, N, 3, D, BT);
          const int rc = gdn2_chunk_combine(nullptr, B, N, 3, D, BT, fa, fa, fa, fa, fa, fa,
                                            nullptr, 0.1f, fo, fh, nullptr, nullptr,
                                            P(0xb00000), cws ? cws - 1 : 0);
          CHECK(known(rc) && rc != GDN2_OK);
          if (cws > 0) CHECK(rc == GDN2_ERR_WORKSPACE);
        }
  for (long long nc : {LLONG_MIN, -1LL, 0LL, 5LL, (long long)INT_MAX, (long long)INT_MAX + 1,
                       LLONG_MAX}) {
    const int rc = gdn2_wy_solve(nullptr, nc, 64, fa, fo);
    CHECK(known(rc));
    if (nc < 0 || nc > INT_MAX) CHECK(rc == GDN2_ERR_SHAPE);
    if (nc == 0) CHECK(rc == GDN2_OK);
  }
  CHECK(gdn2_wy_solve(nullptr, 5, 128, fa, fo) == GDN2_ERR_CHUNK);
  CHECK(gdn2_wy_solve(nullptr, 5, 64, nullptr, fo) == GDN2_ERR_NULL);
  // the backward stage entry points (kernels B1-B5 one at a time): workspace sizes
  // stay finite and a workspace one byte short is refused before any launch
  void* wsp = P(0xc00000);
  for (int B : Bs)
    for (int T : Ts)
      for (int D : Ds)
        for (int BT : {0, 64, 128}) {
          const int N = T / 64;
          for (int stage = 0; stage <= 5; ++stage) {
            const size_t need = gdn2_bwd_stage_workspace_bytes(stage, B, N, 3, D, BT);
            CHECK(need < ((size_t)1 << 50));
            if (need > 0) CHECK(stage >= 1 && stage <= 4 && BT == 64 && N >= 1 && B >= 1);
          }
          if (N <= 0) continue;   // B1 with no chunk writes dh0 = sanitize(dht)
          const size_t w1 = gdn2_bwd_stage_workspace_bytes(GDN2_STAGE_DHU, B, N, 3, D, BT);
          int rc = gdn2_bwd_dhu(nullptr, B, N, 3, D, BT, fa, fa, fa, fa, fa, fa, 0.1f, nullptr,
                                fo, fh, fo, wsp, w1 ? w1 - 1 : 0);
          CHECK(known(rc) && rc != GDN2_OK);
          const size_t w2 = gdn2_bwd_stage_workspace_bytes(GDN2_STAGE_DAV, B, N, 3, D, BT);
          rc = gdn2_bwd_dav(nullptr, B, N, 3, D, BT, fa, fa, fa, fo, fo, wsp, w2 ? w2 - 1 : 0);
          CHECK(known(rc) && rc != GDN2_OK);
          const size_t w3 = gdn2_bwd_stage_workspace_bytes(GDN2_STAGE_WY, B, N, 3, D, BT);
          rc = gdn2_bwd_wy_dqkg(nullptr, B, N, 3, D, BT, fa, fa, fa, fa, fa, fa, fa, fa, fa, fa,
                                fa, fa, 0.1f, fo, fo, fo, fo, fo, fo, fo, wsp, w3 ? w3 - 1 : 0);
          CHECK(known(rc) && rc != GDN2_OK);
          const size_t w4 = gdn2_bwd_stage_workspace_bytes(GDN2_STAGE_INTRA, B, N, 3, D, BT);
          rc = gdn2_bwd_intra(nullptr, B, T, 3, D, BT, fa, fa, fa, fa, fa, fa, 0.1f, fo, fo, fo,
                              fo, wsp, w4 ? w4 - 1 : 0);
          CHECK(known(rc) && rc != GDN2_OK);
        }
  for (long long tiles : {LLONG_MIN, -1LL, (long long)INT_MAX, LLONG_MAX})
    for (int bt : {-1, 0, 64, 4097})
      for (int d : {0, 128, INT_MAX}) {
        const int rc = gdn2_bwd_reverse_cumsum(nullptr, tiles, bt, d, fa, fo);
        CHECK(known(rc));
        if (rc == GDN2_OK || rc == GDN2_ERR_LAUNCH)   // only in-range shapes reach a launch
          CHECK(tiles >= 0 && bt >= 1 && bt <= 4096 && d >= 1 && d <= 65536);
      }
  // the clip bound: not finite and positive -> refused before any copy
  for (float c : {0.f, -0.f, -1e4f, std::numeric_limits<float>::quiet_NaN(),
                  std::numeric_limits<float>::infinity(), -std::numeric_limits<float>::infinity(),
                  -std::numeric_limits<float>::denorm_min()})
    CHECK(gdn2_set_clip(c) == GDN2_ERR_SHAPE);
  for (int c = -20; c <= 5; ++c) CHECK(gdn2_strerror(c) != nullptr);
  CHECK(gdn2_set_launch_events(nullptr, -5) == 0);
  std::printf("host checks: %ld shape combinations, %d failures\n", n, g_fail);
  return g_fail ? 1 : 0;
}
