// GDN-2 backward on gfx950 (reference: gdn2_bwd.py B1-B5, assembled by
// gdn2_pipeline.py:70-137).  Everything computes in float32 on
// v_mfma_f32_16x16x4_f32; the chunk size is 64.
//
// Per chunk c with state h = h_c entering it, dh' = dh_{c+1} leaving it
// (kg = k e^{gl-gc}, qg = q e^{gc}, W = A (b k e^{gc}), u = A (w v)):
//   B2   dAqk = (do v_new^T) . causal              Aqk^T do, scale qg^T do   (bwd_b2)
//   B1   dv_new = Aqk^T do + kg dh'                                          (bwd_state,
//        dh = e^{gl} dh' + scale qg^T do - W^T dv_new                         serial)
//   B3   dqg = scale do h^T, dW = -dv_new h^T, dkg = v_new dh'^T,
//        dA = dW (b k e^gc)^T + dv_new (w v)^T, d(bke^gc) = A^T dW, d(wv) = A^T dv_new,
//        dv = d(wv) w, dw = d(wv) v, dAkk = -(A^T dA A^T) . strict             (bwd_wy)
//   B4   gradients of Aqk/Akk wrt q, k, b k, gc, then the chain rule through
//        the exponentials (B3 tail) and the reverse cumsum of dgc (B5)       (gram_bwd)

#include "gdn2_common.h"
#include "gdn2_layout.h"
#include "gdn2_stage.h"

namespace gdn2 {

// ============================================================================
// Operand staging: a stored per-chunk matrix into LDS as float32, all loads
// issued before any LDS store (one memory round trip per operand).
// ============================================================================
struct GMat {
  const void* p;
  int bf16;                 // element type in memory
  int ld;                   // row pitch of the stored matrix
  int mask;                 // on stored (row, col): 1 keep col <= row, 2 keep col < row
  int chained;              // bfloat16 columns stored in chained order (kpos)
};
__device__ __forceinline__ void load4_any(const void* p, int bf16, size_t idx, float* v) {
  if (bf16) {
    const bf16x4 t = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16_t*>(p) + idx);
    v[0] = (float)t[0]; v[1] = (float)t[1]; v[2] = (float)t[2]; v[3] = (float)t[3];
  } else {
    const f32x4 t = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + idx);
    v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
  }
}

// Staging of one operand: the stored matrix (R x Cc, R*Cc <= 128*128) as float4
// runs, all loads issued before any LDS store (one memory round trip per chunk).
// dst (pitch ld) <- S: dst[r][c] = S[r][c], or dst[c][r] when `transposed`.
// (r0, c0) place the tile in the stored matrix for the masks.
// Up to 4096 16-byte runs (64 KB of float32) per call, over NT threads.
struct Staged {
  float v[16][4];
};
// Run i = tid + nt u of a staging loop (tid < nt) exists.  With `ct` it is
// decided at compile time for whole rounds (total constant after inlining), so
// full rounds carry no branch and rounds past the end no code; without it each
// run tests i < total (branches the scheduler does not move loads across).
__device__ __forceinline__ bool run_in(bool ct, int u, int i, int total, int nt) {
  return ct ? (u + 1) * nt <= total || (u * nt < total && i < total) : i < total;
}
template <int NT = 256, bool CT = false>
__device__ __forceinline__ void stage_load(Staged& s, const GMat& m, size_t off, int R, int Cc,
                                           int tid) {
  const int cq = Cc >> 2, total = R * cq;
#pragma unroll
  for (int u = 0; u < 4096 / NT; ++u) {
    const int i = tid + NT * u;
    if (run_in(CT, u, i, total, NT)) {
      const int r = i / cq, c = (i - r * cq) * 4;
      const int sc = m.chained ? kpos<bf16_t>(c) : c;
      load4_any(m.p, m.bf16, off + (size_t)r * m.ld + sc, s.v[u]);
    }
  }
}
template <int NT = 256, bool CT = false>
__device__ __forceinline__ void stage_store(float* dst, int ld, const Staged& s, const GMat& m,
                                            int R, int Cc, int r0, int c0, bool transposed,
                                            int tid) {
  const int cq = Cc >> 2, total = R * cq;
#pragma unroll
  for (int u = 0; u < 4096 / NT; ++u) {
    const int i = tid + NT * u;
    if (run_in(CT, u, i, total, NT)) {
      const int r = i / cq, c = (i - r * cq) * 4;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = s.v[u][e];
        const int gr = r0 + r, gc = c0 + c + e;
        if ((m.mask == 1 && gc > gr) || (m.mask == 2 && gc >= gr)) v[e] = 0.f;
      }
      if (!transposed) {
        *reinterpret_cast<f32x4*>(&dst[r * ld + c]) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(c + e) * ld + r] = v[e];
      }
    }
  }
}

// ============================================================================
// bwd_state (B1): reverse scan over chunks; workgroup = (b,h, 32 value columns of dh).
// ============================================================================
template <typename T>
struct BStateArgs {
  const T* W;        // [cid][BT][D]
  const T* KgT;      // [cid][D][BT]
  const float* GL;   // [cid][D]
  const float* DVPT; // [cid][D][BT]  (Aqk^T do)^T
  const float* QDOT; // [cid][D][D]   (scale qg^T do)^T
  const float* dh_final;  // nullable (B,H,D,D)
  int N;
  float* DHT;        // [cid][D][D]   dh_{c+1}^T
  float* DVNT;       // [cid][D][BT]  dv_new^T
  float* dh0;        // (B,H,D,D)
  const int* cu;     // variable-length batch (B = 1): unit (h, sequence s) scans chunks
                     // [cu[s], cu[s+1]) in reverse; dh_final / dh0 are [s][h][D][D]
  int S, H;          // sequences and heads of a variable-length batch
};

// One workgroup = one (b,h) and 16*NW value columns of dh: NW compute waves (16
// columns each, dh in MFMA accumulators) and NP producer waves, scanning the
// chunks in reverse.  Per chunk (gdn2_bwd.py:45-80):
//   dv_new = dvp + kg dh,   dh <- e^{g_last} dh + scale qg^T do - W^T dv_new.
// As in fwd_state, the producers stream the next chunk (W, kg^T, g_last) into the
// other half of an LDS double buffer with global_load_lds_dwordx4 and gather the
// workgroup's dvp and qg^T do rows into the compute lanes' order (one buffer,
// freed by barrier B once copied to registers); the compute waves issue no
// global loads.  Both products read their tile transposed.  Float32 tiles (in
// the split pair layout of gdn2_common.h, as fwd_prep writes W and kg^T) are
// staged by the producers through registers and stored transposed (W^T, kg),
// still split, so each operand pair is two 16-byte LDS reads and each 32-deep k
// step three bfloat16 MFMAs (the split form; dh and dv_new are split once per
// chunk); bfloat16 tiles move by DMA, one 2-byte LDS read per element (chained
// column order).  The XOR swizzle of the 16-byte chunks keeps either free of
// bank conflicts.
//
// K-split (KS = 2; bfloat16 residuals only up to D = 128, where its registers
// fit), as in fwd_state: two compute waves per
// 16-column slice, each holding half of dh's rows; the halves of kg dh are
// exchanged through LDS (barrier X, after B).  The exchange buffer takes the
// place of the qdot gather: each compute wave then loads its own 16-byte qdot
// pieces (four per step) straight from global memory one step ahead, hitting
// L2 behind the producers' touch.
template <typename T, int D>
constexpr int bstate_ksplit() { return sizeof(T) == 4 || D <= 128 ? 2 : 1; }

template <typename T, int BT, int D, int NW, int NP, int KS>
__global__ void __launch_bounds__(64 * (NW * KS + NP)) bwd_state(BStateArgs<T> a) {
  constexpr int NB = BT / 16, NDT = D / 16;
  constexpr int NCW = NW * KS, NDH = NDT / KS;
  static_assert(KS == 1 || (NDT % KS == 0 && NB % KS == 0), "K-split must tile dh and dv_new");
  static_assert(sizeof(T) == 2 || KS == 2, "float32 tiles (split products) run the K-split");
  constexpr int NVS = D / (16 * NW);
  constexpr int WBYTES = BT * D * (int)sizeof(T);
  constexpr int BUF = 2 * WBYTES;
  constexpr int PIECES = BUF / 1024;
  // two tile buffers where they fit (float32 at D = 256: one, with a third
  // barrier E per chunk after which the producers refill it)
  constexpr int NBUF = 2 * BUF <= 132 * 1024 ? 2 : 1;
  // qdot straight from global memory by the compute waves (K-split: its LDS goes
  // to the exchange buffer; D = 256: it does not fit beside the tiles); one step
  // ahead in spare registers up to 4 row tiles per wave, else loaded right before
  // the dh update that uses it (registers)
  constexpr bool QG = KS > 1 || D > 128;
  constexpr bool QAHEAD = NDH <= 4;
  static_assert(BUF % 1024 == 0, "tiles must split into 1 KB pieces");
  __shared__ __align__(16) char sbuf0[BUF];
  __shared__ __align__(16) char sbuf1[NBUF == 2 ? BUF : 16];
  __shared__ __align__(16) f32x4 sDV[NW * NB * 64];    // dvp^T in compute-lane order
  __shared__ __align__(16) f32x4 sQD[QG ? 1 : NW * NDT * 64];   // (scale qg^T do)^T, same
  __shared__ __align__(16) f32x4 sX[KS > 1 ? NCW * NB * 64 : 1];     // K-split partials of kg dh
  __shared__ __align__(16) float sGL0[D];
  __shared__ __align__(16) float sGL1[NBUF == 2 ? D : 4];
  __shared__ __align__(16) float sJunk[64];

  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  int unit, vs;
  bool one_xcd = false;   // all slices of the unit on this workgroup's XCD
  {
    const int nwg = gridDim.x, id = blockIdx.x;
    const int per_xcd = nwg / 8;
    if (nwg % 8 == 0 && per_xcd % NVS == 0) {
      const int xcd = id % 8, slot = id / 8;
      unit = xcd * (per_xcd / NVS) + slot / NVS;
      vs = slot % NVS;
      one_xcd = true;
    } else {
      unit = id / NVS;
      vs = id % NVS;
    }
  }
  // a unit is one (b,h), or one (head, sequence) of a variable-length batch
  int bh = unit, c0 = 0, n = a.N;
  size_t st_idx = (size_t)unit;          // index of this unit's dh_final / dh0
  if (a.cu) {
    const int sg = unit % a.S;
    bh = unit / a.S;
    const SeqChunks sc = seq_chunks(a.cu, sg, a.N);
    c0 = sc.c0;
    n = sc.n;
    st_idx = (size_t)sg * a.H + bh;
  }
  // step i works on chunk c0 + n-1-i
  auto chunk_id = [&](int i) { return (size_t)bh * a.N + c0 + (n - 1 - i); };
  // float32 tiles are stored transposed in LDS (W^T [d][t], kg [t][d]), so that
  // every MFMA operand of the compute waves is one 16-byte LDS read; bfloat16 tiles
  // keep the stored layout (DMA, chained columns).  With one tile buffer (D = 256)
  // the producers stage one tile at a time (four blocks per lane and tile: both
  // at once would spill)
  constexpr bool TR = sizeof(T) == 4;
  // element offset of logical (row r, element e) in a float32 tile with `re`
  // elements per row, its 16-byte chunks XOR-swizzled by the row: by r ^ (r >> 4),
  // a permutation over any 16 consecutive rows (the MFMA operand reads), which also
  // spreads the rows 4 w + c that the producers' transposed stores of one
  // instruction write (by r alone those take four chunk places, an 8-way LDS bank
  // conflict)
  auto swz = [](int r, int e, int re) {
    const int nchunk = re / 4, m = (nchunk < 16 ? nchunk : 16) - 1;
    return r * re + (((e / 4) ^ ((r ^ (r >> 4)) & m)) * 4) + (e % 4);
  };
  // the same for byte `pos` of row r, as a byte offset
  auto swzb = [](int r, int pos, int re) {
    const int nchunk = re / 4, m = (nchunk < 16 ? nchunk : 16) - 1;
    return r * re * 4 + (((pos / 16) ^ ((r ^ (r >> 4)) & m)) * 16) + (pos % 16);
  };

  if (wv >= NCW) {
    // ---- producers ----------------------------------------------------------
    constexpr int ROWB_W = D * (int)sizeof(T), ROWB_K = BT * (int)sizeof(T);
    constexpr int WPIECES = WBYTES / 1024;
    constexpr int PP = PIECES / NP;
    static_assert(PIECES % NP == 0 && (NW * NB) % NP == 0 && (NW * NDT) % NP == 0,
                  "work must split evenly");
    const int p = wv - NCW;
    // TR: W and kg^T through registers in 4 x 4 blocks, four 16-byte global loads
    // (rows of the stored tile, consecutive lanes on consecutive columns) and four
    // 16-byte LDS stores (rows of the transposed tile) per block
    constexpr int NBLK = (BT / 4) * (D / 4);                // blocks per tile
    constexpr int BPL = TR ? NBLK / (64 * NP) : 1;          // blocks per producer lane
    static_assert(!TR || NBLK % (64 * NP) == 0, "blocks must split over the producers");
    // The stored tiles are in the split pair layout (gdn2_common.h): a block row's
    // four elements are 8 bytes of hi and 8 of lo, moved and transposed as they
    // are, into the same layout of the transposed tile (no arithmetic)
    Split4 stW[BPL][4], stK[BPL][4];
    auto tr_load_w = [&](int i) __attribute__((always_inline)) {
      const char* w = reinterpret_cast<const char*>(a.W + chunk_id(i) * BT * D);  // [t][d]
      int ln = lane;   // one tile buffer: the block offsets are recomputed per
      if constexpr (NBUF == 1) asm volatile("" : "+v"(ln));   // staging, not kept live
#pragma unroll
      for (int q = 0; q < BPL; ++q) {
        const int b = (q * NP + p) * 64 + ln;
        const int wt4 = b / (D / 4), wd4 = b % (D / 4);     // W rows 4 wt4 + r, columns 4 wd4
#pragma unroll
        for (int r = 0; r < 4; ++r) stW[q][r] = split_load4(w + (size_t)(4 * wt4 + r) * D * 4, 4 * wd4);
      }
    };
    auto tr_load_k = [&](int i) __attribute__((always_inline)) {
      const char* k = reinterpret_cast<const char*>(a.KgT + chunk_id(i) * D * BT);  // [d][t]
      int ln = lane;   // one tile buffer: the block offsets are recomputed per
      if constexpr (NBUF == 1) asm volatile("" : "+v"(ln));   // staging, not kept live
#pragma unroll
      for (int q = 0; q < BPL; ++q) {
        const int b = (q * NP + p) * 64 + ln;
        const int kd4 = b / (BT / 4), kt4 = b % (BT / 4);   // kg^T rows 4 kd4 + r, columns 4 kt4
#pragma unroll
        for (int r = 0; r < 4; ++r) stK[q][r] = split_load4(k + (size_t)(4 * kd4 + r) * BT * 4, 4 * kt4);
      }
    };
    // hi and lo of column c of a staged block as the 4-element runs of the
    // transposed row, at element e of row r of a swizzled tile with `re` elements
    // per row
    auto put_t = [&](char* tile, int r, int e, int re, const Split4 (&s)[4], int c) __attribute__((always_inline)) {
      const bf16x4 hi = {s[0].hi[c], s[1].hi[c], s[2].hi[c], s[3].hi[c]};
      const bf16x4 lo = {s[0].lo[c], s[1].lo[c], s[2].lo[c], s[3].lo[c]};
      const int pos = (e / 32) * 128 + split_pos(e % 32);     // unswizzled byte in the row
      *reinterpret_cast<bf16x4*>(tile + swzb(r, pos, re)) = hi;
      *reinterpret_cast<bf16x4*>(tile + swzb(r, pos + 64, re)) = lo;
    };
    auto tr_store_w = [&](char* base) __attribute__((always_inline)) {
      int ln = lane;   // one tile buffer: the block offsets are recomputed per
      if constexpr (NBUF == 1) asm volatile("" : "+v"(ln));   // staging, not kept live
#pragma unroll
      for (int q = 0; q < BPL; ++q) {
        const int b = (q * NP + p) * 64 + ln;
        const int wt4 = b / (D / 4), wd4 = b % (D / 4);
#pragma unroll
        for (int c = 0; c < 4; ++c) put_t(base, 4 * wd4 + c, 4 * wt4, BT, stW[q], c);   // W^T [d][t]
      }
    };
    auto tr_store_k = [&](char* base) __attribute__((always_inline)) {
      int ln = lane;   // one tile buffer: the block offsets are recomputed per
      if constexpr (NBUF == 1) asm volatile("" : "+v"(ln));   // staging, not kept live
#pragma unroll
      for (int q = 0; q < BPL; ++q) {
        const int b = (q * NP + p) * 64 + ln;
        const int kd4 = b / (BT / 4), kt4 = b % (BT / 4);
#pragma unroll
        for (int c = 0; c < 4; ++c) put_t(base + WBYTES, 4 * kt4 + c, 4 * kd4, D, stK[q], c);   // kg [t][d]
      }
    };
    auto tr_load = [&](int i) __attribute__((always_inline)) {
      tr_load_w(i);
      tr_load_k(i);
    };
    auto tr_store = [&](char* base) __attribute__((always_inline)) {
      tr_store_w(base);
      tr_store_k(base);
    };
    // g_last of chunk i into `gl`
    auto gl_dma = [&](int i, float* gl) __attribute__((always_inline)) {
      if (p == NP - 1 && lane < D / 4) lds_dma16(a.GL + chunk_id(i) * D + lane * 4, gl);
    };
    // dvp^T[col][t] of chunk i: compute wave w, row block it -> sDV[(w NB + it) 64 + lane]
    auto gather_dv = [&](int i) __attribute__((always_inline)) {
      const float* dsrc =
          a.DVPT + chunk_id(i) * D * BT + (size_t)(vs * 16 * NW + li) * BT + 4 * lg;
#pragma unroll
      for (int j = 0; j < NW * NB / NP; ++j) {
        const int q = j * NP + p, w = q / NB, it = q % NB;
        lds_dma16(dsrc + (size_t)w * 16 * BT + it * 16, &sDV[q * 64]);
      }
    };
    // loads of chunk i, in parts: kTiles the tiles (DMA, or TR: into registers),
    // kGl g_last, kGather the gathers (dvp^T, qdot)
    constexpr int kTiles = 1, kGl = 2, kGather = 4, kAll = 7;
    auto issue = [&](int i, char* base, float* gl, int parts) __attribute__((always_inline)) {
      const size_t cid = chunk_id(i);
      const char* wsrc = reinterpret_cast<const char*>(a.W + cid * BT * D);
      const char* ksrc = reinterpret_cast<const char*>(a.KgT + cid * D * BT);
      if (parts & kTiles) {
      if constexpr (TR) tr_load(i);
#pragma unroll
      for (int j = 0; j < (TR ? 0 : PP); ++j) {
        const int piece = p * PP + j;
        char* dst = base + piece * 1024;
        if (piece < WPIECES) {
          const int ib = piece * 1024 + lane * 16;
          const int r = ib / ROWB_W, pch = (ib % ROWB_W) / 16;
          constexpr int NCH = ROWB_W / 16, M = (NCH < 16 ? NCH : 16) - 1;
          lds_dma16(wsrc + (size_t)r * ROWB_W + ((pch ^ (r & M)) * 16), dst);
        } else {
          const int ib = (piece - WPIECES) * 1024 + lane * 16;
          const int r = ib / ROWB_K, pch = (ib % ROWB_K) / 16;
          constexpr int NCH = ROWB_K / 16, M = (NCH < 16 ? NCH : 16) - 1;
          lds_dma16(ksrc + (size_t)r * ROWB_K + ((pch ^ (r & M)) * 16), dst);
        }
      }
      }
      if (parts & kGl) gl_dma(i, gl);
      if (!(parts & kGather)) return;
      gather_dv(i);
      // (scale qg^T do)^T[col][d]: wave w, tile at -> sQD[(w NDT + at) 64 + lane]
      if constexpr (!QG) {
        const float* qsrc = a.QDOT + cid * D * D + (size_t)(vs * 16 * NW + li) * D + 4 * lg;
#pragma unroll
        for (int j = 0; j < NW * NDT / NP; ++j) {
          const int q = j * NP + p, w = q / NDT, at = q % NDT;
          lds_dma16(qsrc + (size_t)w * 16 * D + at * 16, &sQD[q * 64]);
        }
      }
    };
    constexpr int LINE = 128;
    constexpr int LW = WBYTES / LINE;
    constexpr int LDV = 16 * NW * (BT * 4 / LINE);
    constexpr int LQD = 16 * NW * (D * 4 / LINE);
    constexpr int LG = (D * 4 + LINE - 1) / LINE;
    constexpr int LTOT = 2 * LW + LDV + LQD + LG;           // at most (one slice)
    constexpr int NTP = ((LTOT + 63) / 64 + NP - 1) / NP;
    // W / kg^T lines are read by every column slice of the unit: when the
    // slices share an XCD (one L2), slice v touches only the v-th share of them
    const int lws = one_xcd ? (2 * LW + NVS - 1) / NVS : 2 * LW;
    const int lw0 = one_xcd ? vs * lws : 0;
    const int ltot = lws + LDV + LQD + LG;
    auto touch = [&](int i) __attribute__((always_inline)) {
      const size_t cid = chunk_id(i);
      const char* wsrc = reinterpret_cast<const char*>(a.W + cid * BT * D);
      const char* ksrc = reinterpret_cast<const char*>(a.KgT + cid * D * BT);
      const char* dsrc =
          reinterpret_cast<const char*>(a.DVPT + cid * D * BT + (size_t)vs * 16 * NW * BT);
      const char* qsrc =
          reinterpret_cast<const char*>(a.QDOT + cid * D * D + (size_t)vs * 16 * NW * D);
      const char* gsrc = reinterpret_cast<const char*>(a.GL + cid * D);
#pragma unroll
      for (int j = 0; j < NTP; ++j) {
        int l = (j * NP + p) * 64 + lane;
        l = l < ltot ? l : ltot - 1;
        const int lw = min(lw0 + l, 2 * LW - 1);               // line of W | kg^T
        const char* src = l < lws ? (lw < LW ? wsrc + lw * LINE : ksrc + (lw - LW) * LINE)
                        : l < lws + LDV ? dsrc + (l - lws) * LINE
                        : l < lws + LDV + LQD ? qsrc + (l - lws - LDV) * LINE
                        : gsrc + (l - lws - LDV - LQD) * LINE;
        lds_dma4(src, sJunk);
      }
    };
    auto wait_step = [&](int i) __attribute__((always_inline)) {
      if (i + 1 < n) wait_vmcnt<NTP>();
      else wait_vmcnt<0>();
    };
    auto barrier = []() __attribute__((always_inline)) {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    auto exp_gl = [&](float* gl) __attribute__((always_inline)) {
      if (p == NP - 1) {
#pragma unroll
        for (int j = 0; j < (D + 63) / 64; ++j)
          if (j * 64 + lane < D) gl[j * 64 + lane] = __expf(gl[j * 64 + lane]);
      }
    };
    if constexpr (NBUF == 1 && TR) {
      // One tile buffer, tiles through registers one at a time.  Chunk i+1's
      // dvp gather and kg^T loads go out after B(i) (dvp(i) is in registers), its
      // kg is stored after X(i) (the first product has read kg(i)) and its W loads
      // issued; g_last after E(i) (the dh update has read e^{g_last}(i)); W and
      // e^{g_last} are stored after B(i+1), before X(i+1) where the dh update
      // starts reading them.  Register results are waited for by the compiler; the
      // LDS-DMA gathers before the barrier that publishes them.
      if (n > 0) {
        gather_dv(0);
        gl_dma(0, sGL0);
        tr_load_k(0);
        tr_store_k(sbuf0);
        __builtin_amdgcn_sched_barrier(0);
        tr_load_w(0);
      }
      if (n > 1) touch(1);
      for (int i = 0; i < n; ++i) {
        if (i == 0) wait_vmcnt<0>();   // chunk 0's gather, g_last and W
        barrier();  // A(i)
        barrier();  // B(i)
        // W(i) and e^{g_last}(i) are first read after X(i): stored behind the
        // compute waves' kg dh (between A and B they would hold up B)
        if (i > 0) wait_step(i);       // g_last(i): only the touches may be outstanding
        tr_store_w(sbuf0);
        exp_gl(sGL0);
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < n) {
          gather_dv(i + 1);
          tr_load_k(i + 1);
        }
        barrier();  // X(i)
        if (i + 1 < n) {
          tr_store_k(sbuf0);   // waits for the kg loads and so for the gather issued before
          // one tile's registers at a time: the W loads stay behind the kg stores
          __builtin_amdgcn_sched_barrier(0);
          tr_load_w(i + 1);
        }
        barrier();  // E(i): chunk i's W and e^{g_last} are no longer read
        if (i + 1 < n) {
          gl_dma(i + 1, sGL0);
          if (i + 2 < n) touch(i + 2);
        }
      }
      return;
    }
    // The dvp / qdot buffer is single: the next chunk's gather goes out after B.
    if (n > 0) issue(0, sbuf0, sGL0, kAll);
    if (n > 1) touch(1);
    if constexpr (NBUF == 1) {
      for (int i = 0; i < n; ++i) {
        wait_step(i);
        if constexpr (TR) tr_store(sbuf0);
        exp_gl(sGL0);
        barrier();  // A(i)
        barrier();  // B(i)
        if constexpr (KS > 1) barrier();  // X(i)
        barrier();  // E(i): chunk i's tiles are no longer read
        if (i + 1 < n) {
          issue(i + 1, sbuf0, sGL0, kAll);
          if (i + 2 < n) touch(i + 2);
        }
      }
      return;
    }
    // The next chunk's tiles and g_last move once A(i) has passed (their buffers
    // were last read in chunk i-1), its gathers once B(i) has (single buffers,
    // read between A(i) and B(i)); the touch comes last, so waiting for all but
    // the touch waits for all of them.
    if constexpr (TR) {
      // Through registers: chunk i's kg is stored before A(i) (the first product
      // reads it after B(i)), its W after B(i), behind the compute waves' kg dh
      // (the dh update reads it after X(i)); chunk i+1's tile loads then go out
      // with its gathers, g_last once A(i) has freed its buffer.
      for (int i = 0; i < n; i += 2) {
        wait_step(i);
        tr_store_k(sbuf0);
        exp_gl(sGL0);
        barrier();  // A(i)
        if (i + 1 < n) issue(i + 1, sbuf1, sGL1, kGl);
        barrier();  // B(i)
        tr_store_w(sbuf0);
        if (i + 1 < n) {
          issue(i + 1, sbuf1, sGL1, kTiles | kGather);
          if (i + 2 < n) touch(i + 2);
          barrier();  // X(i)
          wait_step(i + 1);
          tr_store_k(sbuf1);
          exp_gl(sGL1);
          barrier();  // A(i+1)
          if (i + 2 < n) issue(i + 2, sbuf0, sGL0, kGl);
          barrier();  // B(i+1)
          tr_store_w(sbuf1);
          if (i + 2 < n) {
            issue(i + 2, sbuf0, sGL0, kTiles | kGather);
            if (i + 3 < n) touch(i + 3);
          }
          barrier();  // X(i+1)
        } else {
          barrier();  // X(i)
        }
      }
      return;
    }
    constexpr int kEarly = 0, kAfterA = kTiles | kGl;
    for (int i = 0; i < n; i += 2) {
      wait_step(i);
      if constexpr (TR) tr_store(sbuf0);
      if (kEarly && i + 1 < n) issue(i + 1, sbuf1, sGL1, kEarly);
      exp_gl(sGL0);
      barrier();  // A(i)
      if (i + 1 < n) issue(i + 1, sbuf1, sGL1, kAfterA);
      barrier();  // B(i)
      if (i + 1 < n) {
        issue(i + 1, sbuf1, sGL1, kGather);
        if (i + 2 < n) touch(i + 2);
        if constexpr (KS > 1) barrier();  // X(i)
        wait_step(i + 1);
        if constexpr (TR) tr_store(sbuf1);
        if (kEarly && i + 2 < n) issue(i + 2, sbuf0, sGL0, kEarly);
        exp_gl(sGL1);
        barrier();  // A(i+1)
        if (i + 2 < n) issue(i + 2, sbuf0, sGL0, kAfterA);
        barrier();  // B(i+1)
        if (i + 2 < n) issue(i + 2, sbuf0, sGL0, kGather);
        if (i + 3 < n) touch(i + 3);
        if constexpr (KS > 1) barrier();  // X(i+1)
      } else {
        if constexpr (KS > 1) barrier();  // X(i)
      }
    }
    return;
  }

  // ---- compute waves ----------------------------------------------------------
  const int wcol = wv % NW, ks = wv / NW;   // column slice, k-half (K-split)
  const int col = vs * 16 * NW + wcol * 16 + li;
  // element (row r, logical column c) of a swizzled tile with `re` elements per row
  auto elem = [](const T* tile, int r, int c, int re) -> float {
    constexpr int EPC = 16 / sizeof(T);
    const int sc = kpos<T>(c);
    const int nchunk = re / EPC;
    const int m = (nchunk < 16 ? nchunk : 16) - 1;
    const int j = sc / EPC;
    return to_f(tile[r * re + ((j ^ (r & m)) * EPC) + (sc % EPC)]);
  };

  f32x4 dh[NDH];   // row tiles at = ks NDH + j of this slice's dh
  if (a.dh_final) {
#pragma unroll
    for (int j = 0; j < NDH; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dh[j][r] = sanitize(
            a.dh_final[(st_idx * D + (ks * NDH + j) * 16 + 4 * lg + r) * D + col]);
  } else {
#pragma unroll
    for (int j = 0; j < NDH; ++j) dh[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // The last chunk's dh' is dh_final as given: B3 takes it raw (gdn2_pipeline.py:
  // 52-56,105) while the carry above starts from its sanitized value (gdn2_bwd.py:53)
  if (n > 0) {
    float* dht = a.DHT + chunk_id(0) * D * D + (size_t)col * D;
#pragma unroll
    for (int j = 0; j < NDH; ++j) {
      f32x4 raw = {0.f, 0.f, 0.f, 0.f};
      if (a.dh_final) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          raw[r] = a.dh_final[(st_idx * D + (ks * NDH + j) * 16 + 4 * lg + r) * D + col];
      }
      store4(dht + (ks * NDH + j) * 16 + 4 * lg, raw);
    }
  }
  // this wave's qdot pieces from global memory (QG), loaded ahead
  f32x4 qnext[QG && QAHEAD ? NDH : 1], qd[NDH];
  auto load_qd = [&](int i, f32x4* dst) __attribute__((always_inline)) {
    const float* qsrc = a.QDOT + chunk_id(i) * D * D + (size_t)col * D + 4 * lg;
#pragma unroll
    for (int j = 0; j < NDH; ++j) dst[j] = load4f(qsrc + (ks * NDH + j) * 16);
  };
  if constexpr (QG && QAHEAD) {
    if (n > 0) load_qd(0, qnext);
  }

  auto step = [&](int i, const char* cur, const float* eglc) __attribute__((always_inline)) {
    const size_t cid = chunk_id(i);
    // qdot from global: LDS-only barriers, so its loads stay in flight (the
    // producers order their DMA with their own vmcnt waits)
    if constexpr (QG) lds_barrier(); else __syncthreads();  // A(i)
    f32x4 dvn[NB];
#pragma unroll
    for (int it = 0; it < NB; ++it) dvn[it] = sDV[(wcol * NB + it) * 64 + lane];
    if constexpr (QG && QAHEAD) {
#pragma unroll
      for (int j = 0; j < NDH; ++j) qd[j] = qnext[j];
      if (i + 1 < n) load_qd(i + 1, qnext);
    } else if constexpr (!QG) {
#pragma unroll
      for (int at = 0; at < NDT; ++at) qd[at] = sQD[(wv * NDT + at) * 64 + lane];
    }
    if constexpr (QG) lds_barrier(); else __syncthreads();  // B(i)
    const T* sW = reinterpret_cast<const T*>(cur);
    const T* sK = reinterpret_cast<const T*>(cur + WBYTES);
    // MFMA row operands: kg[t][d] for rows d = 16 at + 4 lg + e, column t = 16 it + li
    // (dv_new), W[t][d] for rows t = 16 it + 4 lg + e, column d = 16 at + li (dh)
    // (TR: one 16-byte read from the transposed tiles; otherwise four reads below)
    auto xk = [&](int at, int it) __attribute__((always_inline)) {
      return load4f(reinterpret_cast<const float*>(cur + WBYTES) +
                    swz(it * 16 + li, at * 16 + 4 * lg, D));
    };
    auto xw = [&](int it, int at) __attribute__((always_inline)) {
      return load4f(reinterpret_cast<const float*>(cur) + swz(at * 16 + li, it * 16 + 4 * lg, BT));
    };

    if (i > 0) {   // dh_{c+1} (chunk n-1's was stored raw before the scan)
      float* dht = a.DHT + cid * D * D + (size_t)col * D;
#pragma unroll
      for (int j = 0; j < NDH; ++j) store4(dht + (ks * NDH + j) * 16 + 4 * lg, dh[j]);
    }

    // dv_new = dvp + kg dh: X[t][d] = kg^T[d][t]
    if constexpr (KS > 1) {
      // this wave's half of kg dh; the NB row blocks are independent accumulators
      f32x4 part[NB];
#pragma unroll
      for (int it = 0; it < NB; ++it) part[it] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (TR) {
        // split form: dh split once per chunk; the kg tile holds the split pairs
        static_assert(NDH % 2 == 0, "pairs of k-groups");
        Split8 dhs[NDH / 2];
#pragma unroll
        for (int q = 0; q < NDH / 2; ++q) dhs[q] = split8(dh[2 * q], dh[2 * q + 1]);
#pragma unroll
        for (int q = 0; q < NDH / 2; ++q)
#pragma unroll
          for (int it = 0; it < NB; ++it)
            mma3(part[it], split_read(xk(ks * NDH + 2 * q, it), xk(ks * NDH + 2 * q + 1, it)), dhs[q]);
      } else {
#pragma unroll
      for (int j = 0; j < NDH; ++j) {
        const int at = ks * NDH + j;
#pragma unroll
        for (int it = 0; it < NB; ++it) {
          f32x4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = elem(sK, at * 16 + 4 * lg + e, it * 16 + li, BT);
          mma(part[it], x, dh[j]);
        }
      }
      }
      // exchange the halves; both waves form dv_new in the same order
#pragma unroll
      for (int it = 0; it < NB; ++it) sX[(wv * NB + it) * 64 + lane] = part[it];
      lds_barrier();  // X(i)
      const int pw = (1 - ks) * NW + wcol;
#pragma unroll
      for (int it = 0; it < NB; ++it) {
        const f32x4 o = sX[(pw * NB + it) * 64 + lane];
        const f32x4 sum = ks == 0 ? part[it] + o : o + part[it];
#pragma unroll
        for (int r = 0; r < 4; ++r) dvn[it][r] = sanitize(dvn[it][r] + sum[r]);
      }
    } else {
#pragma unroll
      for (int it = 0; it < NB; ++it) {
#pragma unroll
        for (int at = 0; at < NDT; ++at) {
          f32x4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = elem(sK, at * 16 + 4 * lg + e, it * 16 + li, BT);
          mma(dvn[it], x, dh[at]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) dvn[it][r] = sanitize(dvn[it][r]);
        // D = 256: keep the operand reads of one row block in flight at a time
        if constexpr (NDT > 8) __builtin_amdgcn_sched_barrier(0);
      }
    }
    float* dvo = a.DVNT + cid * D * BT + (size_t)col * BT;
#pragma unroll
    for (int it = ks * (NB / KS); it < (ks + 1) * (NB / KS); ++it)
      store4(dvo + it * 16 + 4 * lg, dvn[it]);

    // dh <- e^{gl} dh + qdot - W^T dv_new: X[d][t] = W[t][d]
    if constexpr (QG && !QAHEAD) load_qd(i, qd);
    // split form: dv_new split once per chunk; the W^T tile holds the split pairs
    Split8 dvs[TR ? NB / 2 : 1];
    if constexpr (TR) {
#pragma unroll
      for (int q = 0; q < NB / 2; ++q) dvs[q] = split8(dvn[2 * q], dvn[2 * q + 1]);
    }
#pragma unroll
    for (int j = 0; j < NDH; ++j) {
      const int at = ks * NDH + j;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (TR) {
#pragma unroll
        for (int q = 0; q < NB / 2; ++q) mma3(acc, split_read(xw(2 * q, at), xw(2 * q + 1, at)), dvs[q]);
      } else {
#pragma unroll
        for (int it = 0; it < NB; ++it) {
          f32x4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = elem(sW, it * 16 + 4 * lg + e, at * 16 + li, D);
          mma(acc, x, dvn[it]);
        }
      }
      const f32x4 egl = load4f(eglc + at * 16 + 4 * lg);
#pragma unroll
      for (int r = 0; r < 4; ++r) dh[j][r] = sanitize(egl[r] * dh[j][r] + qd[j][r] - acc[r]);
      if constexpr (NDT > 8) {
        if (j % 4 == 3) __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  if constexpr (NBUF == 1) {
    for (int i = 0; i < n; ++i) {
      step(i, sbuf0, sGL0);
      lds_barrier();  // E(i)
    }
  } else {
    for (int i = 0; i < n; i += 2) {
      step(i, sbuf0, sGL0);
      if (i + 1 < n) step(i + 1, sbuf1, sGL1);
    }
  }
#pragma unroll
  for (int j = 0; j < NDH; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      a.dh0[(st_idx * D + (ks * NDH + j) * 16 + 4 * lg + r) * D + col] = dh[j][r];
}

// ============================================================================
// bwd_b2 (B2, fused): per chunk (gdn2_bwd.py:84-122 and the qg^T do term of B1)
//   dAqk = (do v_new^T) . causal        [t][s]
//   dvp^T = (Aqk^T do)^T                [e][s]   (the causal Aqk)
//   qdot = scale do^T qg                [e][d]   ((scale qg^T do)^T)
// with do, v_new^T, Aqk and qg staged once in LDS as float32.  Wave w owns the
// 16-row block w of dAqk and of Aqk^T do, and row blocks 2w, 2w+1 (over e) of
// qdot (D = 128; one block per wave at D = 64, four at D = 256).  do stays in LDS
// throughout; the second operand of each product takes one region in turn
// (v_new^T, then Aqk, then qg, each loaded into registers ahead and stored after a
// barrier), so the kernel needs 67 KB of LDS at D = 128: two workgroups per CU, one
// streaming while the other computes (136 KB and one at D = 256).
// ============================================================================
template <typename T>
struct B2Args {
  const float* dout;
  const T* VnT;       // forward residual v_new^T [cid][D][BT] (bfloat16: chained columns)
  const T* Aqk;       // forward residual Aqk [cid][BT][BT] (entries right of the diagonal
                      // block are not written: masked here)
  const T* Qg;        // forward residual qg [cid][BT][D]
  int T_len, H, N;
  float scale;
  float *DAQK, *DVPT, *QDOT;
};

// What one bwd_b2 launch forms: all three products (the fused backward), or for
// the stage entry points only B2's dAqk and Aqk^T do (dav_backward_pallas) or only
// B1's scale qg^T do (gdn2_dhu_backward).
enum B2Mode { kB2All = 0, kB2Dav = 1, kB2Qdot = 2 };

// Waves of a bwd_b2 workgroup: four (one per 16-token row block), eight at D = 256,
// where the 136 KB of LDS leave one workgroup per CU: the row blocks' column
// tiles are then dealt over two waves each (two waves per SIMD instead of one).
constexpr int b2_waves(int D) { return D > 128 ? 8 : 4; }

template <typename T, int D, int B2M = kB2All>
__global__ void __launch_bounds__(64 * b2_waves(D), 2) bwd_b2(B2Args<T> a) {
  constexpr int BT = 64, NDT = D / 16, NKT = BT / 16;
  constexpr int NWV = b2_waves(D), NT = 64 * NWV, WPB = NWV / 4;   // waves per row block
  constexpr int LDO = D + 4, LDV = BT + 4, LDA = BT + 4, LDQ = D + 4;
  constexpr int BF = sizeof(T) == 2;
  constexpr int RV = D * LDV, RA = BT * LDA, RQ = BT * LDQ;
  constexpr int RS = RV > RQ ? (RV > RA ? RV : RA) : (RQ > RA ? RQ : RA);
  __shared__ __align__(16) float sDo[BT * LDO];
  __shared__ __align__(16) float sR[RS];   // v_new^T [e][s], then Aqk [t][s], then qg [t][d]
  float* const sV = sR;
  float* const sA = sR;
  float* const sQ = sR;
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: MFMA under branches
  // row block; part of its column tiles (WPB parts; a constant 0 with one wave per block)
  const int rb = WPB == 1 ? wv : wv % 4, part = WPB == 1 ? 0 : wv / 4;
  const int cid = blockIdx.x;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  const size_t HD = (size_t)a.H * D;
  const size_t tok0 = ((size_t)bb * a.T_len + (size_t)c * BT) * HD + (size_t)hh * D;
  auto rowop = [&](const float* base, int ld, int r0, int k0) __attribute__((always_inline)) {
    return load4f(&base[(r0 + li) * ld + k0 + 4 * lg]);
  };
  auto colop = [&](const float* base, int ld, int k0, int c0) __attribute__((always_inline)) {
    f32x4 y;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = base[(k0 + 4 * lg + r) * ld + c0 + li];
    return y;
  };
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  const GMat mQ{a.Qg, BF, D, 0, 0};
  Staged s1, s2;   // s1: do, then qg (stored after the dvp^T product)
  {
    // do rows are (B,T,H,D) token rows: pitch H*D
    const GMat mDo{a.dout, 0, (int)HD, 0, 0};
    const GMat mV{a.VnT, BF, BT, 0, BF};
    // Aqk: blocks right of the diagonal block are unwritten; causal mask on load
    const GMat mA{a.Aqk, BF, BT, 1, 0};
    stage_load<NT>(s1, mDo, tok0, BT, D, tid);
    if constexpr (B2M != kB2Qdot) stage_load<NT>(s2, mV, (size_t)cid * D * BT, D, BT, tid);
    stage_store<NT>(sDo, LDO, s1, mDo, BT, D, 0, 0, false, tid);
    if constexpr (B2M != kB2Qdot) stage_store<NT>(sV, LDV, s2, mV, D, BT, 0, 0, false, tid);
    // qg and Aqk are in flight while dAqk is formed (LDS-only barriers)
    if constexpr (B2M != kB2Dav) stage_load<NT>(s1, mQ, (size_t)cid * BT * D, BT, D, tid);
    if constexpr (B2M != kB2Qdot) stage_load<NT>(s2, mA, (size_t)cid * BT * BT, BT, BT, tid);
    lds_barrier();
    if constexpr (B2M != kB2Qdot) {
    // dAqk[t][s] = sum_e do[t][e] v_new[s][e], s <= t: column blocks right of
    // the own row block are zero and not formed; column tile st of row block rb
    // belongs to part st mod WPB
    {
      f32x4 acc[NKT];
#pragma unroll
      for (int st = 0; st < NKT; ++st) acc[st] = z4;
#pragma unroll
      for (int kg = 0; kg < NDT; ++kg) {
        const f32x4 x = rowop(sDo, LDO, rb * 16, kg * 16);
#pragma unroll
        for (int st = 0; st < NKT; ++st)
          if (st <= rb && st % WPB == part) mma(acc[st], x, colop(sV, LDV, kg * 16, st * 16));
      }
      float* o = a.DAQK + (size_t)cid * BT * BT;
#pragma unroll
      for (int st = 0; st < NKT; ++st) {
        if (st % WPB != part) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb * 16 + 4 * lg + r, s2 = st * 16 + li;
          o[row * BT + s2] = s2 <= row ? sanitize(acc[st][r]) : 0.f;   // gdn2_bwd.py:95
        }
      }
    }
    lds_barrier();  // every wave is done with v_new^T
    stage_store<NT>(sA, LDA, s2, mA, BT, BT, 0, 0, false, tid);
    }  // B2M != kB2Qdot
  }
  lds_barrier();
  if constexpr (B2M != kB2Qdot) {
  // dvp^T[e][s] = sum_t Aqk[t][s] do[t][e]: rows s of the own block, stored as
  // [e][s]; Aqk[t][s] = 0 for t < s, so token blocks before the own one add nothing
  // (with dAqk's skipped blocks: 5 of 8 block-products per row block); the e tiles
  // of a row block are split over its WPB parts
  {
    constexpr int NDV = NDT / WPB;
    f32x4 acc[NDV];
#pragma unroll
    for (int n = 0; n < NDV; ++n) acc[n] = z4;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      if (kt < rb) continue;
      const f32x4 x = colop(sA, LDA, kt * 16, rb * 16);      // Aqk^T rows s, k = t
#pragma unroll
      for (int n = 0; n < NDV; ++n)
        mma(acc[n], x, colop(sDo, LDO, kt * 16, (part * NDV + n) * 16));
    }
    float* o = a.DVPT + (size_t)cid * D * BT;
#pragma unroll
    for (int n = 0; n < NDV; ++n)
      store4(o + (size_t)((part * NDV + n) * 16 + li) * BT + rb * 16 + 4 * lg,
             sanitize4(acc[n]));  // :96
  }
  }  // B2M != kB2Qdot
  if constexpr (B2M == kB2Dav) return;
  lds_barrier();  // every wave is done with Aqk
  stage_store<NT>(sQ, LDQ, s1, mQ, BT, D, 0, 0, false, tid);
  lds_barrier();
  // qdot[e][d] = scale sum_t do[t][e] qg[t][d], in items of one row block e and
  // QCT column tiles d (at D = 256 half a row: eight accumulator tiles, 32
  // registers), QI items per wave, one at a time
  {
    constexpr int QCT = D > 128 ? NDT / 2 : NDT, NCH = NDT / QCT, QI = NDT * NCH / NWV;
    static_assert(QI * NWV == NDT * NCH, "qdot items must split over the waves");
#pragma unroll (D <= 128 ? QI : 1)
    for (int qi = 0; qi < QI; ++qi) {
      const int item = wv * QI + qi, eb = item / NCH, d0 = (item % NCH) * QCT;
      f32x4 acc[QCT];
#pragma unroll
      for (int n = 0; n < QCT; ++n) acc[n] = z4;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        const f32x4 x = colop(sDo, LDO, kt * 16, eb * 16);   // do^T rows e, k = t
#pragma unroll
        for (int n = 0; n < QCT; ++n) mma(acc[n], x, colop(sQ, LDQ, kt * 16, (d0 + n) * 16));
      }
      float* o = a.QDOT + (size_t)cid * D * D;
#pragma unroll
      for (int n = 0; n < QCT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[(eb * 16 + 4 * lg + r) * D + (d0 + n) * 16 + li] = a.scale * acc[n][r];
    }
  }
}

// ============================================================================
// bwd_wy (B3, fused): per chunk the products of gdn2_bwd.py:126-210 and the
// element-wise b k e^{gc}, w v, with dW, dA and dA A^T kept on chip:
//   dqg  = scale do h^T              dW    = -dv_new h^T
//   dkg  = v_new dh'^T               dA    = (dW (b k e^gc)^T + dv_new (w v)^T) . strict
//   d(bke^gc) = A^T dW               d(wv) = A^T dv_new -> dv = d(wv) w, dw = d(wv) v
//   dAkk = -(A^T (dA A^T)) . strict
// Stored operands per chunk: do in (B,T,H,D) rows; h^T, dh'^T as [e][d]; v_new^T,
// dv_new^T as [e][t]; A as [t][s].  One workgroup per chunk; wave w owns the
// 16-token row block w of every product.
// The channels are taken in halves of 64 (two at D = 128): every product above
// except dA is separable over them (dqg, dW, dkg, d(bke^gc) over the key channel
// d; d(wv), dv, dw over the value channel e), and dA's two half sums accumulate in
// registers.  Per half: h^T[:, half] staged (dqg, dW of the half), dh'^T[:, half]
// staged over it (dkg, sum_e dh' h), (b k e^gc | w v) of the half (dA half sum),
// then A and dv_new^T[half] (d(bke^gc), d(wv)); after the last half dA A^T and
// dAkk.  71 KB of LDS and under 256 registers: two workgroups per CU, one
// streaming while the other computes (the next half's h^T and step 5's operands
// are also loaded one phase ahead).  The triangular products skip the 16 x 16
// blocks that A (lower triangular) and the strict masks make zero.
// A stored matrix read with its row index as the MFMA k index is read per lane
// as four scalars (colop); one read with k contiguous is one 16-byte load (rowop).
// ============================================================================
// T: workspace and MFMA operand type; TI: the type of the inputs k, w, v, b and
// of the gradients dv, dw (T, or bfloat16 with float32 tiles).
template <typename T, typename TG, typename TI = T>
struct WyArgs {
  const TI *k, *w, *v, *b;
  const TG* g;
  const float* dout;
  const T* HT;        // forward residual h^T [cid][D][D] (bfloat16: chained columns)
  const T* VnT;       // forward residual v_new^T [cid][D][BT] (bfloat16: chained columns)
  const float* A;     // forward residual A [cid][BT][BT]
  const float* DHT;   // dh'^T [cid][D][D]
  const float* DVNT;  // dv_new^T [cid][D][BT]
  int T_len, H, N;
  float scale;
  float *DQG, *DKG, *DKBD, *DAKK;  // [cid][BT][D] x 3, [cid][BT][BT]
  float* SDH;         // [cid][D]: sum_e dh'[d][e] h[d][e] (the g_last term of dgc)
  TI *dv, *dw;        // gradients (B,T,H,D): d(wv) w, d(wv) v (gdn2_bwd.py:204-205)
};

template <typename T, typename TG, int D, typename TI>
__global__ void __launch_bounds__(256, 2) bwd_wy(WyArgs<T, TG, TI> a) {
  constexpr int BT = 64, NB = BT / 16, NDT = D / 16, NKT = BT / 16;
  constexpr int DH = D < 64 ? D : 64, NH = D / DH, NDH = DH / 16;   // channel halves
  constexpr int LDH = DH + 4;   // [e][d of the half], [s][d of the half]
  constexpr int LD4 = BT + 4;   // [t][s], [e][t]
  constexpr int BF = sizeof(T) == 2;
  // R1 in turn: h^T[:, half] (D x DH), dh'^T[:, half], (b k e^gc | w v) of the half
  // (2 x BT x DH), A (BT x BT) with dv_new^T[half] (DH x BT)
  constexpr int R1 = (D * LDH > 2 * BT * LD4) ? D * LDH : 2 * BT * LD4;
  static_assert(2 * BT * LDH <= R1, "(b k e^gc | w v) must fit R1");
  __shared__ __align__(16) float sR1[R1];
  __shared__ __align__(16) float sW[BT * LDH];    // dW[:, half] [t][d]
  __shared__ __align__(16) float sDA[BT * LD4];   // dA, then dA A^T
  __shared__ __align__(16) float sTot[NB * DH];
  __shared__ __align__(16) float sSdh[DH];
  float* const sKB = sR1;                // (b k e^gc)[s][d]
  float* const sWV = sR1 + BT * LDH;     // (w v)[s][e]
  float* const sA = sR1;                 // A [t][s]
  float* const sDV = sR1 + BT * LD4;     // dv_new^T[e][t]
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  // the wave's row block as a scalar: the triangular products below skip the
  // blocks that A (lower triangular) and the strict masks make zero, by uniform
  // branches (every skipped term is an exact zero, so results are unchanged)
  const int wb = __builtin_amdgcn_readfirstlane(wv);
  const int cid = blockIdx.x;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  const size_t HD = (size_t)a.H * D;
  const size_t tok0 = ((size_t)bb * a.T_len + (size_t)c * BT) * HD + (size_t)hh * D;
  const int t0 = wv * 16 + li;   // this lane's row for row operands of the own block
  // Barriers order LDS data only (lds_barrier): no wave reads global memory
  // another wave of this workgroup wrote.

  auto rowop = [&](const float* base, int ld, int r0, int k0) __attribute__((always_inline)) {
    return load4f(&base[(r0 + li) * ld + k0 + 4 * lg]);
  };
  auto colop = [&](const float* base, int ld, int k0, int c0) __attribute__((always_inline)) {
    f32x4 y;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = base[(k0 + 4 * lg + r) * ld + c0 + li];
    return y;
  };
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

  const GMat mH{a.HT, BF, D, 0, BF};
  const GMat mDH{a.DHT, 0, D, 0, 0};
  const GMat mA{a.A, 0, BT, 0, 0};
  const GMat mDV{a.DVNT, 0, BT, 0, 0};
  const size_t offDD = (size_t)cid * D * D;
  // tid, opaque to the compiler: each staging computes its own addresses (the
  // stagings share their offset pattern, and one shared set of 64-bit addresses
  // would stay live through the kernel)
  auto otid = [&]() __attribute__((always_inline)) {
    int x = tid;
    asm volatile("" : "+v"(x));
    return x;
  };

  // The own rows of do, dv_new and v_new (k = value channel e) are loaded per half
  // (from L2 the second time) ahead of the step using them: the registers stay
  // within two workgroups per CU.
  Staged st;
  stage_load<256, true>(st, mH, offDD, D, DH, otid());   // h^T[:, half 0]
  // rows e0 .. e0 + 16 n of a stored [e][t] matrix at column col, as k = e operands
  // (lane offsets from the chunk's tile, opaque per call like the stagings)
  auto load_rows = [&](f32x4* x, auto src, int e0, int n, int col) __attribute__((always_inline)) {
    const auto* tile = src + (size_t)cid * D * BT;
    int off = (e0 + 4 * lg) * BT + col;
    asm volatile("" : "+v"(off));
#pragma unroll
    for (int kg = 0; kg < n; ++kg)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[kg][r] = to_f(tile[off + (kg * 16 + r) * BT]);
  };
  f32x4 ada[NKT];   // dA rows of the own block, summed over the halves
#pragma unroll
  for (int s2 = 0; s2 < NKT; ++s2) ada[s2] = z4;

#pragma unroll
  for (int hf = 0; hf < NH; ++hf) {
    // the half's own token row and first channel, opaque to the compiler: the two
    // halves then compute their addresses where they use them instead of sharing
    // them (a shared address stays live across the whole kernel)
    int t = t0, d0 = hf * DH;
    asm volatile("" : "+v"(t), "+v"(d0));
    // C-layout element (r) of the own block's tile: its row
    auto orow = [&](int r) { return t - li + 4 * lg + r; };
    // ---- 1. dqg = scale do h^T, dW = -dv_new h^T (columns d of the half) -------
    f32x4 xdo[NDT], xdv[NDT], xvn[NDT];
#pragma unroll
    for (int kg = 0; kg < NDT; ++kg)
      xdo[kg] = load4f(a.dout + tok0 + (size_t)t * HD + kg * 16 + 4 * lg);
    load_rows(xdv, a.DVNT, 0, NDT, t);
    if (hf > 0) lds_barrier();   // the previous half's A, dv_new^T and dW reads are done
    if (tid < DH) sSdh[tid] = 0.f;
    stage_store<256, true>(sR1, LDH, st, mH, D, DH, 0, 0, false, tid);
    lds_barrier();
    {
      f32x4 aq[NDH], aw[NDH];
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) aq[nt] = aw[nt] = z4;
#pragma unroll
      for (int kg = 0; kg < NDT; ++kg) {
#pragma unroll
        for (int nt = 0; nt < NDH; ++nt) {
          // h[d][e] as the row operand (rows d, k = e): the lane's sums are 4
          // consecutive channels d of its own token t, stored as one 16-byte run
          const f32x4 y = colop(sR1, LDH, kg * 16, nt * 16);
          mma(aq[nt], y, xdo[kg]);
          mma(aw[nt], y, xdv[kg]);
        }
      }
      float* dqg = a.DQG + (size_t)cid * BT * D + d0;
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) {
        store4(dqg + (size_t)t * D + nt * 16 + 4 * lg, a.scale * aq[nt]);
        store4(&sW[t * LDH + nt * 16 + 4 * lg], -aw[nt]);
      }
    }

    // ---- 2. dkg = v_new dh'^T, sum_e dh'[d][e] h[d][e] (columns d of the half) --
    Staged sd;   // dh'^T[:, half]
    stage_load<256, true>(sd, mDH, offDD + d0, D, DH, otid());
    load_rows(xvn, a.VnT, 0, NDT, BF ? kpos<bf16_t>(t) : t);
    // each thread multiplies the dh'^T runs it staged with the h^T runs still at
    // the same places in R1 (its column group is fixed: index tid + 256 u keeps
    // tid mod DH/4), then one LDS add per column
    {
      float part[4] = {0.f, 0.f, 0.f, 0.f};
      constexpr int CQ = DH / 4;
      static_assert(256 % CQ == 0, "a thread's column group must stay fixed");
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int i = tid + 256 * u;
        if (i < D * CQ) {
          const f32x4 hv = load4f(&sR1[(i / CQ) * LDH + (i % CQ) * 4]);
#pragma unroll
          for (int e = 0; e < 4; ++e) part[e] += sd.v[u][e] * hv[e];
        }
      }
      lds_barrier();   // every wave is done with h^T
#pragma unroll
      for (int e = 0; e < 4; ++e) atomicAdd(&sSdh[(tid % CQ) * 4 + e], part[e]);
    }
    stage_store<256, true>(sR1, LDH, sd, mDH, D, DH, 0, 0, false, tid);
    lds_barrier();
    if (tid < DH) a.SDH[(size_t)cid * D + d0 + tid] = sSdh[tid];
    {
      f32x4 ak[NDH];
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) ak[nt] = z4;
#pragma unroll
      for (int kg = 0; kg < NDT; ++kg) {
#pragma unroll
        for (int nt = 0; nt < NDH; ++nt)
          mma(ak[nt], colop(sR1, LDH, kg * 16, nt * 16), xvn[kg]);   // token t, 4 channels
      }
      float* dkg = a.DKG + (size_t)cid * BT * D + d0;
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) store4(dkg + (size_t)t * D + nt * 16 + 4 * lg, ak[nt]);
    }
    // step 3's inputs (channels of the half)
    constexpr int NJ = NDH;
    float gv[NJ][4], bv[NJ][4], kv[NJ][4], wvv[NJ][4], vv[NJ][4];
    {
      const size_t row = tok0 + (size_t)t * HD + d0;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const size_t o = row + j * 16 + 4 * lg;
        load_f<4>(a.g + o, gv[j]);
        load_f<4>(a.b + o, bv[j]);
        load_f<4>(a.k + o, kv[j]);
        load_f<4>(a.w + o, wvv[j]);
        load_f<4>(a.v + o, vv[j]);
      }
    }

    // ---- 3. b k e^{gc} and w v of the half into R1 (rows s of the own block) ---
    // lane (li, lg): token s = t, channels d0 + 16 j + 4 lg + e; gc = in-block
    // cumsum over the 16 lanes li (DPP) + the sums of the earlier blocks (sTot)
    float loc[NJ][4], bk[NJ][4];
    lds_barrier();   // every wave is done with dh'^T
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      f32x4 wvo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        loc[j][e] = row_scan16(gv[j][e]);
        bk[j][e] = bv[j][e] * kv[j][e];
        wvo[e] = wvv[j][e] * vv[j][e];
      }
      *reinterpret_cast<f32x4*>(&sWV[t * LDH + j * 16 + 4 * lg]) = wvo;
      if (li == 15) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sTot[wv * DH + j * 16 + 4 * lg + e] = loc[j][e];
      }
    }
    lds_barrier();
    // gc = loc + sums of the earlier blocks: independent 16-byte LDS reads per
    // (block, channel group), all issued before the exponentials
#pragma unroll
    for (int m = 0; m < NB - 1; ++m) {
      if (m < wv) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const f32x4 tv = load4f(&sTot[m * DH + j * 16 + 4 * lg]);
#pragma unroll
          for (int e = 0; e < 4; ++e) loc[j][e] += tv[e];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      f32x4 kb;
#pragma unroll
      for (int e = 0; e < 4; ++e) kb[e] = bk[j][e] * __expf(loc[j][e]);
      *reinterpret_cast<f32x4*>(&sKB[t * LDH + j * 16 + 4 * lg]) = kb;
    }
    // the own rows of dv_new in the half, and step 5's A and dv_new^T[half], in
    // flight during the dA products
    f32x4 xdh[NDH];
    load_rows(xdh, a.DVNT, d0, NDH, t);
    Staged sa, sv;
    stage_load<256, true>(sa, mA, (size_t)cid * BT * BT, BT, BT, otid());
    stage_load<256, true>(sv, mDV, ((size_t)cid * D + d0) * BT, DH, BT, otid());
    lds_barrier();

    // ---- 4. dA += dW[:, half] (b k e^gc)[:, half]^T + dv_new[:, half] (w v)[:, half]^T
#pragma unroll
    for (int kg = 0; kg < NDH; ++kg) {
      const f32x4 x1 = rowop(sW, LDH, wv * 16, kg * 16);   // dW rows, k = d
#pragma unroll
      for (int s2 = 0; s2 < NKT; ++s2) {
        if (s2 <= wb) {   // dA is strictly lower: blocks s > t are masked
          mma(ada[s2], x1, rowop(sKB, LDH, s2 * 16, kg * 16));       // (b k e^gc)[s][d]
          mma(ada[s2], xdh[kg], rowop(sWV, LDH, s2 * 16, kg * 16));  // (w v)[s][e]
        }
      }
    }
    if (hf == NH - 1) {
#pragma unroll
      for (int s2 = 0; s2 < NKT; ++s2)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int sc = s2 * 16 + li;
          sDA[orow(r) * LD4 + sc] = sc < orow(r) ? sanitize(ada[s2][r]) : 0.f;   // :168
        }
    }
    lds_barrier();   // (b k e^gc | w v) no longer read

    // ---- 5. d(bke^gc)[:, half] = A^T dW[:, half], d(wv)[:, half] = A^T dv_new[:, half]
    stage_store<256, true>(sA, LD4, sa, mA, BT, BT, 0, 0, false, tid);
    stage_store<256, true>(sDV, LD4, sv, mDV, DH, BT, 0, 0, false, tid);
    if (hf + 1 < NH) stage_load<256, true>(st, mH, offDD + d0 + DH, D, DH, otid());   // next half's h^T
    lds_barrier();
    {
      f32x4 akb[NDH], awv[NDH];
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) akb[nt] = awv[nt] = z4;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        if (kt >= wb) {   // A[t][m] = 0 for t < m
          const f32x4 x = colop(sA, LD4, kt * 16, wv * 16);   // A^T rows m, k = t
#pragma unroll
          for (int nt = 0; nt < NDH; ++nt) {
            // the channel operand as the rows: the lane's sums are 4 consecutive
            // channels of token m = 16 w + li
            mma(akb[nt], colop(sW, LDH, kt * 16, nt * 16), x);   // dW[t][d] as (rows d, k = t)
            mma(awv[nt], rowop(sDV, LD4, nt * 16, kt * 16), x);  // dv_new^T[e][t]
          }
        }
      }
      // dv = d(wv) w, dw = d(wv) v: w and v re-read in this layout (L2: step 3
      // read them), so the element-wise pass does not need them
      float* dkbd = a.DKBD + (size_t)cid * BT * D + d0;
      f32x4 wl[NDH], vl[NDH];
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) {
        const size_t o = tok0 + (size_t)t * HD + d0 + nt * 16 + 4 * lg;
        wl[nt] = load4f(a.w + o);
        vl[nt] = load4f(a.v + o);
      }
#pragma unroll
      for (int nt = 0; nt < NDH; ++nt) {
        const size_t o = tok0 + (size_t)t * HD + d0 + nt * 16 + 4 * lg;
        store4(dkbd + (size_t)t * D + nt * 16 + 4 * lg, akb[nt]);
        store4(a.dv + o, sanitize4(awv[nt] * wl[nt]));
        store4(a.dw + o, sanitize4(awv[nt] * vl[nt]));
      }
    }
  }

  // ---- 6. TMP = dA A^T (the own rows of dA are read only by this wave) ----------
  // Only the columns n < m <= t of TMP enter dAkk[m][n] (strict), so columns past
  // the own block are not formed (those entries keep dA's zeros)
  auto orow = [&](int r) { return wv * 16 + 4 * lg + r; };
  {
    f32x4 atm[NKT];
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt) atm[nt] = z4;
#pragma unroll
    for (int ks = 0; ks < NKT; ++ks) {
      if (ks <= wb) {   // dA[t][s] = 0 for s > t
        const f32x4 x = rowop(sDA, LD4, wv * 16, ks * 16);    // dA rows t, k = s
#pragma unroll
        for (int nt = 0; nt < NKT; ++nt)
          if (nt <= wb) mma(atm[nt], x, rowop(sA, LD4, nt * 16, ks * 16));  // A[n][s]
      }
    }
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
      if (nt <= wb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sDA[orow(r) * LD4 + nt * 16 + li] = sanitize(atm[nt][r]);  // :174
      }
  }
  lds_barrier();

  // ---- 7. dAkk = -(A^T (dA A^T)) . strict -----------------------------------------
  {
    f32x4 aak[NKT];
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt) aak[nt] = z4;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      if (kt >= wb) {   // A[t][m] = 0 for t < m; columns n >= m are masked
        const f32x4 x = colop(sA, LD4, kt * 16, wv * 16);    // A^T rows m, k
#pragma unroll
        for (int nt = 0; nt < NKT; ++nt)
          if (nt <= wb) mma(aak[nt], x, colop(sDA, LD4, kt * 16, nt * 16));
      }
    }
    float* dakk = a.DAKK + (size_t)cid * BT * BT;
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n2 = nt * 16 + li;
        dakk[orow(r) * BT + n2] = n2 < orow(r) ? sanitize(-aak[nt][r]) : 0.f;   // :209
      }
  }
}

// Diagonal-block gradients of one row block, summed exactly for strong decay
// (when more than kMaxDiagExp of log-decay lies between a token and the block's
// 8th, the factors e^{lc - lm}, e^{lm - lc} of gram_bwd's factorisation would
// overflow).  As in the forward's diag_block_exact: for groups of G = 16, 8, 4, 2
// tokens the pairs (i in the upper, j in the lower half of one group) are
// factorised around the group's boundary token b, where both e^{lc_i - lc_b}
// and e^{lc_b - lc_j} are <= 1 for g <= 0, then the diagonal i = j (factor 1).
// Returns, in gram_bwd's token layout (lane li = token I*16 + li, channel
// dt*16 + 4 lg + r of the panel), the diagonal parts of the score gradients wrt
// q (unscaled), b k and k with their factors applied.  Each level's factored
// q, b k, k go into this wave's own rows of the LDS tiles (the caller's rows,
// free at this point; every write is waited for before other lanes read it);
// the operands are loaded again from `rowo` (this lane's token row plus the
// panel's first channel) and the levels run in a loop the compiler keeps
// rolled, so that this rarely taken path adds few registers to gram_bwd.
template <int NDT>
struct DiagGrads {
  f32x4 q[NDT], b[NDT], k[NDT];
};
template <typename TI, typename TG, int NDT>
__device__ __forceinline__ DiagGrads<NDT> diag_grads_exact(
    const TI* __restrict__ q, const TI* __restrict__ k, const TI* __restrict__ b,
    const TG* __restrict__ g, size_t rowo, float scale, int I, float* sAQ, float* sABK,
    float* sKH, int LD1, const float* sDQK, const float* sDKK, int LD2) {
  constexpr int DQ = 4 * NDT;
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int t = I * 16 + li, dblk = I * 16 * LD2 + I * 16;
  DiagGrads<NDT> d;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) d.q[dt] = d.b[dt] = d.k[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int L = 0; L < 5; ++L) {   // L < 4: groups of 16 >> L tokens; L = 4: i = j
    const int G = 16 >> L, half = G / 2;
    const bool upper = (li % G) >= half;
    const int bnd = (li / G) * G + half - 1;   // boundary token of li's group
    float f[DQ];
#pragma unroll
    for (int j = 0; j < NDT; ++j) {   // (NDT = 2: f stays in registers)
      float lc[4], qv[4], kv[4], bv[4];
      load_f<4>(g + rowo + j * 16 + lg * 4, lc);
      load_f<4>(q + rowo + j * 16 + lg * 4, qv);
      load_f<4>(k + rowo + j * 16 + lg * 4, kv);
      load_f<4>(b + rowo + j * 16 + lg * 4, bv);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float c = row_scan16(lc[e]), cb = __shfl(c, bnd, 16);
        // (g > 0 lies outside the domain: the exponent is held below overflow)
        const float fx = L == 4 ? 1.f : __expf(fminf(upper ? c - cb : cb - c, kMaxDiagExp));
        f[4 * j + e] = fx;
        const int o = t * LD1 + j * 16 + lg * 4 + e;
        sAQ[o] = scale * qv[e] * fx;
        sABK[o] = bv[e] * kv[e] * fx;
        sKH[o] = kv[e] * fx;
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    f32x4 mq, mk, cq, ck;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = 4 * lg + e;
      // pair (i = li, j = s) and pair (i = s, j = li) of this level
      const bool pq = L < 4 ? (li / G == s / G) && upper && (s % G < half) : s == li;
      const bool pk = L < 4 ? (li / G == s / G) && (s % G >= half) && !upper : s == li;
      mq[e] = pq ? sDQK[dblk + li * LD2 + s] : 0.f;
      mk[e] = (pq && L < 4) ? sDKK[dblk + li * LD2 + s] : 0.f;
      cq[e] = pk ? sDQK[dblk + s * LD2 + li] : 0.f;
      ck[e] = (pk && L < 4) ? sDKK[dblk + s * LD2 + li] : 0.f;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      f32x4 ke, qe, be;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int o = (I * 16 + 4 * lg + e) * LD1 + dt * 16 + li;
        ke[e] = sKH[o];
        qe[e] = sAQ[o];
        be[e] = sABK[o];
      }
      f32x4 tq = {0.f, 0.f, 0.f, 0.f}, tb = {0.f, 0.f, 0.f, 0.f}, tk = {0.f, 0.f, 0.f, 0.f};
      mma(tq, ke, mq);
      mma(tb, ke, mk);
      mma(tk, qe, cq);
      mma(tk, be, ck);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float fx = f[4 * dt + r];   // this lane's token, channel dt*16 + 4lg + r
        d.q[dt][r] += fx * tq[r];
        d.b[dt][r] += fx * tb[r];
        d.k[dt][r] += fx * tk[r];
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  }
  return d;
}

// ============================================================================
// gram_bwd (B4, with the B3 elementwise tail and B5): gradients of the
// intra-chunk scores
//   Aqk[i,j] = scale sum_d q_i k_j e^{gc_i-gc_j} (j<=i),  Akk[i,j] = sum_d (bk)_i k_j e^{..} (j<i)
// and from them the input gradients.  Off-diagonal 16-row block pairs (I > J) use
// the forward's factorisation around P_J (gc at the end of block J); the MFMA sums
// are formed without their row factors:
//   RQ [i]  = sum_J F_IJ (dAqk_IJ  Khat_J),   dq_g  = scale e^{loc_i} RQ
//   RBK[i]  = sum_J F_IJ (dAkk_IJ  Khat_J),   dbk_g = e^{loc_i} RBK
//   RK [j]  = sum_I F_IJ (scale dAqk_IJ^T AQ_I + dAkk_IJ^T ABK_I),  dk_g = e^{T_J-loc_j} RK
// with loc = in-block cumsum of g, T_J = block sum, F_IJ = exp(sum of T over blocks
// strictly between J and I), Khat = k e^{T-loc}, AQ = q e^{loc}, ABK = b k e^{loc}.
// Every wave does three block pairs per 16-channel slice, so a barrier after each
// slice frees that slice of AQ / ABK / Khat and RQ / RBK / RK take its place in LDS.
// Diagonal blocks, factorised around the block's 8th token as in the forward, run
// first on MFMA, transposed (channel x token) so that their sums arrive in the
// token layout of the chain rule, which adds them.  Then, one lane per token and
// four channels per 16-byte access, the chain rule through the
// exponentials of qg, kg and b k e^gc (gdn2_bwd.py:186-210; dqg, dkg, d(b k e^gc)
// and sum_e dh' h come from bwd_wy, which also forms dv and dw) and the reverse
// cumsum of dgc (gdn2_bwd.py:32-41): DPP suffix sums inside each 16-token block,
// block totals across the waves through LDS.  Wave w owns row block w (BT = 64).
// ============================================================================
template <typename T, typename TG, typename TI = T>
struct GramArgs {
  const TI *q, *k, *b;
  const TG* g;
  const float *DAQK, *DAKK, *SDH, *DQG, *DKG, *DKBD;
  int T_len, H, N;
  float scale;
  TI *dq, *dk, *db;
  TG* dg;
};

// Channels are independent in all of this, so a workgroup takes one chunk and
// one panel of GP = 32 channels (63 KB of LDS: two workgroups per CU, one
// streaming while the other computes).  The panels of a chunk run on one XCD,
// sharing the chunk's dAqk / dAkk tiles in its L2.
constexpr int gram_panel() { return 32; }

// What one gram_bwd launch forms: the fused B4 + B3 tail + B5 (kGramAll), or for
// the stage entry points B3's element-wise tail alone (kGramB3: the score
// gradients taken as zero; wy_dqkg_backward_pallas's dq, dk, db, dgc) or B4 alone
// (kGramB4: the B3 partials taken as zero; intra_backward_pallas), both writing
// dgc per token (no B5) into `dg`.
enum GramMode { kGramAll = 0, kGramB3 = 1, kGramB4 = 2 };

template <typename T, typename TG, int D, typename TI, int GM = kGramAll>
__global__ void __launch_bounds__(256) gram_bwd(GramArgs<T, TG, TI> a) {
  constexpr int BT = 64, NB = 4, GP = gram_panel(), NPN = D / GP, NDT = GP / 16, DQ = GP / 4;
  constexpr int LD1 = GP + 4, LD2 = BT + 4;
  static_assert(D % GP == 0, "panels must tile D");
  __shared__ __align__(16) float sAQ[BT * LD1];    // q e^loc, then RQ, then gq, then dgc sums
  __shared__ __align__(16) float sABK[BT * LD1];   // b k e^loc, then RBK, then gbk
  __shared__ __align__(16) float sKH[BT * LD1];    // k e^{T-loc}, then RK, then gk
  __shared__ __align__(16) float sDQK[BT * LD2];
  __shared__ __align__(16) float sDKK[BT * LD2];
  __shared__ __align__(16) float sTot[NB * GP];
  __shared__ __align__(16) float sETot[NB * GP];   // e^{T_m}, then per-block sums of dgc
  __shared__ __align__(16) float sSkg[NB * GP];    // per-block sums of dkg kg
  __shared__ __align__(16) float sLm[NB * GP];     // in-block cumsum at the block's 8th token
  __shared__ __align__(16) float sB3L[GP];         // B3's dgc at the chunk's last token

  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const UnitPart up = xcd_split(blockIdx.x, gridDim.x, NPN);   // a chunk's panels on one XCD
  const int cid = up.unit, pn = up.part;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  const size_t HD = (size_t)a.H * D;
  const int ch0 = pn * GP;   // first channel of the panel
  const size_t tok0 = ((size_t)bb * a.T_len + (size_t)c * BT) * HD + (size_t)hh * D + ch0;
  auto chan = [&](int x) { return (x / 4) * 16 + lg * 4 + (x % 4); };
  const int I = wv;

  // score gradients, then this lane's g, q, k, b (token t, channels chan(x)), all
  // in flight together; the staged tiles go to LDS first (they arrive first), the
  // cumsum then waits for g alone while q, k, b arrive behind it
  constexpr int SU = BT * BT / 4 / 256;
  const int t = I * 16 + li;
  const size_t rowo = tok0 + (size_t)t * HD;
  f32x4 dqd[NDT], dbd[NDT], dkd[NDT];   // diagonal-block sums, token t, channels chan()
  bool hier = false;   // the diagonal sums come from diag_grads_exact (factors applied)
  // this lane's in-block cumsum of g and q, k, b (token t, channels chan(x)), kept
  // for the chain rule
  float loc[DQ], qv[DQ], kv[DQ], bv[DQ];
  {
    const float* dq = a.DAQK + (size_t)cid * BT * BT;
    const float* dk = a.DAKK + (size_t)cid * BT * BT;
    f32x4 sq[SU], sk[SU];
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int i = tid + 256 * u, r = i / (BT / 4), cc = (i % (BT / 4)) * 4;
      if constexpr (GM == kGramB3) {
        sq[u] = sk[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        sq[u] = load4f(dq + r * BT + cc);
        sk[u] = load4f(dk + r * BT + cc);
      }
    }
#pragma unroll
    for (int j = 0; j < NDT; ++j) load_f<4>(a.g + rowo + j * 16 + lg * 4, &loc[j * 4]);
#pragma unroll
    for (int j = 0; j < NDT; ++j) {
      load_f<4>(a.q + rowo + j * 16 + lg * 4, &qv[j * 4]);
      load_f<4>(a.k + rowo + j * 16 + lg * 4, &kv[j * 4]);
      load_f<4>(a.b + rowo + j * 16 + lg * 4, &bv[j * 4]);
    }
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int i = tid + 256 * u, r = i / (BT / 4), cc = (i % (BT / 4)) * 4;
      *reinterpret_cast<f32x4*>(&sDQK[r * LD2 + cc]) = sq[u];
      *reinterpret_cast<f32x4*>(&sDKK[r * LD2 + cc]) = sk[u];
    }
#pragma unroll
    for (int x = 0; x < DQ; ++x) loc[x] = row_scan16(loc[x]);
    if (li == 15) {
#pragma unroll
      for (int x = 0; x < DQ; ++x) sTot[I * GP + chan(x)] = loc[x];
    }
    if (li == 7) {
#pragma unroll
      for (int x = 0; x < DQ; ++x) sLm[I * GP + chan(x)] = loc[x];
    }
    lds_barrier();
    for (int i = tid; i < NB * GP; i += 256) sETot[i] = __expf(sTot[i]);
    // Diagonal block first, on MFMA, with e^{lc_i - lc_j} = e^{lc_i - lm} e^{lm - lc_j}
    // around the block's 8th token (as the forward's diagonal blocks): this wave's
    // own rows of sAQ, sABK, sKH take QE = scale q e^{loc-lm}, BE = b k e^{loc-lm},
    // KE = k e^{lm-loc} (only this wave reads them), and the products are formed
    // transposed (channel x token), so that lane li holds token li, channels
    // dt*16 + 4lg + r: the layout of the chain rule below, where the row factors
    // are applied.
    bool wide = false;   // a channel's decay across the block exceeds the factors' range
#pragma unroll
    for (int x = 0; x < DQ; ++x) {
      const int ch = chan(x);
      const float lm = sLm[I * GP + ch];
      wide = wide || !(fabsf(loc[x] - lm) <= kMaxDiagExp);
      const float fl = __expf(loc[x] - lm), fr = __expf(lm - loc[x]);
      sAQ[t * LD1 + ch] = a.scale * qv[x] * fl;
      sABK[t * LD1 + ch] = bv[x] * kv[x] * fl;
      sKH[t * LD1 + ch] = kv[x] * fr;
    }
    {
      const int dblk = I * 16 * LD2 + I * 16;
      const f32x4 rq = load4f(&sDQK[dblk + li * LD2 + 4 * lg]);   // row li, cols 4lg + e
      const f32x4 rk = load4f(&sDKK[dblk + li * LD2 + 4 * lg]);
      f32x4 mq, mk, cq, ck;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = 4 * lg + e;
        mq[e] = s <= li ? rq[e] : 0.f;                          // dAqk[li][s], s <= li
        mk[e] = s < li ? rk[e] : 0.f;                           // dAkk[li][s], s < li
        cq[e] = s >= li ? sDQK[dblk + s * LD2 + li] : 0.f;     // dAqk[s][li], s >= li
        ck[e] = s > li ? sDKK[dblk + s * LD2 + li] : 0.f;      // dAkk[s][li], s > li
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        f32x4 ke, qe, be;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int o = (I * 16 + 4 * lg + e) * LD1 + dt * 16 + li;
          ke[e] = sKH[o];
          qe[e] = sAQ[o];
          be[e] = sABK[o];
        }
        dqd[dt] = dbd[dt] = dkd[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        mma(dqd[dt], ke, mq);   // sum_{j <= i} dAqk[i][j] KE_j
        mma(dbd[dt], ke, mk);   // sum_{j < i}  dAkk[i][j] KE_j
        mma(dkd[dt], qe, cq);   // sum_{i >= j} dAqk[i][j] QE_i
        mma(dkd[dt], be, ck);   //  + sum_{i > j} dAkk[i][j] BE_i
      }
    }
    // strong decay: the diagonal parts again, exactly and with their factors
    // applied (the chain rule below then takes them as they are)
    hier = __ballot(wide) != 0;
    if (hier) {
      const DiagGrads<NDT> dg = diag_grads_exact<TI, TG, NDT>(
          a.q, a.k, a.b, a.g, rowo, a.scale, I, sAQ, sABK, sKH, LD1, sDQK, sDKK, LD2);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        dqd[dt] = dg.q[dt];
        dbd[dt] = dg.b[dt];
        dkd[dt] = dg.k[dt];
      }
    }
    // then the off-diagonal operands in the same rows (in order within the wave)
#pragma unroll
    for (int x = 0; x < DQ; ++x) {
      const int ch = chan(x);
      const float el = __expf(loc[x]);
      sAQ[t * LD1 + ch] = qv[x] * el;
      sABK[t * LD1 + ch] = bv[x] * kv[x] * el;
      sKH[t * LD1 + ch] = kv[x] * __expf(sTot[I * GP + ch] - loc[x]);
    }
  }
  // operands of the chain rule below, loaded now so that they arrive while the
  // products run
  const size_t wrow_t = ((size_t)cid * BT + t) * D + ch0;
  f32x4 pdqg[NDT], pdkg[NDT], pdkbd[NDT], psdh[NDT];
#pragma unroll
  for (int j = 0; j < NDT; ++j) {
    const int c0 = j * 16 + lg * 4;
    if constexpr (GM == kGramB4) {
      pdqg[j] = pdkg[j] = pdkbd[j] = psdh[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      pdqg[j] = load4f(a.DQG + wrow_t + c0);
      pdkg[j] = load4f(a.DKG + wrow_t + c0);
      pdkbd[j] = load4f(a.DKBD + wrow_t + c0);
      psdh[j] = load4f(a.SDH + (size_t)cid * D + ch0 + c0);
    }
  }
  lds_barrier();

  // ---- off-diagonal pairs on MFMA --------------------------------------------
  // The reference accumulates B4 over pairs of two 32-token sub-blocks S0 = {blocks
  // 0, 1}, S1 = {2, 3}, in the order (S0,S0), (S1,S0), (S1,S1), clipping every
  // accumulator after each pair (_clip_acc, gdn2_bwd.py:287-328).  The sums that
  // cross the sub-blocks are therefore kept apart: the rows of S1 against J in S0
  // (cq, cb) and the columns of S0 against I' in S1 (ck); the rest of each sum
  // belongs to the row block's own sub-block pair.
  constexpr int SB = NB / 2;   // row blocks per sub-block
  const bool rowx = I >= SB;   // this block's rows have a (S1,S0) part, its columns none
  f32x4 cq[NDT], cb[NDT];      // (S1,S0) row sums of block I in S1; ck in cq for S0
  // Compiled once per row block (the wave's block is fixed), so every pair loop
  // has constant bounds, unrolls, and picks its accumulator at compile time.
  auto offdiag = [&](auto Ic) __attribute__((always_inline)) {
    constexpr int IC = decltype(Ic)::value;
    constexpr bool RX = IC >= SB;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int dcol = dt * 16 + li;
      // rows of block IC against J < IC (J from IC-1 down): the blocks of IC's own
      // sub-block, then (rows of S1) those of S0
      f32x4 aq = {0.f, 0.f, 0.f, 0.f}, ab = {0.f, 0.f, 0.f, 0.f};
      cq[dt] = cb[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      float F = 1.f;
#pragma unroll
      for (int J = IC - 1; J >= 0; --J) {
        f32x4 y, tq = {0.f, 0.f, 0.f, 0.f}, tk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = sKH[(J * 16 + 4 * lg + e) * LD1 + dcol];
        mma(tq, load4f(&sDQK[(IC * 16 + li) * LD2 + J * 16 + 4 * lg]), y);
        mma(tk, load4f(&sDKK[(IC * 16 + li) * LD2 + J * 16 + 4 * lg]), y);
        f32x4& sq = (RX && J < SB) ? cq[dt] : aq;
        f32x4& sb = (RX && J < SB) ? cb[dt] : ab;
#pragma unroll
        for (int r = 0; r < 4; ++r) { sq[r] += F * tq[r]; sb[r] += F * tk[r]; }
        if (J > 0) F *= sETot[J * GP + dcol];
      }
      // rows of block IC (as the column block) against I' > IC: IC's own
      // sub-block, then (columns of S0) S1's
      f32x4 akk = {0.f, 0.f, 0.f, 0.f};
      F = 1.f;
#pragma unroll
      for (int Ip = IC + 1; Ip < NB; ++Ip) {
        f32x4 xq, xk, yq, yk, t1 = {0.f, 0.f, 0.f, 0.f}, t2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = Ip * 16 + 4 * lg + e;
          xq[e] = sDQK[i * LD2 + IC * 16 + li];
          xk[e] = sDKK[i * LD2 + IC * 16 + li];
          yq[e] = sAQ[i * LD1 + dcol];
          yk[e] = sABK[i * LD1 + dcol];
        }
        mma(t1, xq, yq);
        mma(t2, xk, yk);
        f32x4& sk = (!RX && Ip >= SB) ? cq[dt] : akk;
#pragma unroll
        for (int r = 0; r < 4; ++r) sk[r] += F * (a.scale * t1[r] + t2[r]);
        if (Ip + 1 < NB) F *= sETot[Ip * GP + dcol];
      }
      lds_barrier();  // every wave is done with channel slice dt of sAQ, sABK, sKH, sETot
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = (IC * 16 + 4 * lg + r) * LD1 + dcol;
        sAQ[o] = aq[r];
        sABK[o] = ab[r];
        sKH[o] = akk[r];
      }
    }
  };
  static_assert(NB == 4, "one specialisation per row block");
  switch (I) {   // wave-uniform
    case 0: offdiag(std::integral_constant<int, 0>{}); break;
    case 1: offdiag(std::integral_constant<int, 1>{}); break;
    case 2: offdiag(std::integral_constant<int, 2>{}); break;
    default: offdiag(std::integral_constant<int, 3>{}); break;
  }
  // The score-gradient tiles are no longer read (the last barrier above): the
  // cross sums go into their space, in the same [token][channel] layout, rows of
  // this wave's own block only
  float* const sXQ = sDQK;   // cq: (S1,S0) rows of dAqk (S1) / (S1,S0) columns (S0)
  float* const sXB = sDKK;   // cb: (S1,S0) rows of dAkk (S1)
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = (I * 16 + 4 * lg + r) * LD1 + dt * 16 + li;
      sXQ[o] = cq[dt][r];
      if (rowx) sXB[o] = cb[dt][r];
    }

  // ---- chain rule, lane = token t of block I, channels chan(x) -----------------
  // (gdn2_bwd.py:186-210; dqg, dkg, dkbd come from bwd_wy).  First the score
  // gradients wrt q, b k, k: the off-diagonal sums (wave I reads its own rows,
  // written by its own lanes above) with their row factors, plus the diagonal
  // block's.  dgc is summed from each token to the block end by a row scan; the
  // block totals cross the waves through LDS.
#pragma unroll
  for (int j = 0; j < NDT; ++j) {
    const int c0 = j * 16 + lg * 4;
    const f32x4 dqg = pdqg[j], dkg = pdkg[j], dkbd = pdkbd[j];
    const f32x4 rq = load4f(&sAQ[t * LD1 + c0]), rbk = load4f(&sABK[t * LD1 + c0]),
                rk = load4f(&sKH[t * LD1 + c0]), lm = load4f(&sLm[I * GP + c0]);
    const f32x4 xrq = load4f(&sXQ[t * LD1 + c0]);
    const f32x4 xrb = rowx ? load4f(&sXB[t * LD1 + c0]) : f32x4{0.f, 0.f, 0.f, 0.f};
    // channel c0 + e is x = 4j + e of the start's registers
    const float* const lc = &loc[4 * j];
    const float* const xq = &qv[4 * j];
    const float* const xk = &kv[4 * j];
    const float* const xb = &bv[4 * j];
    f32x4 pre = {0.f, 0.f, 0.f, 0.f}, gl = {0.f, 0.f, 0.f, 0.f}, totI;
#pragma unroll
    for (int m = 0; m < NB; ++m) {
      const f32x4 tm = load4f(&sTot[m * GP + c0]);
      if (m == I) totI = tm;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gl[e] += tm[e];
        pre[e] += m < I ? tm[e] : 0.f;
      }
    }
    // B4's gradients wrt q, b k, k of this token: gq, gbk, gk from its own sub-block
    // pair, xq, xbk (rows of S1) or xk (columns of S0) from the (S1,S0) pair
    f32x4 gq, gbk, gk, xgq, xgb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float fl = __expf(lc[e] - lm[e]), fr = __expf(lm[e] - lc[e]);
      const float el = __expf(lc[e]), ek = __expf(totI[e] - lc[e]);
      gq[e] = a.scale * (el * rq[e] + (hier ? dqd[j][e] : fl * dqd[j][e]));
      gbk[e] = el * rbk[e] + (hier ? dbd[j][e] : fl * dbd[j][e]);
      gk[e] = ek * rk[e] + (hier ? dkd[j][e] : fr * dkd[j][e]);
      xgq[e] = (rowx ? a.scale * el : ek) * xrq[e];
      xgb[e] = el * xrb[e];
    }
    // B4's accumulators in the pair order of gdn2_bwd.py:287-328, each clipped
    // after its pair: rows of S1 take (S1,S0) then (S1,S1); columns of S0 take
    // (S0,S0) then (S1,S0); dgc takes a pair's row terms, then its column terms.
    // Those intermediate clips change nothing unless a partial sum reaches the
    // clip: a wave whose partial sums all stay inside (the input domain) takes the
    // totals directly.
    f32x4 aq4, ab4, ak4, ag4;
    bool inside = true;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float bk = xb[e] * xk[e];
      const float tq = rowx ? gq[e] + xgq[e] : gq[e];
      const float tb = rowx ? gbk[e] + xgb[e] : gbk[e];
      const float tk = rowx ? gk[e] : gk[e] + xgq[e];
      const float gi = xq[e] * tq + bk * tb;           // all row terms of dgc
      const float in = !rowx ? gi : xq[e] * xgq[e] + bk * xgb[e];
      const float p1 = rowx ? xgq[e] : gk[e] + xgq[e], p2 = rowx ? xgb[e] : gi - xk[e] * gk[e];
      inside = inside && fabsf(p1) <= g_clip && fabsf(p2) <= g_clip && fabsf(in) <= g_clip &&
               fabsf(gi) <= g_clip && fabsf(tb) <= g_clip && fabsf(gk[e]) <= g_clip;
      aq4[e] = tq;
      ab4[e] = tb;
      ak4[e] = tk;
      ag4[e] = gi - xk[e] * tk;
    }
    if (__ballot(!inside) != 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float bk = xb[e] * xk[e];
        if (rowx) {
          aq4[e] = sanitize(sanitize(xgq[e]) + gq[e]);
          ab4[e] = sanitize(sanitize(xgb[e]) + gbk[e]);
          ak4[e] = sanitize(gk[e]);
          const float gi0 = xq[e] * xgq[e] + bk * xgb[e];
          const float gi1 = xq[e] * gq[e] + bk * gbk[e];
          ag4[e] = sanitize(sanitize(sanitize(gi0) + gi1) - xk[e] * gk[e]);
        } else {
          aq4[e] = sanitize(gq[e]);
          ab4[e] = sanitize(gbk[e]);
          ak4[e] = sanitize(sanitize(gk[e]) + xgq[e]);
          const float gi0 = xq[e] * gq[e] + bk * gbk[e];
          ag4[e] = sanitize(sanitize(sanitize(gi0) - xk[e] * gk[e]) - xk[e] * xgq[e]);
        }
      }
    }
    f32x4 odq, odk, odb, suf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float gc = pre[e] + lc[e];
      const float eg = __expf(gc), ekg = __expf(gl[e] - gc);
      const float kgv = xk[e] * ekg;
      // B3's and B4's outputs are sanitized as each kernel's output, then their
      // sum (gdn2_bwd.py:212-218, 330-339; gdn2_pipeline.py:121-133)
      odq[e] = sanitize(sanitize(dqg[e] * eg) + sanitize(aq4[e]));
      odk[e] = sanitize(sanitize(dkbd[e] * xb[e] * eg + dkg[e] * ekg) +
                        sanitize(ak4[e] + ab4[e] * xb[e]));
      odb[e] = sanitize(sanitize(dkbd[e] * xk[e] * eg) + sanitize(ab4[e] * xk[e]));
      const float dgc3 = dkbd[e] * xb[e] * xk[e] * eg + dqg[e] * xq[e] * eg - dkg[e] * kgv;
      const float dgc4 = ag4[e];
      // the last token's B3 part still lacks the g_last terms: kept for the end
      if (I == NB - 1 && li == 15) sB3L[c0 + e] = dgc3;
      if constexpr (GM == kGramAll) {
        suf[e] = row_suffix16(sanitize(dgc3) + sanitize(dgc4));
      } else {   // dgc per token (one of the two parts is zero)
        suf[e] = sanitize(dgc3) + sanitize(dgc4);
      }
      const float skg = row_suffix16(dkg[e] * kgv);   // lane 0: the block's sum
      if (li == 0) {
        sETot[I * GP + c0 + e] = suf[e];
        sSkg[I * GP + c0 + e] = skg;
      }
    }
    if constexpr (GM != kGramAll) store4(a.dg + rowo + c0, suf);
    store4(&sAQ[t * LD1 + c0], suf);   // in place of gq, read by this lane only
    store4(a.dq + rowo + c0, odq);
    store4(a.dk + rowo + c0, odk);
    store4(a.db + rowo + c0, odb);
  }
  lds_barrier();
  // dg[t] = sum_{s >= t} dgc[s], where the chunk's last token also carries
  // dgl = sum_t dkg kg + e^{gl} sum_e dh' h (gdn2_bwd.py:196-201) inside its B3
  // part: that part was summed as sanitize(b3), and becomes sanitize(b3 + dgl)
  // -- exactly b3 + dgl whenever neither saturates
#pragma unroll
  for (int j = 0; j < NDT; ++j) {
    const int c0 = j * 16 + lg * 4;
    const f32x4 sdh = psdh[j], b3l = load4f(&sB3L[c0]);
    f32x4 gl = {0.f, 0.f, 0.f, 0.f}, skg = {0.f, 0.f, 0.f, 0.f}, later = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < NB; ++m) {
      const f32x4 tm = load4f(&sTot[m * GP + c0]), sk = load4f(&sSkg[m * GP + c0]),
                  bt = load4f(&sETot[m * GP + c0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gl[e] += tm[e];
        skg[e] += sk[e];
        later[e] += m > I ? bt[e] : 0.f;
      }
    }
    const f32x4 suf = load4f(&sAQ[t * LD1 + c0]);
    f32x4 odg;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float dgl = skg[e] + __expf(gl[e]) * sdh[e];
      const float b3 = b3l[e], b3g = b3 + dgl;
      if constexpr (GM == kGramAll) {
        const float corr = (fabsf(b3) < g_clip && fabsf(b3g) < g_clip)
                               ? dgl : sanitize(b3g) - sanitize(b3);
        odg[e] = sanitize(suf[e] + later[e] + corr);
      } else {   // the last token: B3's dgc with the g_last terms (gdn2_bwd.py:199-201)
        odg[e] = sanitize(b3g) + (suf[e] - sanitize(b3));
      }
    }
    if constexpr (GM == kGramAll) store4(a.dg + rowo + c0, odg);
    else if (t == BT - 1) store4(a.dg + rowo + c0, odg);
  }
}

// ============================================================================
// bwd_wy_wide (B3 at D = 256, chunk 64): the products of bwd_wy with the D x D
// and BT x D operands streamed through LDS in slices, one workgroup of eight
// waves per chunk.  Wave (rb, hf) owns the 16-token row block rb and half hf of
// every product's output column tiles.
//   1-2. e-slices of 32: h^T and dh'^T rows [e][d] staged together; dqg, dW
//        (both against h) and dkg (against dh') accumulate over the slices;
//        sum_e dh' h is formed from the staged registers.  dW then sits whole in
//        LDS (R_W, [t][d]).
//   3.   d-slices of 64: b k e^{gc} and w v of the slice's channels into LDS
//        ([s][d]); dA accumulates dW (b k e^gc)^T + dv_new (w v)^T.
//   4.   A and dv_new^T staged: d(bke^gc) = A^T dW, d(wv) = A^T dv_new -> dv, dw.
//   5.   dA A^T and dAkk = -(A^T (dA A^T)) . strict, as in bwd_wy.
// LDS: R_S 68 KB (the slices, then dv_new^T, then dA / dA A^T), R_W 65 KB, A 17 KB.
// ============================================================================
template <typename T, typename TG, typename TI>
__global__ void __launch_bounds__(512) bwd_wy_wide(WyArgs<T, TG, TI> a) {
  constexpr int BT = 64, D = 256, NB = BT / 16, NKT = BT / 16, NT = 512;
  constexpr int HDT = D / 32;                  // output column tiles per wave (half of D/16)
  constexpr int HKT = NKT / 2;                 // token column tiles per wave
  constexpr int ES = 32, LDE = D + 4;          // e-slices of phases 1-2: [ES][D] x 2
  constexpr int DS = 64, LDD = DS + 4;         // d-slices of phase 3: [BT][DS] x 2
  constexpr int LDV = BT + 4, LDW = D + 4, LDA = BT + 4;
  constexpr int RS = (2 * ES * LDE > D * LDV) ? 2 * ES * LDE : D * LDV;
  static_assert(2 * BT * LDD <= RS && BT * LDA <= RS, "slices must fit R_S");
  constexpr int BF = sizeof(T) == 2;
  __shared__ __align__(16) float sS[RS];
  __shared__ __align__(16) float sW[BT * LDW];
  __shared__ __align__(16) float sA[BT * LDA];
  __shared__ __align__(16) float sTot[NB * DS];
  __shared__ __align__(16) float sSdh[D];
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rb = wv & 3, hf = wv >> 2;
  const int cid = blockIdx.x;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  const size_t HD = (size_t)a.H * D;
  const size_t tok0 = ((size_t)bb * a.T_len + (size_t)c * BT) * HD + (size_t)hh * D;
  const int t = rb * 16 + li;                  // this lane's row for row operands
  const int tp = BF ? kpos<bf16_t>(t) : t;     // stored column of token t (v_new^T)
  // Barriers order LDS data only: no wave reads global memory another wave of
  // this workgroup wrote.
  if (tid < D) sSdh[tid] = 0.f;

  auto rowop = [&](const float* base, int ld, int r0, int k0) __attribute__((always_inline)) {
    return load4f(&base[(r0 + li) * ld + k0 + 4 * lg]);
  };
  auto colop = [&](const float* base, int ld, int k0, int c0) __attribute__((always_inline)) {
    f32x4 y;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = base[(k0 + 4 * lg + r) * ld + c0 + li];
    return y;
  };
  auto orow = [&](int r) { return rb * 16 + 4 * lg + r; };
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  // dv_new rows t, k = e (dv_new^T [e][t] read across rows)
  auto dvn_op = [&](int e0) __attribute__((always_inline)) {
    f32x4 x;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = a.DVNT[((size_t)cid * D + e0 + 4 * lg + r) * BT + t];
    return x;
  };

  // ---- 1-2. dqg = scale do h^T, dW = -dv_new h^T, dkg = v_new dh'^T ----------------
  const GMat mH{a.HT, BF, D, 0, BF};
  const GMat mDH{a.DHT, 0, D, 0, 0};
  const GMat mA{a.A, 0, BT, 0, 0};
  float* sH = sS;                 // h^T slice [ES][D]
  float* sDH = sS + ES * LDE;     // dh'^T slice [ES][D]
  f32x4 aq[HDT], aw[HDT], ak[HDT];
#pragma unroll
  for (int n = 0; n < HDT; ++n) aq[n] = aw[n] = ak[n] = z4;
  float part[4] = {0.f, 0.f, 0.f, 0.f};   // sum_e dh' h, column group tid mod D/4
  {
    Staged sa;
    stage_load<NT>(sa, mA, (size_t)cid * BT * BT, BT, BT, tid);
    stage_store<NT>(sA, LDA, sa, mA, BT, BT, 0, 0, false, tid);
  }
  for (int es = 0; es < D / ES; ++es) {
    const int e0 = es * ES;
    Staged sh, sd;
    stage_load<NT>(sh, mH, (size_t)cid * D * D + (size_t)e0 * D, ES, D, tid);
    stage_load<NT>(sd, mDH, (size_t)cid * D * D + (size_t)e0 * D, ES, D, tid);
    f32x4 xdo[ES / 16], xdv[ES / 16], xvn[ES / 16];
#pragma unroll
    for (int kk = 0; kk < ES / 16; ++kk) {
      xdo[kk] = load4f(a.dout + tok0 + (size_t)t * HD + e0 + kk * 16 + 4 * lg);
      xdv[kk] = dvn_op(e0 + kk * 16);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        xvn[kk][r] = to_f(a.VnT[((size_t)cid * D + e0 + kk * 16 + 4 * lg + r) * BT + tp]);
    }
    static_assert(NT % (D / 4) == 0, "column group must stay fixed over the pieces");
#pragma unroll
    for (int u = 0; u < ES * D / 4 / NT; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) part[e] += sd.v[u][e] * sh.v[u][e];
    if (es > 0) lds_barrier();   // the previous slice is read
    stage_store<NT>(sH, LDE, sh, mH, ES, D, 0, 0, false, tid);
    stage_store<NT>(sDH, LDE, sd, mDH, ES, D, 0, 0, false, tid);
    lds_barrier();
#pragma unroll
    for (int kk = 0; kk < ES / 16; ++kk)
#pragma unroll
      for (int n = 0; n < HDT; ++n) {
        const int c0 = (hf * HDT + n) * 16;
        const f32x4 y = colop(sH, LDE, kk * 16, c0);    // h[d][e] as (n = d, k = e)
        mma(aq[n], xdo[kk], y);
        mma(aw[n], xdv[kk], y);
        mma(ak[n], xvn[kk], colop(sDH, LDE, kk * 16, c0));
      }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) atomicAdd(&sSdh[(tid % (D / 4)) * 4 + e], part[e]);
  {
    float* dqg = a.DQG + (size_t)cid * BT * D;
    float* dkg = a.DKG + (size_t)cid * BT * D;
#pragma unroll
    for (int n = 0; n < HDT; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = (hf * HDT + n) * 16 + li;
        dqg[orow(r) * D + col] = a.scale * aq[n][r];
        dkg[orow(r) * D + col] = ak[n][r];
        sW[orow(r) * LDW + col] = -aw[n][r];
      }
  }
  lds_barrier();   // dW and sum_e dh' h complete; the e-slices are read
  if (tid < D) a.SDH[(size_t)cid * D + tid] = sSdh[tid];

  // ---- 3. dA = (dW (b k e^gc)^T + dv_new (w v)^T) . strict, over d-slices ---------
  // lane (li, lg): token s = t; channels d0 + 32 hf + 16 j + 4 lg + e of the slice
  float* sK = sS;                 // b k e^gc [s][DS]
  float* sV = sS + BT * LDD;      // w v [s][DS]
  f32x4 ada[HKT];
#pragma unroll
  for (int n = 0; n < HKT; ++n) ada[n] = z4;
  for (int ds = 0; ds < D / DS; ++ds) {
    const int d0 = ds * DS;
    float loc[2][4], bk[2][4];
    {
      const size_t row = tok0 + (size_t)t * HD;
      float gv[2][4], bv[2][4], kv[2][4], wvv[2][4], vv[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const size_t o = row + d0 + hf * 32 + j * 16 + 4 * lg;
        load_f<4>(a.g + o, gv[j]);
        load_f<4>(a.b + o, bv[j]);
        load_f<4>(a.k + o, kv[j]);
        load_f<4>(a.w + o, wvv[j]);
        load_f<4>(a.v + o, vv[j]);
      }
      lds_barrier();   // the previous slice's b k e^gc, w v and sums are read
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cl = hf * 32 + j * 16 + 4 * lg;   // channel within the slice
        f32x4 wvo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          loc[j][e] = row_scan16(gv[j][e]);
          bk[j][e] = bv[j][e] * kv[j][e];
          wvo[e] = wvv[j][e] * vv[j][e];
        }
        *reinterpret_cast<f32x4*>(&sV[t * LDD + cl]) = wvo;
        if (li == 15) {
#pragma unroll
          for (int e = 0; e < 4; ++e) sTot[rb * DS + cl + e] = loc[j][e];
        }
      }
    }
    lds_barrier();
#pragma unroll
    for (int m = 0; m < NB - 1; ++m) {
      if (m < rb) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const f32x4 tv = load4f(&sTot[m * DS + hf * 32 + j * 16 + 4 * lg]);
#pragma unroll
          for (int e = 0; e < 4; ++e) loc[j][e] += tv[e];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 kb;
#pragma unroll
      for (int e = 0; e < 4; ++e) kb[e] = bk[j][e] * __expf(loc[j][e]);
      *reinterpret_cast<f32x4*>(&sK[t * LDD + hf * 32 + j * 16 + 4 * lg]) = kb;
    }
    lds_barrier();
#pragma unroll
    for (int kg = 0; kg < DS / 16; ++kg) {
      const f32x4 x1 = rowop(sW, LDW, rb * 16, d0 + kg * 16);   // dW rows, k = d
      const f32x4 x2 = dvn_op(d0 + kg * 16);                    // dv_new rows, k = e
#pragma unroll
      for (int n = 0; n < HKT; ++n) {
        if (hf * HKT + n <= rb) {   // dA is strictly lower: blocks s > t are masked
          const int s0 = (hf * HKT + n) * 16;
          mma(ada[n], x1, rowop(sK, LDD, s0, kg * 16));
          mma(ada[n], x2, rowop(sV, LDD, s0, kg * 16));
        }
      }
    }
  }
  // dA . strict (gdn2_bwd.py:168), kept in registers until step 5
#pragma unroll
  for (int n = 0; n < HKT; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int s2 = (hf * HKT + n) * 16 + li;
      ada[n][r] = s2 < orow(r) ? sanitize(ada[n][r]) : 0.f;
    }

  // ---- 4. d(bke^gc) = A^T dW, d(wv) = A^T dv_new -> dv, dw --------------------------
  const GMat mDV{a.DVNT, 0, BT, 0, 0};
  {
    Staged sv;
    stage_load<NT>(sv, mDV, (size_t)cid * D * BT, D, BT, tid);
    lds_barrier();   // the last d-slice is read
    stage_store<NT>(sS, LDV, sv, mDV, D, BT, 0, 0, false, tid);
  }
  lds_barrier();
  {
    f32x4 akb[HDT], awv[HDT];
#pragma unroll
    for (int n = 0; n < HDT; ++n) akb[n] = awv[n] = z4;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      if (kt < rb) continue;   // A[t][m] = 0 for t < m
      const f32x4 x = colop(sA, LDA, kt * 16, rb * 16);   // A^T rows m, k = t
#pragma unroll
      for (int n = 0; n < HDT; ++n) {
        const int c0 = (hf * HDT + n) * 16;
        mma(akb[n], x, colop(sW, LDW, kt * 16, c0));   // dW[t][d] as (n = d, k = t)
        mma(awv[n], x, rowop(sS, LDV, c0, kt * 16));   // dv_new^T[e][t]
      }
    }
    float* dkbd = a.DKBD + (size_t)cid * BT * D;
#pragma unroll
    for (int n = 0; n < HDT; ++n) {
      float wl[4], vl[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t o = tok0 + (size_t)orow(r) * HD + (hf * HDT + n) * 16 + li;
        wl[r] = to_f(a.w[o]);
        vl[r] = to_f(a.v[o]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = (hf * HDT + n) * 16 + li;
        const size_t o = tok0 + (size_t)orow(r) * HD + col;
        dkbd[orow(r) * D + col] = akb[n][r];
        a.dv[o] = from_f<TI>(sanitize(awv[n][r] * wl[r]));
        a.dw[o] = from_f<TI>(sanitize(awv[n][r] * vl[r]));
      }
    }
  }
  lds_barrier();   // dv_new^T is read

  // ---- 5. dA A^T, dAkk = -(A^T (dA A^T)) . strict -----------------------------------
  float* sDA = sS;   // dA, then dA A^T [t][s]
#pragma unroll
  for (int n = 0; n < HKT; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) sDA[orow(r) * LDA + (hf * HKT + n) * 16 + li] = ada[n][r];
  lds_barrier();
  {
    f32x4 atm[HKT];
#pragma unroll
    for (int n = 0; n < HKT; ++n) atm[n] = z4;
#pragma unroll
    // dA[t][s] = 0 for s > t; only the columns n < m <= t of dA A^T enter dAkk,
    // so columns past the own row block are not formed (they keep dA's zeros)
    for (int ks = 0; ks < NKT; ++ks) {
      if (ks > rb) continue;
      const f32x4 x = rowop(sDA, LDA, rb * 16, ks * 16);    // dA rows t, k = s
#pragma unroll
      for (int n = 0; n < HKT; ++n)
        if (hf * HKT + n <= rb)
          mma(atm[n], x, rowop(sA, LDA, (hf * HKT + n) * 16, ks * 16));   // A[n][s]
    }
    lds_barrier();   // both waves of the row block have read its rows of dA
#pragma unroll
    for (int n = 0; n < HKT; ++n)
      if (hf * HKT + n <= rb) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sDA[orow(r) * LDA + (hf * HKT + n) * 16 + li] = sanitize(atm[n][r]);   // :174
      }
  }
  lds_barrier();
  {
    f32x4 aak[HKT];
#pragma unroll
    for (int n = 0; n < HKT; ++n) aak[n] = z4;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      if (kt < rb) continue;   // A[t][m] = 0 for t < m; columns n >= m are masked
      const f32x4 x = colop(sA, LDA, kt * 16, rb * 16);    // A^T rows m, k
#pragma unroll
      for (int n = 0; n < HKT; ++n)
        if (hf * HKT + n <= rb) mma(aak[n], x, colop(sDA, LDA, kt * 16, (hf * HKT + n) * 16));
    }
    float* dakk = a.DAKK + (size_t)cid * BT * BT;
#pragma unroll
    for (int n = 0; n < HKT; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n2 = (hf * HKT + n) * 16 + li;
        dakk[orow(r) * BT + n2] = n2 < orow(r) ? sanitize(-aak[n][r]) : 0.f;   // :209
      }
  }
}

// ============================================================================
// Host side
// ============================================================================
size_t bwd_ws_bytes(size_t nchunks, int BT, int D, size_t) {
  return BT == 64 ? bwd_layout(nchunks, BT, D).total : 0;
}


// The backward at D = 256 (chunk 64): B2 by bwd_b2 (its tiles still fit LDS,
// 136 KB), B3 by bwd_wy_wide (the D x D operands streamed in slices: the D = 128
// kernel would need 266 KB), the reverse scan (single-buffered at this width) and
// gram_bwd (32-channel panels) as at D <= 128.  Launch marks: before B2, after B2,
// after the scan, after B3, after gram_bwd (as the fused path).
template <typename T, typename TG, typename TI>
hipError_t launch_bwd_wide(hipStream_t st, int B, int T_len, int H, const void* q,
                           const void* k, const void* v, const void* w, const void* b,
                           const void* g, float scale, const float* dout,
                           const float* dh_final, void* dq, void* dk, void* dv, void* dw,
                           void* db, void* dg, float* dh0, const char* fws, char* ws,
                           const int* cu_chunks, int nseq) {
  constexpr int BT = 64, D = 256;
  const int N = T_len / BT;
  const size_t NC = (size_t)B * H * N;
  const FwdLayout F = fwd_layout(NC, BT, D, sizeof(T));
  const BwdLayout L = bwd_layout(NC, BT, D);
  auto buf = [&](BwdBuf i) { return reinterpret_cast<float*>(ws + L.off[i]); };
  const void* fVnT = fws + F.VnT;
  const void* fHT = fws + F.HT;
  const float* fA = reinterpret_cast<const float*>(fws + F.A);
  launch_mark(st);
  if (NC > 0) {
    // B2: dAqk = (do v_new^T) . causal, dvp^T = (Aqk^T do)^T, qdot = scale (qg^T do)^T
    B2Args<T> ba{dout, (const T*)fVnT, (const T*)(fws + F.Aqk), (const T*)(fws + F.Qg), T_len,
                 H, N, scale, buf(B_DAQK), buf(B_DVPT), buf(B_QDOT)};
    hipLaunchKernelGGL((bwd_b2<T, D>), dim3(NC), dim3(64 * b2_waves(D)), 0, st, ba);
    launch_mark(st);
  }
  BStateArgs<T> sa{(const T*)(fws + F.W), (const T*)(fws + F.KgT),
                   reinterpret_cast<const float*>(fws + F.GL), buf(B_DVPT), buf(B_QDOT),
                   dh_final, N, buf(B_DHT), buf(B_DVNT), dh0, cu_chunks, cu_chunks ? nseq : 1, H};
  constexpr int BW = 2, BK = bstate_ksplit<T, D>(), BP = BK > 1 ? 4 : 2;
  const size_t units = cu_chunks ? (size_t)H * nseq : (size_t)B * H;
  hipLaunchKernelGGL((bwd_state<T, BT, D, BW, BP, BK>), dim3(units * (D / (16 * BW))),
                     dim3(64 * (BW * BK + BP)), 0, st, sa);
  launch_mark(st);
  if (NC > 0) {
    // B3 (gdn2_bwd.py:126-210): one fused kernel with the D x D operands streamed
    WyArgs<T, TG, TI> wa{(const TI*)k, (const TI*)w,   (const TI*)v, (const TI*)b, (const TG*)g,
                         dout,         (const T*)fHT,   (const T*)fVnT,
                         fA,           buf(B_DHT),      buf(B_DVNT),
                         T_len, H, N, scale, buf(B_DQG), buf(B_DKG), buf(B_DKBD),
                         buf(B_DAKK), buf(B_SDH), (TI*)dv, (TI*)dw};
    hipLaunchKernelGGL((bwd_wy_wide<T, TG, TI>), dim3(NC), dim3(512), 0, st, wa);
    launch_mark(st);
    // B4 + B3 element-wise tail + B5
    GramArgs<T, TG, TI> gr{(const TI*)q, (const TI*)k, (const TI*)b, (const TG*)g,
                           buf(B_DAQK),  buf(B_DAKK),  buf(B_SDH),   buf(B_DQG),
                           buf(B_DKG),   buf(B_DKBD),  T_len,        H,
                           N,            scale,        (TI*)dq,      (TI*)dk,
                           (TI*)db,      (TG*)dg};
    hipLaunchKernelGGL((gram_bwd<T, TG, D, TI>), dim3(NC * (D / gram_panel())), dim3(256), 0,
                       st, gr);
    launch_mark(st);
  }
  return hipGetLastError();
}

template <typename T, typename TG, int BT, int D, typename TI>
hipError_t launch_bwd(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                      const void* v, const void* w, const void* b, const void* g,
                      const float* h0, float scale, const float* dout, const float* dh_final,
                      void* dq, void* dk, void* dv, void* dw, void* db, void* dg, float* dh0,
                      const char* fws, char* ws, const int* cu_chunks, int nseq) {
  if constexpr (BT != 64) {
    return hipErrorNotSupported;
  } else if constexpr (D > 128) {
    (void)h0;
    return launch_bwd_wide<T, TG, TI>(st, B, T_len, H, q, k, v, w, b, g, scale, dout, dh_final,
                                      dq, dk, dv, dw, db, dg, dh0, fws, ws, cu_chunks, nseq);
  } else {
    (void)h0;
    const int N = T_len / BT;
    const size_t NC = (size_t)B * H * N;
    const FwdLayout F = fwd_layout(NC, BT, D, sizeof(T));
    const BwdLayout L = bwd_layout(NC, BT, D);
    auto buf = [&](BwdBuf i) { return reinterpret_cast<float*>(ws + L.off[i]); };
    const void* fW = fws + F.W;
    const void* fKgT = fws + F.KgT;
    const void* fQg = fws + F.Qg;
    const void* fAqk = fws + F.Aqk;
    const float* fGL = reinterpret_cast<const float*>(fws + F.GL);
    const void* fHT = fws + F.HT;
    const void* fVnT = fws + F.VnT;
    const void* fA = fws + F.A;
    launch_mark(st);
    if (NC == 0) {
      // empty sequence: dh0 = sanitize(dh_final) (or zeros) via the state kernel
    }
    // B2: dAqk, Aqk^T do, scale qg^T do
    if (NC > 0) {
      B2Args<T> ba{dout, (const T*)fVnT, (const T*)fAqk, (const T*)fQg, T_len, H, N, scale,
                   buf(B_DAQK), buf(B_DVPT), buf(B_QDOT)};
      hipLaunchKernelGGL((bwd_b2<T, D>), dim3(NC), dim3(64 * b2_waves(D)), 0, st, ba);
      launch_mark(st);
    }
    // B1: reverse state scan
    // variable-length batch (B = 1): one scan unit per (head, sequence)
    BStateArgs<T> sa{(const T*)fW, (const T*)fKgT, fGL, buf(B_DVPT), buf(B_QDOT), dh_final, N,
                     buf(B_DHT), buf(B_DVNT), dh0, cu_chunks, cu_chunks ? nseq : 1, H};
    constexpr int BW = 2;                       // column slices per scan workgroup
    constexpr int BK = bstate_ksplit<T, D>();   // compute waves per column slice
    // producer waves: four with the K-split (float32: the next chunk's DMA is bound
    // by how fast it is issued), else two, which leaves the compute waves one per
    // SIMD with 512 registers
    constexpr int BP = BK > 1 ? 4 : 2;
    const size_t units = cu_chunks ? (size_t)H * nseq : (size_t)B * H;
    hipLaunchKernelGGL((bwd_state<T, BT, D, BW, BP, BK>), dim3(units * (D / (16 * BW))),
                       dim3(64 * (BW * BK + BP)), 0, st, sa);
    launch_mark(st);
    if (NC > 0) {
      // B3, one fused kernel
      WyArgs<T, TG, TI> wa{(const TI*)k, (const TI*)w,   (const TI*)v, (const TI*)b, (const TG*)g,
                           dout,         (const T*)fHT,   (const T*)fVnT,
                           reinterpret_cast<const float*>(fA), buf(B_DHT), buf(B_DVNT),
                           T_len, H, N, scale, buf(B_DQG), buf(B_DKG), buf(B_DKBD),
                           buf(B_DAKK), buf(B_SDH), (TI*)dv, (TI*)dw};
      hipLaunchKernelGGL((bwd_wy<T, TG, D, TI>), dim3(NC), dim3(256), 0, st, wa);
      launch_mark(st);
      // B4 + B3 elementwise tail + B5
      GramArgs<T, TG, TI> gr{(const TI*)q, (const TI*)k, (const TI*)b, (const TG*)g,
                             buf(B_DAQK),  buf(B_DAKK),  buf(B_SDH),   buf(B_DQG),
                             buf(B_DKG),   buf(B_DKBD),  T_len,        H,
                             N,            scale,        (TI*)dq,      (TI*)dk,
                             (TI*)db,      (TG*)dg};
      hipLaunchKernelGGL((gram_bwd<T, TG, D, TI>), dim3(NC * (D / gram_panel())), dim3(256), 0,
                         st, gr);
      launch_mark(st);
    }
    return hipGetLastError();
  }
}

// ---------------------------------------------------------------------------
// The reference's backward kernels one at a time (gdn2_bwd.py:32-342): float32,
// chunk 64, the reference's (B,H,N,BT,.) chunk layouts.  The kernels read token
// rows and transposed tiles, so each launcher copies its operands into `ws`
// (chunk_rows_permute, transpose_all) and its results back.  With ws == nullptr a
// launcher only reports the workspace it needs in *need.
namespace {
struct Bump {
  char* base;
  size_t off = 0;
  float* take(size_t floats) {
    const size_t o = off;
    off = align256(off + floats * 4);
    return base ? reinterpret_cast<float*>(base + o) : nullptr;
  }
};
constexpr int SBT = 64;   // chunk of the stage entry points
}  // namespace

// B2, dav_backward_pallas: dAqk = (do v_new^T) . causal, dv_new = Aqk^T do (the causal
// Aqk, as kernel A gives it).
template <int D>
hipError_t launch_stage_dav(hipStream_t st, int B, int N, int H, const float* aqk,
                            const float* v_new, const float* dout, float* daqk, float* dv_new,
                            char* ws, size_t* need) {
  const size_t NC = (size_t)B * H * N;
  Bump m{ws};
  float* dtok = m.take(NC * SBT * D);
  float* VnT = m.take(NC * D * SBT);
  float* DVPT = m.take(NC * D * SBT);
  if (!ws) { *need = m.off; return hipSuccess; }
  if (NC == 0) return hipSuccess;
  chunk_rows_permute(st, dout, dtok, B, H, N, SBT, D, true, false);
  transpose_all(st, v_new, VnT, NC, SBT, D);
  B2Args<float> ba{dtok, VnT, aqk, nullptr, N * SBT, H, N, 1.f, daqk, DVPT, nullptr};
  hipLaunchKernelGGL((bwd_b2<float, D, kB2Dav>), dim3(NC), dim3(64 * b2_waves(D)), 0, st, ba);
  transpose_all(st, DVPT, dv_new, NC, D, SBT);
  return hipGetLastError();
}

// B1, gdn2_dhu_backward: the reverse state scan; dh_all[c] is the gradient of the
// state entering chunk c (dh_all[0] = dh0), dv_all the chunks' dv_new.
template <int D>
hipError_t launch_stage_dhu(hipStream_t st, int B, int N, int H, const float* dout,
                            const float* dv_partial, const float* w_pseudo, const float* qg,
                            const float* kg, const float* gc_last, float scale,
                            const float* dht, float* dh_all, float* dh0, float* dv_all,
                            char* ws, size_t* need) {
  const size_t NC = (size_t)B * H * N, BH = (size_t)B * H;
  Bump m{ws};
  float* dtok = m.take(NC * SBT * D);
  float* QDOT = m.take(NC * D * D);
  float* DVPT = m.take(NC * D * SBT);
  float* KgT = m.take(NC * D * SBT);
  float* Wsp = m.take(NC * SBT * D);
  float* DHT = m.take(NC * D * D);
  float* DVNT = m.take(NC * D * SBT);
  if (!ws) { *need = m.off; return hipSuccess; }
  if (N == 0) {   // no chunk: dh0 = sanitize(dht) (the scan's initial carry)
    sanitized_copy(st, dht, dh0, BH * D * D);
    return hipGetLastError();
  }
  if (NC > 0) {
    chunk_rows_permute(st, dout, dtok, B, H, N, SBT, D, true, false);
    B2Args<float> ba{dtok, nullptr, nullptr, qg, N * SBT, H, N, scale, nullptr, nullptr, QDOT};
    hipLaunchKernelGGL((bwd_b2<float, D, kB2Qdot>), dim3(NC), dim3(64 * b2_waves(D)), 0, st, ba);
    transpose_all(st, dv_partial, DVPT, NC, SBT, D);
    transpose_all(st, kg, KgT, NC, SBT, D);
    // the scan's float32 tiles in the split pair layout, as fwd_prep writes them
    split_runs(st, KgT, KgT, NC * D * SBT / 32);
    split_runs(st, w_pseudo, Wsp, NC * SBT * D / 32);
  }
  BStateArgs<float> sa{Wsp, KgT, gc_last, DVPT, QDOT, dht, N, DHT, DVNT, dh0, nullptr, 1, H};
  constexpr int BW = 2, BK = bstate_ksplit<float, D>(), BP = BK > 1 ? 4 : 2;
  hipLaunchKernelGGL((bwd_state<float, SBT, D, BW, BP, BK>), dim3(BH * (D / (16 * BW))),
                     dim3(64 * (BW * BK + BP)), 0, st, sa);
  if (NC > 0) {
    // DHT[c] = dh_{c+1}^T: dh_all[c+1] = DHT[c]^T, and dh_all[0] = dh0
    transpose_shift(st, DHT, dh_all, BH, N, D, D);
    const hipError_t e = hipMemcpy2DAsync(dh_all, (size_t)N * D * D * 4, dh0, (size_t)D * D * 4,
                                          (size_t)D * D * 4, BH, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return e;
    transpose_all(st, DVNT, dv_all, NC, D, SBT);
  }
  return hipGetLastError();
}

// B3, wy_dqkg_backward_pallas: the gradients through the WY factors, kg and qg;
// dgc per token (the g_last terms on each chunk's last token), dAkk.
template <int D>
hipError_t launch_stage_wy_dqkg(hipStream_t st, int B, int N, int H, const float* q,
                                const float* k, const float* b, const float* w, const float* v,
                                const float* gc, const float* A, const float* h_pre,
                                const float* v_new, const float* dout, const float* dv,
                                const float* dh_next, float scale, float* dq, float* dk,
                                float* db, float* dw, float* dv_raw, float* dgc, float* dakk,
                                char* ws, size_t* need) {
  const size_t NC = (size_t)B * H * N, rows = NC * SBT * D;
  Bump m{ws};
  float* tq = m.take(rows);
  float* tk = m.take(rows);
  float* tb = m.take(rows);
  float* tw = m.take(rows);
  float* tv = m.take(rows);
  float* tg = m.take(rows);
  float* tdo = m.take(rows);
  float* HT = m.take(NC * D * D);
  float* VnT = m.take(NC * D * SBT);
  float* DHT = m.take(NC * D * D);
  float* DVNT = m.take(NC * D * SBT);
  float* DQG = m.take(rows);
  float* DKG = m.take(rows);
  float* DKBD = m.take(rows);
  float* SDH = m.take(NC * D);
  float* oq = m.take(rows);
  float* ok = m.take(rows);
  float* ob = m.take(rows);
  float* ow = m.take(rows);
  float* ov = m.take(rows);
  float* og = m.take(rows);
  if (!ws) { *need = m.off; return hipSuccess; }
  if (NC == 0) return hipSuccess;
  const float* in[] = {q, k, b, w, v, dout};
  float* tok[] = {tq, tk, tb, tw, tv, tdo};
  for (int i = 0; i < 6; ++i) chunk_rows_permute(st, in[i], tok[i], B, H, N, SBT, D, true, false);
  chunk_rows_permute(st, gc, tg, B, H, N, SBT, D, true, true);   // g from the cumsum
  transpose_all(st, h_pre, HT, NC, D, D);
  transpose_all(st, v_new, VnT, NC, SBT, D);
  transpose_all(st, dh_next, DHT, NC, D, D);
  transpose_all(st, dv, DVNT, NC, SBT, D);
  const int T_len = N * SBT;
  WyArgs<float, float, float> wa{tk,  tw,  tv,  tb,  tg,  tdo, HT,  VnT, A,  DHT, DVNT, T_len,
                                 H,   N,   scale, DQG, DKG, DKBD, dakk, SDH, ov, ow};
  if constexpr (D > 128)
    hipLaunchKernelGGL((bwd_wy_wide<float, float, float>), dim3(NC), dim3(512), 0, st, wa);
  else
    hipLaunchKernelGGL((bwd_wy<float, float, D, float>), dim3(NC), dim3(256), 0, st, wa);
  GramArgs<float, float, float> gr{tq,  tk,    tb, tg, nullptr, nullptr, SDH, DQG, DKG, DKBD,
                                   T_len, H,   N,  scale, oq, ok, ob, og};
  hipLaunchKernelGGL((gram_bwd<float, float, D, float, kGramB3>), dim3(NC * (D / gram_panel())),
                     dim3(256), 0, st, gr);
  const float* res[] = {oq, ok, ob, ow, ov, og};
  float* outs[] = {dq, dk, db, dw, dv_raw, dgc};
  for (int i = 0; i < 6; ++i) chunk_rows_permute(st, res[i], outs[i], B, H, N, SBT, D, false, false);
  return hipGetLastError();
}

// B4, intra_backward_pallas: the gradients through the score blocks; q, k, b, g in
// (B,T,H,D) as the reference takes them, dq, dk, db, dgc per chunk.
template <int D>
hipError_t launch_stage_intra(hipStream_t st, int B, int T_len, int H, const float* daqk,
                              const float* dakk, const float* q, const float* k, const float* b,
                              const float* g, float scale, float* dq, float* dk, float* db,
                              float* dgc, char* ws, size_t* need) {
  const int N = T_len / SBT;
  const size_t NC = (size_t)B * H * N, rows = NC * SBT * D;
  Bump m{ws};
  float* oq = m.take(rows);
  float* ok = m.take(rows);
  float* ob = m.take(rows);
  float* og = m.take(rows);
  if (!ws) { *need = m.off; return hipSuccess; }
  if (NC == 0) return hipSuccess;
  GramArgs<float, float, float> gr{q,  k,     b,  g,  daqk, dakk, nullptr, nullptr, nullptr,
                                   nullptr, T_len, H, N, scale, oq, ok, ob, og};
  hipLaunchKernelGGL((gram_bwd<float, float, D, float, kGramB4>), dim3(NC * (D / gram_panel())),
                     dim3(256), 0, st, gr);
  const float* res[] = {oq, ok, ob, og};
  float* outs[] = {dq, dk, db, dgc};
  for (int i = 0; i < 4; ++i) chunk_rows_permute(st, res[i], outs[i], B, H, N, SBT, D, false, false);
  return hipGetLastError();
}

#define GDN2_INST_BSTAGE(D)                                                                   \
  template hipError_t launch_stage_dav<D>(hipStream_t, int, int, int, const float*,           \
                                          const float*, const float*, float*, float*, char*,  \
                                          size_t*);                                           \
  template hipError_t launch_stage_dhu<D>(hipStream_t, int, int, int, const float*,           \
                                          const float*, const float*, const float*,           \
                                          const float*, const float*, float, const float*,    \
                                          float*, float*, float*, char*, size_t*);             \
  template hipError_t launch_stage_wy_dqkg<D>(                                                \
      hipStream_t, int, int, int, const float*, const float*, const float*, const float*,     \
      const float*, const float*, const float*, const float*, const float*, const float*,     \
      const float*, const float*, float, float*, float*, float*, float*, float*, float*,      \
      float*, char*, size_t*);                                                                \
  template hipError_t launch_stage_intra<D>(hipStream_t, int, int, int, const float*,         \
                                            const float*, const float*, const float*,         \
                                            const float*, const float*, float, float*,        \
                                            float*, float*, float*, char*, size_t*);
GDN2_INST_BSTAGE(64)
GDN2_INST_BSTAGE(128)
GDN2_INST_BSTAGE(256)

#define GDN2_INST_BWD(T, TG, BT, D, TI)                                                    \
  template hipError_t launch_bwd<T, TG, BT, D, TI>(                                        \
      hipStream_t, int, int, int, const void*, const void*, const void*, const void*,      \
      const void*, const void*, const float*, float, const float*, const float*, void*,    \
      void*, void*, void*, void*, void*, float*, const char*, char*, const int*, int);
GDN2_INST_BWD(float, float, 64, 64, float)
GDN2_INST_BWD(float, float, 64, 128, float)
GDN2_INST_BWD(float, float, 64, 256, float)
// float32 arithmetic on bfloat16 inputs and gradients (GDN2_BF16_F32)
GDN2_INST_BWD(float, float, 64, 64, bf16_t)
GDN2_INST_BWD(float, float, 64, 128, bf16_t)
GDN2_INST_BWD(float, float, 64, 256, bf16_t)
GDN2_INST_BWD(float, bf16_t, 64, 64, bf16_t)
GDN2_INST_BWD(float, bf16_t, 64, 128, bf16_t)
GDN2_INST_BWD(float, bf16_t, 64, 256, bf16_t)

// This translation unit's clip bound on the current device (gdn2_set_clip).
hipError_t set_clip_bwd(float c) { return set_unit_clip(c); }

}  // namespace gdn2
