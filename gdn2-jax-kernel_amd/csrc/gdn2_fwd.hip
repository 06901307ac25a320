// GDN-2 forward on gfx950: three kernels per call.
//
//   fwd_prep  (one workgroup per chunk)      reference kernels A, B, C
//             gdn2_fwd.py:99-139, 174-243, 264-295
//   fwd_state (one workgroup per (b,h,64 value columns), serial over chunks)
//             the state half of kernel D, gdn2_fwd.py:347-358
//   fwd_out   (one workgroup per chunk)      the output half of kernel D,
//             gdn2_fwd.py:349-353
//
// Decay handling.  Inside a chunk the scores need exp(gc_i - gc_j) per channel
// (gc = in-chunk cumsum of g).  The chunk is cut into 16-token row blocks; a
// pair of blocks (I > J) is factorised around gc at the last token of block J,
// so both factors, x_i exp(gc_i - P_J) and k_j exp(P_J - gc_j), are <= 1 for
// g <= 0 and the 16x16 block is an MFMA product.  Diagonal blocks are
// factorised around their 8th token (|exponent| <= 8 tokens of decay) and
// masked; a block with more than kMaxDiagExp of decay on either side of that
// token takes the exact hierarchical sums of diag_block_exact.  All exponents
// are formed from in-block partial sums, so they never subtract two large
// prefix sums.  This is exact math; the reference's +-20 clip of gc_i - gc_j
// (gdn2_fwd.py:125) is not applied (it changes results by < exp(-20) * |q||k|
// in the documented input domain).
//
// Saturation.  Every stage output the reference sanitizes (clip to +-1e4,
// nan -> 0) is sanitized here too before it is stored: the score blocks Aqk,
// Akk (gdn2_fwd.py:138-139), the blocks of A = (I + Akk)^{-1} (:183,199,208-211,
// 236-238, at the blocks of this kernel's own inversion order), W, u, kg, qg
// and gc_last (:281-289), each chunk state h and each output tile (:359-360).

#include "gdn2_common.h"
#include "gdn2_layout.h"
#include "gdn2_stage.h"

namespace gdn2 {

// T is the workspace / MFMA operand type; TI the type q, k, v, w, b are stored
// in (T, or bfloat16 with float32 tiles: the float32 path on bfloat16 inputs).
template <typename T, typename TG, typename TI = T>
struct PrepArgs {
  const TI *q, *k, *v, *w, *b;
  const TG* g;
  int T_len, H, N;
  long long NC;   // number of chunks, B*H*N
  float scale;
  T* W;     // [cid][BT][D]; float32: in the split pair layout (kPrepFull)
  T* UT;
  T* KgT;   // [cid][D][BT]; float32: in the split pair layout (kPrepFull)
  T* Qg;
  T* Aqk;
  float* GL;
  float* a_dbg;  // optional A = (I + Akk)^{-1} output (BT x BT fp32 per chunk)
  int raw;       // inputs before their activations: q,k <- q,k/|.|_2, w,b <- sigmoid,
                 // g <- -softplus(g), applied here as the values are read
  const int* cstart;  // variable-length batch: token row where chunk c starts
                      // ([N+1], B = 1); rows past cstart[c+1] are neutral padding
  int frag;           // Qg and Aqk in operand-fragment order (qg_frag / aqk_frag):
                      // for the scan's output waves, which then read 1 KB per load
  int* sat_clear;     // segmented scan: its saturation flag, cleared here (the first
                      // launch of the call)
  // Stage modes (PrepMode): Akk output of kPrepScores, the given A of kPrepWy,
  // the given Akk of kPrepSolve ([cid][BT][BT] float32 each)
  float* akk_out;
  const float* a_in;
};

// What one fwd_prep launch computes.  kPrepFull: the forward's per-chunk tiles
// (kernels A-C fused).  The reference's stages one at a time, float32 tiles in
// the reference's (B,H,N,BT,.) layout: kPrepScores Aqk and Akk
// (build_chunk_scores_pallas, gdn2_fwd.py:142-170); kPrepSolve A = (I + Akk)^{-1}
// from a given Akk (wy_solve_pallas, :246-260); kPrepWy w_pseudo, u, kg, qg,
// gc_last from a given A (recompute_wy_pallas, :298-330).
enum PrepMode { kPrepFull = 0, kPrepScores = 1, kPrepSolve = 2, kPrepWy = 3 };

// Operand-fragment order of a chunk's q_g [BT][D] tile: the 16-byte operand
// run a lane (li, lg) feeds a 16 x 16 MFMA for row block I and k-group j
// (channels j*KS + lg*KC + e, e < KC) sits at fragment (I, j), lane 16 lg + li,
// so the 64 lanes' operands of one fragment are 1 KB contiguous.
template <typename T, int BT, int D>
__host__ __device__ constexpr size_t qg_frag(int I, int j, int lane) {
  return ((size_t)(I * (D / Tr<T>::KS) + j) * 64 + lane) * Tr<T>::KC;
}
// The same for Aqk [BT][BT], in the chained order of C-layout tiles: lane
// (li, lg) holds row I*16 + li, columns 16 J + 4 lg + r of block J, which for
// bfloat16 is half J % 2 of fragment (I, J / 2) (float32: fragment (I, J)).
template <typename T, int BT>
__host__ __device__ constexpr size_t aqk_frag(int I, int J, int lane) {
  return sizeof(T) == 4 ? ((size_t)(I * (BT / 16) + J) * 64 + lane) * 4
                        : ((size_t)(I * (BT / 32) + J / 2) * 64 + lane) * 8 + (J % 2) * 4;
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + __expf(-x)); }
// -softplus(x) = -(max(x,0) + log(1 + e^{-|x|}))
__device__ __forceinline__ float neg_softplus(float x) {
  return -(fmaxf(x, 0.f) + __logf(1.f + __expf(-fabsf(x))));
}

// Own row blocks of wave `wv` in fwd_out: {wv} and, for 8 blocks, {7 - wv} --
// equal work for the triangular products.
template <int NB>
__device__ __forceinline__ int own_block(int wv, int i) {
  return i == 0 ? wv : NB - 1 - wv;
}

// Own row block(s) of wave `wv` in fwd_prep (PW waves).  With two blocks per
// wave as own_block.  With one block per wave and 8 waves, waves w and w + 4
// share a SIMD (a workgroup's waves are placed on the 4 SIMDs in turn): they
// take blocks w and 7 - w, so every SIMD runs 7 of the 28 triangular block
// pairs (block I has I of them) instead of 4, 6, 8, 10.
template <int NB, int PW>
__device__ __forceinline__ int prep_block(int wv, int i) {
  if constexpr (NB == PW && PW == 8) return wv < 4 ? wv : NB + 3 - wv;
  return own_block<NB>(wv, i);
}


// Diagonal 16 x 16 score block of one row block, summed exactly for strong
// decay: when more than kMaxDiagExp of log-decay lies between a token and the
// block's 8th, the factors e^{lc - lm}, e^{lm - lc} of fwd_prep's
// factorisation would overflow.  For groups of G = 16, 8, 4, 2 tokens the pairs
// (i in the upper, j in the lower half of one group) are factorised around the
// group's boundary token b instead, where both e^{lc_i - lc_b} and
// e^{lc_b - lc_j} are <= 1 for g <= 0, then the diagonal i = j is added (factor
// 1; Aqk only, Akk is strictly lower).  Lane (li, lg) of the caller's wave
// gets [i = li][j = 4 lg + r] of sum_d q_i k_j e^{lc_i - lc_j} (d.q, unscaled)
// and of sum_d (b k)_i k_j e^{..} (d.k), unmasked above the diagonal.  The
// operands are loaded again from `off` (the row of token li plus the panel's
// first channel; the panel's NKD k-groups) and rounded as fwd_prep rounds them;
// `raw` applies the input activations with the caller's norms iq, ik; `real`
// false makes the token neutral.  The operands are loaded again (from L2) and
// the levels run in a loop the compiler keeps rolled, so that this rarely
// taken path adds few registers to fwd_prep.
struct DiagSums {
  f32x4 q, k;
};
template <typename T, typename TI, typename TG, int NKD>
__device__ __forceinline__ DiagSums diag_block_exact(
    const TI* __restrict__ q, const TI* __restrict__ k, const TI* __restrict__ b,
    const TG* __restrict__ g, size_t off, bool raw, bool real, float iq, float ik) {
  using Op = typename Tr<T>::Op;
  constexpr int KC = Tr<T>::KC, KS = Tr<T>::KS;
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  DiagSums d;
  d.q = f32x4{0.f, 0.f, 0.f, 0.f};
  d.k = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int L = 0; L < 5; ++L) {   // L < 4: groups of 16 >> L tokens; L = 4: i = j
    const int G = 16 >> L, half = G / 2;
    const bool upper = (li % G) >= half;
    const int bnd = (li / G) * G + half - 1;   // boundary token of li's group
    f32x4 tq = {0.f, 0.f, 0.f, 0.f}, tk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int j = 0; j < NKD; ++j) {
      float lc[KC], qv[KC], kv[KC], bv[KC];
      load_f<KC>(g + off + j * KS + lg * KC, lc);
      load_f<KC>(q + off + j * KS + lg * KC, qv);
      load_f<KC>(k + off + j * KS + lg * KC, kv);
      load_f<KC>(b + off + j * KS + lg * KC, bv);
#pragma unroll
      for (int e = 0; e < KC; ++e) {
        if (raw) {
          lc[e] = neg_softplus(lc[e]);
          qv[e] *= iq;
          kv[e] *= ik;
          bv[e] = sigmoidf(bv[e]);
        }
        qv[e] = real ? to_f(from_f<T>(qv[e])) : 0.f;
        kv[e] = real ? to_f(from_f<T>(kv[e])) : 0.f;
        bv[e] = real ? to_f(from_f<T>(bv[e])) : 0.f;
        lc[e] = row_scan16(real ? lc[e] : 0.f);
        const float lb = __shfl(lc[e], bnd, 16);
        // (g > 0 lies outside the domain: the exponent is held below overflow)
        const float f = L == 4 ? 1.f
                      : __expf(fminf(upper ? lc[e] - lb : lb - lc[e], kMaxDiagExp));
        qv[e] *= f;
        bv[e] *= kv[e] * f;
        kv[e] *= f;
      }
      const Op xo = op_from<T>(kv);
      mma(tq, xo, op_from<T>(qv));
      mma(tk, xo, op_from<T>(bv));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int jj = 4 * lg + r;
      const bool cross = L < 4 && (li / G == jj / G) && (li % G >= half) && (jj % G < half);
      d.q[r] += (cross || (L == 4 && jj == li)) ? tq[r] : 0.f;
      d.k[r] += cross ? tk[r] : 0.f;
    }
  }
  return d;
}

// One workgroup per chunk with prep_waves(BT) waves.  A wave owns one 16-token
// row block (8 waves at BT = 128), or the pair {wv, NB-1-wv} when there are
// twice as many blocks as waves (equal work for the triangular loops).  Per element four
// exponentials are evaluated (e^{loc}, e^{T_I - loc} and the two diagonal-block
// factors); the block-level factors e^{P_{I-1}}, e^{S_{I+1}} come from LDS.
//
// Channels are processed in panels of up to 128 (D = 256: two panels; chunk 64
// at D = 128: two panels of 64).  The
// cumsum, decay factors, q_g / kg^T / (b k e^gc)^T and khat are per channel, so
// steps 1-3 run once per panel; the score blocks Aqk, Akk are sums over
// channels, accumulated over the panels (Akk in float32 LDS, sA; Aqk in the
// registers of the wave that owns the row block) and stored after the last
// one.  u = A (w v) is computed per panel of (w v)^T.  With one panel every
// score block is stored as soon as it is computed.
constexpr int prep_waves(int BT) { return BT >= 128 ? 8 : 4; }
// Workgroups per CU the register allocation is held to: three for bfloat16 at
// chunk 64 and D = 128 (50 KB of LDS each), else what the kernel needs.
constexpr int prep_min_blocks(int esize, int BT, int D) {
  return esize == 2 && BT == 64 && D == 128 ? 3 : 1;
}

template <typename T, typename TG, int BT, int D, typename TI, int MODE = kPrepFull>
__global__ void __launch_bounds__(64 * prep_waves(BT), prep_min_blocks(sizeof(T), BT, D))
    fwd_prep(PrepArgs<T, TG, TI> a) {
  static_assert(MODE == kPrepFull || (sizeof(T) == 4 && BT == 64),
                "the stage modes run float32 tiles at chunk 64");
  // float32 tiles of the forward: W and kg^T in the split pair layout of the
  // float32 scans (gdn2_common.h), whose MFMA operands they are
  constexpr bool SPF = sizeof(T) == 4 && MODE == kPrepFull;
  using Op = typename Tr<T>::Op;
  constexpr int KC = Tr<T>::KC, KS = Tr<T>::KS;
  constexpr int NB = BT / 16;             // 16-token row blocks
  constexpr int PW = prep_waves(BT), NT = 64 * PW;   // waves, threads
  constexpr int NBW = NB / PW;            // row blocks per wave
  static_assert(NB % PW == 0 && (NBW == 1 || NBW == 2), "row blocks must split over waves");
  // channels per panel: up to 128; chunk 64 at D = 128 takes two 64-channel
  // panels, which brings the LDS under half a CU (float32: two workgroups per CU,
  // bfloat16: three, one loading while the others compute)
  constexpr int DP = D < 128 ? D : (BT == 64 && D == 128 ? 64 : 128);
  constexpr int NPN = D / DP;             // panels
  static_assert(D % DP == 0 && DP <= NT, "panels must tile D");
  constexpr int NKD = DP / KS;            // k-groups over a panel's channels
  constexpr int NKT = BT / KS;            // k-groups over tokens
  constexpr int DQ = NKD * KC;            // channels of a panel owned per lane (= DP/4)
  constexpr int PADT = 16 / sizeof(T);
  constexpr int KH_LD = DP + PADT;        // khat [t][d], one panel
  constexpr int TT_LD = BT + PADT;        // [d][t] tiles
  constexpr int A_LD = BT + 4;            // A [t][s] fp32
  constexpr int R0 = (BT * KH_LD > DP * TT_LD) ? BT * KH_LD : DP * TT_LD;

  __shared__ __align__(16) T sR0[R0];         // khat [t][d]; later (w v)^T [d][t], one panel
  __shared__ __align__(16) T sKbdT[D * TT_LD];  // (b k e^gc)^T [d][t]
  __shared__ __align__(16) float sA[BT * A_LD];
  // per-(block, channel) decay factors of steps 1-3, then (free after step 3)
  // the parked T = L_BA X_AA blocks of the inverse's doubling steps
  constexpr int PARK = 16 * 20;   // one parked 16 x 16 block, rows padded to 20 floats
  constexpr int SMALL = (4 * NB * DP > NB * NB / 4 * PARK) ? 4 * NB * DP : NB * NB / 4 * PARK;
  __shared__ __align__(16) float sSmall[SMALL];
  float* const sTot = sSmall;                  // T_m: per-block sums of g
  float* const sETot = sSmall + NB * DP;       // e^{T_m}
  float* const sF0 = sSmall + 2 * NB * DP;     // e^{P_{I-1}}
  float* const sF1 = sSmall + 3 * NB * DP;     // e^{S_{I+1}}

  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  if (a.sat_clear && blockIdx.x == 0 && tid == 0) *a.sat_clear = 0;
  // Chunk order (the grid is (b,h) pairs x N chunks).  bfloat16: dealt last-first
  // across all (b,h), so the state scan's first chunks are the most recently
  // written (still in the last-level cache): the latency-bound bf16 scan gains 5 %.
  // float32: (b,h)-major, neighbouring workgroups on neighbouring memory; its scan
  // is bound by the MFMA chain, and the last-first order only cost this kernel 5 %.
  int cid = blockIdx.x;
  if constexpr (sizeof(T) == 2) {
    const int nbh = gridDim.x / a.N;
    cid = (blockIdx.x % nbh) * a.N + (a.N - 1 - blockIdx.x / nbh);
  }
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  const size_t HD = (size_t)a.H * D;
  const ChunkRows cr = chunk_rows(a.cstart, c, bb, a.T_len, BT);
  const size_t tok0 = cr.row0 * HD + (size_t)hh * D;
  auto rowp = [&](int t) { return tok0 + (size_t)t * HD; };
  auto chan = [&](int x) { return (x / KC) * KS + lg * KC + (x % KC); };
  // Padding rows of a short chunk act as neutral tokens (k = 0, g = 0: the state
  // passes through unchanged).  They load a real row of the chunk (no branch
  // around the loads) and are zeroed once the values are first needed, only in
  // chunks that have padding.
  const bool padded = cr.valid < BT;
  auto real = [&](int i) { return prep_block<NB, PW>(wv, i) * 16 + li < cr.valid; };
  auto load_row = [&](int i) {
    const int t = prep_block<NB, PW>(wv, i) * 16 + li, last = cr.valid > 0 ? cr.valid - 1 : 0;
    return rowp(t < last ? t : last);
  };
  const bool raw = a.raw != 0;
  // Barriers order LDS data only (lds_barrier): no wave reads global memory
  // another wave of this workgroup wrote, so stores stay in flight across them.
  T* kgT = a.KgT + (size_t)cid * D * BT;
  T* aqk = a.Aqk + (size_t)cid * BT * BT;
  // offset of row I*16 + li, columns 16 J + 4 lg .. + 3 of Aqk
  auto aqk_at = [&](int I, int J) {
    return a.frag ? aqk_frag<T, BT>(I, J, lane) : (size_t)(I * 16 + li) * BT + J * 16 + 4 * lg;
  };

  // raw inputs with several panels: 1 / max(|q|_2, 1e-12) and the same for k over
  // all D channels, before the panel loop
  float iqn[NBW], ikn[NBW];
  if constexpr (NPN > 1) {
    if (raw) {
#pragma unroll
      for (int i = 0; i < NBW; ++i) {
        const size_t off = load_row(i);
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int pn = 0; pn < NPN; ++pn)
#pragma unroll
          for (int j = 0; j < NKD; ++j) {
            const Op qv = op_in<T>(a.q + off + pn * DP + j * KS + lg * KC);
            const Op kv = op_in<T>(a.k + off + pn * DP + j * KS + lg * KC);
#pragma unroll
            for (int e = 0; e < KC; ++e) {
              sq += to_f(qv[e]) * to_f(qv[e]);
              sk += to_f(kv[e]) * to_f(kv[e]);
            }
          }
        sq += __shfl_xor(sq, 16);
        sq += __shfl_xor(sq, 32);
        sk += __shfl_xor(sk, 16);
        sk += __shfl_xor(sk, 32);
        iqn[i] = 1.f / fmaxf(sqrtf(sq), 1e-12f);
        ikn[i] = 1.f / fmaxf(sqrtf(sk), 1e-12f);
      }
    }
  }

  // Aqk partial sums over the panels: the diagonal block and the blocks J < I of
  // this wave's row blocks (several panels only, all at chunk 64)
  static_assert(NPN == 1 || NB == 4, "panel sums of Aqk are held for 4 row blocks");
  f32x4 qdiag[NBW], qoff[NBW][NB];
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    qdiag[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int J = 0; J < NB; ++J) qoff[i][J] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // kPrepSolve: the strictly lower part of the given Akk into sA; no input is read
  if constexpr (MODE == kPrepSolve) {
    const float* src = a.a_in + (size_t)cid * BT * BT;
    for (int i = tid; i < BT * BT / 4; i += NT) {
      const int r = i / (BT / 4), c4 = (i % (BT / 4)) * 4;
      f32x4 x = load4f(src + (size_t)r * BT + c4);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = c4 + e < r ? x[e] : 0.f;
      store4(&sA[r * A_LD + c4], x);
    }
    lds_barrier();
  }

  if constexpr (MODE != kPrepSolve) {
#pragma unroll
  for (int pn = 0; pn < NPN; ++pn) {
    const int d0 = pn * DP;               // first channel of the panel
    constexpr bool one = NPN == 1;
    const bool last_pn = pn == NPN - 1;
    if (pn > 0) lds_barrier();            // the previous panel's LDS reads are done

    // all loads needed before the inverse, issued together, g first: the cumsum
    // waits for g alone (memory operations complete in order) while q, k, b
    // arrive behind it
    float loc[NBW][DQ];
    Op qo[NBW][NKD], ko[NBW][NKD], bo[NBW][NKD];
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const size_t off = load_row(i) + d0;
#pragma unroll
      for (int j = 0; j < NKD; ++j) load_f<KC>(a.g + off + j * KS + lg * KC, &loc[i][j * KC]);
#pragma unroll
      for (int j = 0; j < NKD; ++j) {
        qo[i][j] = op_in<T>(a.q + off + j * KS + lg * KC);
        ko[i][j] = op_in<T>(a.k + off + j * KS + lg * KC);
        bo[i][j] = op_in<T>(a.b + off + j * KS + lg * KC);
      }
    }
    if (pn == 0) {
      for (int i = tid; i < BT * A_LD / 4; i += NT)
        reinterpret_cast<f32x4*>(sA)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // ---- 1. in-block inclusive cumsum of g (lanes li = tokens) --------------
    if (padded) {
#pragma unroll
      for (int i = 0; i < NBW; ++i) {
        if (!real(i)) {
#pragma unroll
          for (int x = 0; x < DQ; ++x) loc[i][x] = 0.f;
#pragma unroll
          for (int j = 0; j < NKD; ++j) {
            qo[i][j] = op_zero<T>();
            ko[i][j] = op_zero<T>();
            bo[i][j] = op_zero<T>();
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int I = prep_block<NB, PW>(wv, i);
      if (raw) {
        const bool rv = real(i);
#pragma unroll
        for (int x = 0; x < DQ; ++x) loc[i][x] = rv ? neg_softplus(loc[i][x]) : 0.f;
      }
#pragma unroll
      for (int x = 0; x < DQ; ++x) loc[i][x] = row_scan16(loc[i][x]);
      if (li == 15) {
#pragma unroll
        for (int x = 0; x < DQ; ++x) sTot[I * DP + chan(x)] = loc[i][x];
      }
    }
    lds_barrier();   // LDS only: q, k, b may still be in flight
    for (int i = tid; i < NB * DP; i += NT) {
      sETot[i] = __expf(sTot[i]);
    }
    if (tid < DP) {
      float run = 0.f;
#pragma unroll
      for (int m = 0; m < NB; ++m) { sF0[m * DP + tid] = __expf(run); run += sTot[m * DP + tid]; }
      if constexpr (MODE != kPrepScores) a.GL[(size_t)cid * D + d0 + tid] = sanitize(run);
      run = 0.f;
#pragma unroll
      for (int m = NB - 1; m >= 0; --m) { sF1[m * DP + tid] = __expf(run); run += sTot[m * DP + tid]; }
    }
    lds_barrier();

    // ---- 2. per-token factors: qg, kbd, kg, khat; diagonal score blocks -----
    float aq[NBW][DQ], ak[NBW][DQ];
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int I = prep_block<NB, PW>(wv, i);
      const int t = I * 16 + li;
      T* qgp = a.Qg + (size_t)cid * BT * D + (size_t)t * D + d0;
      T* qgf = a.Qg + (size_t)cid * BT * D;
      f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
      // raw inputs: q,k <- q,k / max(|.|_2, 1e-12) over D (F.normalize) and
      // b <- sigmoid(b), in place in the loaded registers; a token's channels sit
      // in the four lanes li, li+16, li+32, li+48
      float iq = 1.f, ik = 1.f;
      if (raw) {
        if constexpr (one) {
          float sq = 0.f, sk = 0.f;
#pragma unroll
          for (int j = 0; j < NKD; ++j)
#pragma unroll
            for (int e = 0; e < KC; ++e) {
              const float qv = to_f(qo[i][j][e]), kv = to_f(ko[i][j][e]);
              sq += qv * qv;
              sk += kv * kv;
            }
          sq += __shfl_xor(sq, 16);
          sq += __shfl_xor(sq, 32);
          sk += __shfl_xor(sk, 16);
          sk += __shfl_xor(sk, 32);
          iq = 1.f / fmaxf(sqrtf(sq), 1e-12f);
          ik = 1.f / fmaxf(sqrtf(sk), 1e-12f);
        } else {
          iq = iqn[i];
          ik = ikn[i];
        }
#pragma unroll
        for (int j = 0; j < NKD; ++j)
#pragma unroll
          for (int e = 0; e < KC; ++e) {
            qo[i][j][e] = from_f<T>(to_f(qo[i][j][e]) * iq);
            ko[i][j][e] = from_f<T>(to_f(ko[i][j][e]) * ik);
            bo[i][j][e] = from_f<T>(sigmoidf(to_f(bo[i][j][e])));
          }
      }
      bool wide = false;   // a channel's decay across the block exceeds the factors' range
#pragma unroll
      for (int j = 0; j < NKD; ++j) {
        float qg[KC], kh[KC], dq[KC], dk[KC], db[KC], kgr[KC];
#pragma unroll
        for (int e = 0; e < KC; ++e) {
          const int x = j * KC + e, ch = chan(x);
          const float qv = to_f(qo[i][j][e]), kv = to_f(ko[i][j][e]), bv = to_f(bo[i][j][e]);
          const float lc = loc[i][x];
          const float eloc = __expf(lc);
          const float ekh = __expf(sTot[I * DP + ch] - lc);
          const float egc = eloc * sF0[I * DP + ch];
          const float bk = bv * kv;
          qg[e] = sanitize(qv * egc);
          if constexpr (MODE != kPrepScores) sKbdT[(d0 + ch) * TT_LD + t] = from_f<T>(bk * egc);
          const float kgv = sanitize(kv * ekh * sF1[I * DP + ch]);
          if constexpr (SPF) {
            split_store1(reinterpret_cast<char*>(kgT + (size_t)(d0 + ch) * BT), t, kgv);
          } else if constexpr (MODE == kPrepFull) {
            kgT[(size_t)(d0 + ch) * BT + kpos<T>(t)] = from_f<T>(kgv);
          }
          kgr[e] = kgv;
          kh[e] = kv * ekh;
          aq[i][x] = qv * eloc;
          ak[i][x] = bk * eloc;
          // the diagonal-block factors keep their own exponentials: e^{loc} or
          // e^{T_I-loc} may underflow where e^{loc-loc_m} e^{loc_m-loc'} does not
          const float lm = row_bcast<7>(lc);
          wide = wide || !(fabsf(lc - lm) <= kMaxDiagExp);
          const float edq = __expf(lc - lm), edk = __expf(lm - lc);
          dq[e] = qv * edq;
          db[e] = bk * edq;
          dk[e] = kv * edk;
        }
        if constexpr (MODE != kPrepScores)
          *reinterpret_cast<Op*>(a.frag ? qgf + qg_frag<T, BT, D>(I, d0 / KS + j, lane)
                                        : qgp + j * KS + lg * KC) = op_from<T>(qg);
        if constexpr (MODE == kPrepWy) {   // kg [t][d]
          *reinterpret_cast<Op*>(a.KgT + (size_t)cid * BT * D + (size_t)t * D + d0 + j * KS +
                                 lg * KC) = op_from<T>(kgr);
          continue;                        // no scores
        }
        *reinterpret_cast<Op*>(&sR0[t * KH_LD + j * KS + lg * KC]) = op_from<T>(kh);
        // diagonal block, factorised around its 8th token: X = k rows (j),
        // Y = q / bk rows (i) -> lane holds [i=li][j=4lg+r]
        const Op xo = op_from<T>(dk);
        mma(accq, xo, op_from<T>(dq));
        mma(acck, xo, op_from<T>(db));
      }
      if constexpr (MODE == kPrepWy) continue;
      if (__ballot(wide) != 0) {
        const DiagSums d = diag_block_exact<T, TI, TG, NKD>(a.q, a.k, a.b, a.g,
                                                             load_row(i) + d0, raw, real(i),
                                                             iq, ik);
        accq = d.q;
        acck = d.k;
      }
      f32x4 sq, sk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int jj = 4 * lg + r;
        sq[r] = (jj <= li) ? a.scale * accq[r] : 0.f;
        sk[r] = (jj < li) ? acck[r] : 0.f;
      }
      const int e0 = t * A_LD + I * 16 + 4 * lg;
      if constexpr (one) {
        store4(aqk + aqk_at(I, I), sanitize4(sq));
        store4(&sA[e0], sanitize4(sk));
      } else {
        if (pn > 0) {
          sq += qdiag[i];
          sk += load4f(&sA[e0]);
        }
        if (last_pn) store4(aqk + aqk_at(I, I), sanitize4(sq));
        else qdiag[i] = sq;
        store4(&sA[e0], last_pn ? sanitize4(sk) : sk);
      }
    }
    lds_barrier();

    // ---- 3. off-diagonal score blocks (I > J) on MFMA ------------------------
#pragma unroll
    for (int i = 0; i < (MODE == kPrepWy ? 0 : NBW); ++i) {
      const int I = prep_block<NB, PW>(wv, i);
      const int t = I * 16 + li;
      // block pair (I, J), J < I, in descending J; after each pair aq and ak
      // take the decay e^{T_J} of block J in place (they are not needed after
      // the last pair)
      auto pair = [&](int J, f32x4& qp) __attribute__((always_inline)) {
        f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NKD; ++j) {
          const Op xo = op_load<T>(&sR0[(J * 16 + li) * KH_LD + j * KS + lg * KC]);
          mma(accq, xo, op_from<T>(&aq[i][j * KC]));
          mma(acck, xo, op_from<T>(&ak[i][j * KC]));
        }
        const int e0 = t * A_LD + J * 16 + 4 * lg;
        if constexpr (one) {
          store4(aqk + aqk_at(I, J), sanitize4(accq * a.scale));
          store4(&sA[e0], sanitize4(acck));
        } else {
          f32x4 sq = accq * a.scale;
          if (pn > 0) {
            sq += qp;
            acck += load4f(&sA[e0]);
          }
          if (last_pn) store4(aqk + aqk_at(I, J), sanitize4(sq));
          else qp = sq;
          store4(&sA[e0], last_pn ? sanitize4(acck) : acck);
        }
#pragma unroll
        for (int x = 0; x < DQ; ++x) {
          const float e = sETot[J * DP + chan(x)];
          aq[i][x] *= e;
          ak[i][x] *= e;
        }
      };
      if constexpr (one) {
        for (int J = I - 1; J >= 0; --J) pair(J, qoff[i][0]);   // qoff unused here
      } else {
#pragma unroll
        for (int J = NB - 2; J >= 0; --J)   // static J: the sums stay in registers
          if (J < I) pair(J, qoff[i][J]);
      }
    }
  }
  lds_barrier();
  }  // MODE != kPrepSolve

  // kPrepScores: Akk (sA, zero above the strict lower part) out, Aqk's blocks
  // above the diagonal zeroed (the steps above wrote the others)
  if constexpr (MODE == kPrepScores) {
    float* dst = a.akk_out + (size_t)cid * BT * BT;
    float* aq = reinterpret_cast<float*>(aqk);
    for (int i = tid; i < BT * BT / 4; i += NT) {
      const int r = i / (BT / 4), c4 = (i % (BT / 4)) * 4;
      store4(dst + (size_t)r * BT + c4, load4f(&sA[r * A_LD + c4]));
      if (c4 / 16 > r / 16) store4(aq + (size_t)r * BT + c4, f32x4{0.f, 0.f, 0.f, 0.f});
    }
    return;
  }


  // w, v of the first panel: in flight during the inverse (issued earlier they
  // slow the load-bound first phase or hold registers through steps 2-3)
  Op wo[NBW][NKD], vo[NBW][NKD];
  auto load_wv = [&](int d0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const size_t off = load_row(i) + d0;
#pragma unroll
      for (int j = 0; j < NKD; ++j) {
        wo[i][j] = op_in<T>(a.w + off + j * KS + lg * KC);
        vo[i][j] = op_in<T>(a.v + off + j * KS + lg * KC);
      }
    }
  };
  if constexpr (MODE != kPrepSolve) load_wv(0);

  if constexpr (MODE == kPrepWy) {
    // the given A into sA
    const float* src = a.a_in + (size_t)cid * BT * BT;
    for (int i = tid; i < BT * BT / 4; i += NT) {
      const int r = i / (BT / 4), c4 = (i % (BT / 4)) * 4;
      store4(&sA[r * A_LD + c4], load4f(src + (size_t)r * BT + c4));
    }
    lds_barrier();
  } else {
  // ---- 4. A = (I + Akk)^{-1}: diagonal blocks ---------------------------------
  // The diagonal block L of Akk is strictly lower 16 x 16, so L^16 = 0 and
  // (I + L)^{-1} = (I - L)(I + L^2)(I + L^4)(I + L^8): ten 16 x 16 products in
  // four dependent rounds, on MFMA in registers.  For C-layout tiles
  // mma(acc, C(P), C(Q)) accumulates P^T Q (a C tile read as the row operand is
  // the transposed matrix), so each factor is carried with its transpose.
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int I = prep_block<NB, PW>(wv, i);
    float* blk = &sA[(I * 16) * A_LD + I * 16];
    f32x4 L, E;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      L[r] = blk[(4 * lg + r) * A_LD + li];
      E[r] = (4 * lg + r == li) ? 1.f : 0.f;
    }
    const f32x4 Lt = load4f(&blk[li * A_LD + 4 * lg]);   // C(L^T)
    auto mul = [](f32x4 a, f32x4 b) __attribute__((always_inline)) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
      mma(c, a, b);
      return c;
    };
    const f32x4 P2 = mul(Lt, L), P2t = mul(L, Lt);          // L^2, (L^2)^T
    const f32x4 M1 = mul(E - Lt, E + P2);                    // (I - L)(I + L^2)
    const f32x4 M1t = mul(E + P2, E - Lt);
    const f32x4 P4 = mul(P2t, P2), P4t = mul(P2, P2t);      // L^4, (L^4)^T
    const f32x4 M2 = mul(M1t, E + P4);                       // M1 (I + L^4)
    const f32x4 M2t = mul(E + P4, M1t);
    const f32x4 P8 = mul(P4t, P4);                           // L^8
    const f32x4 M = mul(M2t, E + P8);                        // M2 (I + L^8)
    (void)M2;
#pragma unroll
    for (int r = 0; r < 4; ++r) blk[(4 * lg + r) * A_LD + li] = sanitize(M[r]);
  }
  lds_barrier();

  // ---- 4b. off-diagonal blocks by recursive doubling ------------------------
  // For h = 1, 2, 4, ... 16-row blocks and each group [A0, A0 + 2h) with
  // B0 = A0 + h: X_BA = -X_BB (L_BA X_AA), X_AA and X_BB being inverses from
  // the previous h.  All groups and blocks of one h run in parallel over the
  // waves (at h = NB/2 two blocks per wave, paired for equal work); T = L_BA X_AA
  // is parked in sSmall between its two barriers.  L_BA is read before the
  // barrier after which X_BA overwrites it.
  {
    auto rowop = [&](int R, int C) __attribute__((always_inline)) {
      return load4f(&sA[(R * 16 + li) * A_LD + C * 16 + 4 * lg]);
    };
    auto colop = [&](const float* base, int ld) __attribute__((always_inline)) {
      f32x4 y;
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = base[(4 * lg + r) * ld + li];
      return y;
    };
    auto Xc = [&](int R, int C) __attribute__((always_inline)) {
      return colop(&sA[(R * 16) * A_LD + C * 16], A_LD);
    };
    auto put = [&](float* base, int ld, f32x4 v) __attribute__((always_inline)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) base[(4 * lg + r) * ld + li] = v[r];
    };
    // h = 1: T is one block, kept in registers
    if (wv < NB / 2) {
      const int A0 = 2 * wv, B0 = A0 + 1;
      f32x4 t = {0.f, 0.f, 0.f, 0.f}, x = {0.f, 0.f, 0.f, 0.f};
      mma(t, rowop(B0, A0), Xc(A0, A0));
      mma(x, rowop(B0, B0), t);
      put(&sA[(B0 * 16) * A_LD + A0 * 16], A_LD, sanitize4(-x));
    }
    lds_barrier();
    auto level = [&](auto hc) __attribute__((always_inline)) {
      constexpr int h = decltype(hc)::value;
      constexpr int NOUT = NB * h / 2;          // blocks X_BA of this h, all groups
      static_assert(NOUT <= PW || (NOUT == 2 * PW && h % 2 == 0), "blocks must split over waves");
      auto tblock = [&](int g, int i, int j) __attribute__((always_inline)) {
        const int A0 = g * 2 * h, B0 = A0 + h;
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < h; ++k)
          if (k >= j) mma(t, rowop(B0 + i, A0 + k), Xc(A0 + k, A0 + j));
        put(&sSmall[((g * h + i) * h + j) * PARK], 20, t);
      };
      auto xblock = [&](int g, int i, int j) __attribute__((always_inline)) {
        const int A0 = g * 2 * h, B0 = A0 + h;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < h; ++k)
          if (k <= i) mma(x, rowop(B0 + i, B0 + k), colop(&sSmall[((g * h + k) * h + j) * PARK], 20));
        put(&sA[((B0 + i) * 16) * A_LD + (A0 + j) * 16], A_LD, sanitize4(-x));
      };
      if constexpr (NOUT <= PW) {
        const int g = wv / (h * h), i = (wv / h) % h, j = wv % h;
        if (wv < NOUT) tblock(g, i, j);
        lds_barrier();
        if (wv < NOUT) xblock(g, i, j);
        lds_barrier();
      } else {
        // one group (h = NB/2), two blocks per wave: T_ij costs h - j products,
        // so a wave takes T_{i,q} and T_{i,h-1-q}; X_ij costs i + 1, so it takes
        // X_{q,j} and X_{h-1-q,j} (i1 = its T row and X column)
        static_assert(h * (h / 2) == PW, "pairs must cover the blocks once");
        const int i1 = wv / (h / 2), q = wv % (h / 2);
        tblock(0, i1, q);
        tblock(0, i1, h - 1 - q);
        lds_barrier();
        xblock(0, q, i1);
        xblock(0, h - 1 - q, i1);
        lds_barrier();
      }
    };
    if constexpr (NB >= 4) level(std::integral_constant<int, 2>{});
    if constexpr (NB >= 8) level(std::integral_constant<int, 4>{});
    static_assert(NB <= 8, "doubling steps up to h = 4");
  }
  }  // MODE != kPrepWy

  if constexpr (MODE == kPrepSolve) {
    // A out (the inverse of a lower-triangular matrix: zero above the diagonal)
    float* dst = a.a_dbg + (size_t)cid * BT * BT;
    for (int i = tid; i < BT * BT / 4; i += NT) {
      const int r = i / (BT / 4), c4 = (i % (BT / 4)) * 4;
      store4(dst + (size_t)r * BT + c4, load4f(&sA[r * A_LD + c4]));
    }
    return;
  }
  T* sWVT = sR0;
#pragma unroll
  for (int pn = 0; pn < NPN; ++pn) {
    const int d0 = pn * DP;
    if (pn > 0) {
      load_wv(d0);
      lds_barrier();  // the previous panel's (w v)^T reads are done
    }
    // ---- 5. (w v)^T of the panel into LDS (khat's region, free since step 3) --
    if (padded) {
#pragma unroll
      for (int i = 0; i < NBW; ++i)
        if (!real(i)) {
#pragma unroll
          for (int j = 0; j < NKD; ++j) vo[i][j] = op_zero<T>();
        }
    }
    if (raw) {  // w <- sigmoid(w)
#pragma unroll
      for (int i = 0; i < NBW; ++i)
#pragma unroll
        for (int j = 0; j < NKD; ++j)
#pragma unroll
          for (int e = 0; e < KC; ++e) wo[i][j][e] = from_f<T>(sigmoidf(to_f(wo[i][j][e])));
    }
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int t = prep_block<NB, PW>(wv, i) * 16 + li;
#pragma unroll
      for (int x = 0; x < DQ; ++x)
        sWVT[chan(x) * TT_LD + t] =
            from_f<T>(to_f(wo[i][x / KC][x % KC]) * to_f(vo[i][x / KC][x % KC]));
    }
    lds_barrier();

    if (pn == 0 && a.a_dbg) {
      float* dst = a.a_dbg + (size_t)cid * BT * BT;
      for (int i = tid; i < BT * BT; i += NT) dst[i] = sA[(i / BT) * A_LD + (i % BT)];
    }

    // ---- 6. w_pseudo = A (b k e^gc), u = A (w v), the panel's columns ---------
    // Items (row block I, 16-channel tile dt) are dealt round-robin over the waves
    // (I-major), so every wave gets the same mix of short and long (triangular,
    // K = 16 (I+1)) products; all operands are in LDS.
    constexpr int NDTT = DP / 16;                    // channel tiles of the panel
    static_assert((NB * NDTT) % PW == 0, "W/U items must split over the waves");
    T* Wc = a.W + (size_t)cid * BT * D;
    T* Uc = a.UT + (size_t)cid * D * BT;
#pragma unroll
    for (int step = 0; step < NB * NDTT / PW; ++step) {
      const int j = wv + step * PW, I = j / NDTT, dt = j % NDTT;
      const int kgmax = (I * 16 + 15) / KS;
      const int dg = d0 + dt * 16;      // first channel of the tile
      f32x4 accw = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kg = 0; kg < NKT; ++kg) {
        if (MODE == kPrepWy || kg <= kgmax) {   // kPrepWy: all of the given A
          float tmp[KC];
#pragma unroll
          for (int e = 0; e < KC; e += 4) {
            const f32x4 v4 = load4f(&sA[(I * 16 + li) * A_LD + kg * KS + lg * KC + e]);
            tmp[e] = v4[0]; tmp[e + 1] = v4[1]; tmp[e + 2] = v4[2]; tmp[e + 3] = v4[3];
          }
          const Op af = op_from<T>(tmp);
          mma(accw, op_load<T>(&sKbdT[(dg + li) * TT_LD + kg * KS + lg * KC]), af);
          mma(accu, af, op_load<T>(&sWVT[(dt * 16 + li) * TT_LD + kg * KS + lg * KC]));
        }
      }
      if constexpr (SPF) {
        split_store4(reinterpret_cast<char*>(Wc + (size_t)(I * 16 + li) * D), dg + 4 * lg,
                     sanitize4(accw));
      } else {
        store4(Wc + (size_t)(I * 16 + li) * D + kpos<T>(dg + 4 * lg), sanitize4(accw));
      }
      if constexpr (MODE == kPrepWy) {   // u [t][d]
        T* uc = a.UT + (size_t)cid * BT * D;
#pragma unroll
        for (int r = 0; r < 4; ++r) uc[(size_t)(I * 16 + 4 * lg + r) * D + dg + li] = sanitize(accu[r]);
      } else {
        store4(Uc + (size_t)(dg + li) * BT + kpos<T>(I * 16 + 4 * lg), sanitize4(accu));
      }
    }
  }
}

// ---------------------------------------------------------------------------
template <typename T>
struct StateArgs {
  const T* W;
  const T* UT;
  const T* KgT;
  const float* GL;
  const float* h0;  // nullable, (B,H,D,D)
  int N;            // chunks per (b,h)
  int S, L;         // segments per (b,h), chunks per segment (the last may be shorter)
  int summary;      // segment-summary pass (S > 1): writes `seg`, no h^T / v_new^T
  const float* hin; // S > 1 and !summary: segment entry states [bh][S][D][D]
  float* seg;       // summary: [bh][S][2][D][D] = (end state, transition M_seg)
  T* HT;
  T* VnT;
  float* h_final;
  const int* cu;    // variable-length batch (B = 1): unit (h, sequence s) scans chunks
                    // [cu[s], cu[s+1]); h0 / h_final are [s][h][D][D]
  int H;
  // Output waves (NO > 0): o = scale qg h_c + Aqk v_new formed in this kernel
  // (h^T / v_new^T are then not written)
  const T* Qg;
  const T* Aqk;
  float* out;
  float scale;
  int T_len;
  const int* cstart;  // variable-length chunk table (see PrepArgs)
  // Segmented scan (S > 1): `sat` is set to 1 when a clip of the carried state
  // binds in a segmented pass (the segments' affine combination is exact only
  // while none does); a pass with `gate` runs only if *gate is nonzero -- the
  // serial scan that then replaces the segmented result
  int* sat;
  const int* gate;
};

// One workgroup = one (b,h) and 16*NW value columns: NW compute waves (16
// columns each) and NP producer waves.  While the compute waves work on chunk
// c, the producers stream chunk c+1 (W, kg^T, g_last and this workgroup's u^T
// rows) into LDS with global_load_lds_dwordx4, wait for it and replace g_last
// by e^{g_last}.  A wave
// that issues that much memory traffic stalls at issue (at most 63 vector
// memory instructions in flight per wave), so the compute waves issue none and
// the traffic is split over several producers.  Two barriers per chunk: A
// (chunk c resident, chunk c-1's buffers free) and B (u^T of chunk c copied to
// registers, its buffer free).
//
// Segments (long sequences with few (b,h) pairs).  The chunk map
// h -> M_c h + kg_c^T u_c, M_c = Diag(e^{g_last}) - kg_c^T W_c, is affine.  With
// S > 1 segments of L chunks the scan runs in three launches: a summary pass
// over all segments in parallel gives each segment's end state from h = 0 (h0
// for segment 0) and, in NVS extra column slices that run the same recurrence
// from the identity with u = 0 and no clipping, its transition M_seg; the
// combine kernel chains the segment entry states; the final pass reruns every
// segment from its entry state, writing h^T / v_new^T.  The combine is exact
// while the +-1e4 clip of h does not bind; all three launches flag a binding
// clip (StateArgs::sat), and a flagged call is finished by the serial scan.
//
// W / kg^T tiles are stored unpadded with the 16-byte chunks of row r
// XOR-permuted by (r mod 16), so the 16 rows an MFMA operand read touches land
// in distinct LDS banks.  Float32 tiles arrive in the split pair layout
// (written so by fwd_prep, gdn2_common.h), and the two products run in the split
// form: three bfloat16 MFMAs per 32-deep k step instead of eight float32 ones,
// with h and v_new split once per chunk; the DMA moves the 16-byte chunks as
// they are.  u^T is gathered straight into the order the compute
// lanes read it (one contiguous 1 KB block per wave and row block).  The two
// halves of the W / kg^T double buffer are separate __shared__ arrays selected
// at compile time (the chunk loop is unrolled by two), so the compiler can see
// that reads of one half never alias the DMA into the other.
//
// Where two buffers do not fit in LDS (float32 at D = 256: 128 KB per chunk)
// the kernel runs single-buffered, with a third barrier E per chunk after the
// compute waves' last reads.  The two tiles are read in different phases (W
// before the K-split exchange X, kg^T after it), so the producers refill W and
// u^T after X(c) and kg^T and g_last after E(c): each move hides behind the
// other product, from L2 through the touch issued one chunk ahead.
//
// K-split (KS = 2): the two chained products of a chunk are the step's
// critical path.  Each 16-column slice then has two compute waves, each
// holding half of h's rows: both form their half of W h, exchange it through
// LDS, form the same v_new = u - (W h)_lo - (W h)_hi and update their own rows
// of h -- half the MFMA chain per wave, and all four SIMDs' matrix cores busy.
// float32 exchanges through sX (barrier X, after B); bfloat16, whose two tile
// buffers leave no room for sX, through the W tile of the current buffer once
// every compute wave has read it (barriers X1, X2).  Not at D = 64 in
// bfloat16, where the W tile is smaller than the exchanged partials.
//
// Output waves (NO > 0, inference: nothing reads h^T / v_new^T afterwards).
// The outputs o = scale qg h_c + Aqk v_new of the workgroup's columns are
// formed here instead of by fwd_out, so h_c and v_new never reach HBM.  The
// compute waves keep h_c (bfloat16, natural d order) and v_new (chained order)
// of chunk c in registers and put them into LDS (sHo, sVo) between barriers
// A and B of chunk c+1; NO output waves, each owning the row blocks
// {ow, NB-1-ow} (equal triangular work), read them from B(c+1) to A(c+2): one
// row block while the compute waves form W h (B..X), the other during their h
// update (after the last X barrier), so neither phase of the chain waits for
// them.  q_g and Aqk rows come from global memory one chunk ahead, in the
// operand-fragment order the prep writes for this path (qg_frag, aqk_frag).
// Two barriers A(n), B(n) after the last chunk hand over its tiles.  Needs a
// K-split (an X barrier per chunk) and both tile buffers.
template <typename T, int BT, int D>
constexpr int state_bufs() { return state_bufs_of(sizeof(T), BT, D); }
template <typename T, int BT, int D>
constexpr int state_ksplit() { return state_ksplit_of(sizeof(T), BT, D); }
template <typename T, int BT, int D>
constexpr int state_out_waves() { return state_out_waves_of(sizeof(T), BT, D); }

template <typename T, int BT, int D, int NW, int NP, int KS, int NO = 0>
__global__ void __launch_bounds__(64 * (NW * KS + NP + NO)) fwd_state(StateArgs<T> a) {
  using Op = typename Tr<T>::Op;
  constexpr int NB = BT / 16, NDT = D / 16;
  constexpr int NVS = D / (16 * NW);
  constexpr bool F32 = sizeof(T) == 4;
  constexpr int WBYTES = BT * D * (int)sizeof(T);   // one tile (W or kg^T)
  constexpr int BUF = 2 * WBYTES;                    // W + kg^T
  constexpr int PIECES = BUF / 1024;                 // 1 KB DMA instructions per chunk
  constexpr int NBUF = state_bufs<T, BT, D>();
  constexpr int NCW = NW * KS;                       // compute waves
  constexpr int NDH = NDT / KS;                      // row tiles of h per compute wave
  static_assert(BUF % 1024 == 0, "tiles must split into 1 KB pieces");
  // K-split exchange: through sX (float32, two parts; barrier X) or through the W
  // tile of the current buffer (barriers X1, X2)
  constexpr bool XSX = F32 && KS == 2;
  constexpr int NXB = KS == 1 ? 0 : (XSX ? 1 : 2);
  static_assert(KS == 1 || (NDT % KS == 0 && NB % KS == 0 &&
                            (XSX || NCW * NB * 1024 <= WBYTES) &&
                            (F32 || (KS == 2 && NDH % 2 == 0 && NB % 4 == 0))),
                "K-split: the parts must split into whole k-steps, and the W tile "
                "must hold the exchanged partials");
  __shared__ __align__(16) char sbuf0[BUF];
  __shared__ __align__(16) char sbuf1[NBUF == 2 ? BUF : 16];
  // u^T in compute-lane order: 16 bytes per lane and row block (float32) or
  // row-block pair (bfloat16, chained order)
  constexpr int UB = F32 ? NB : NB / 2;              // u^T pieces per compute wave
  __shared__ __align__(16) uint4 sU[NW * UB * 64];
  __shared__ __align__(16) f32x4 sX[XSX ? NCW * NB * 64 : 1];   // K-split partials of W h
  __shared__ __align__(16) float sGL0[D];
  __shared__ __align__(16) float sGL1[NBUF == 2 ? D : 4];
  __shared__ __align__(16) float sJunk[64];        // target of the L2 touches
  // output waves: h_c^T [col][d] (natural order) and v_new^T [col][t] (chained
  // order, as the v_new^T workspace tile) of the workgroup's columns
  constexpr int PADO = 16 / (int)sizeof(T);
  constexpr int HO_LD = D + PADO, VO_LD = BT + PADO;
  __shared__ __align__(16) T sHo[NO > 0 ? 16 * NW * HO_LD : 8];
  __shared__ __align__(16) T sVo[NO > 0 ? 16 * NW * VO_LD : 8];
  static_assert(NO == 0 || (NXB > 0 && NBUF == 2 && NO == NB / 2),
                "output waves need an X barrier per chunk, two tile buffers and NB/2 waves");

  if (a.gate && *a.gate == 0) return;   // whole workgroups, before any barrier
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // A unit is one (b,h) segment; it has NVS column slices (2 NVS in the summary
  // pass, the second NVS carrying M).  Workgroups are dealt round-robin over the
  // 8 XCDs (XCD = id mod 8): all slices of a unit go to one XCD so the W / kg^T
  // tiles they all stream are fetched into that XCD's L2 once.
  const int NSL = a.summary ? 2 * NVS : NVS;
  int unit, vs;
  bool one_xcd = false;   // all slices of the unit on this workgroup's XCD
  {
    const int nwg = gridDim.x, id = blockIdx.x;
    const int per_xcd = nwg / 8;
    if (nwg % 8 == 0 && per_xcd % NSL == 0) {
      const int xcd = id % 8, slot = id / 8;
      unit = xcd * (per_xcd / NSL) + slot / NSL;
      vs = slot % NSL;
      one_xcd = true;
    } else {
      unit = id / NSL;
      vs = id % NSL;
    }
  }
  const int bh = unit / a.S, sg = unit % a.S;
  const bool mslice = vs >= NVS;             // summary pass: columns of M_seg
  if (mslice && sg == 0) return;             // segment 0 starts from h0: no M needed
  if (mslice) vs -= NVS;
  int c0, n;                                 // chunks [c0, c0 + n) of this unit
  if (a.cu) {
    const SeqChunks sc = seq_chunks(a.cu, sg, a.N);
    c0 = sc.c0;
    n = sc.n;
  } else {
    c0 = sg * a.L;
    n = a.N - c0;
    n = n < a.L ? n : a.L;
  }
  n = n > 0 ? n : 0;

  if constexpr (NO > 0) {
    if (wv >= NCW + NP) {
      // ---- output waves --------------------------------------------------------
      // wave ow owns row blocks {ow, NB-1-ow} of every chunk and all 16 NW
      // columns of the workgroup; out(c) is formed during chunk c+1 (after F for
      // the last chunk) from sHo / sVo and the q_g / Aqk rows loaded one chunk
      // ahead.  The barriers mirror the compute waves' A, B, X.. per chunk and F.
      constexpr int TKC = Tr<T>::KC, TKS = Tr<T>::KS;
      constexpr int OKD = D / TKS, OKT = BT / TKS;
      const int ow = wv - NCW - NP;
      const int hh = bh % a.H, bb = bh / a.H;
      const size_t HD = (size_t)a.H * D;
      auto oblock = [&](int i) { return i == 0 ? ow : NB - 1 - ow; };
      Op qf[2][OKD], af[2][OKT];
      // q_g and Aqk in operand-fragment order (the prep's frag layout): one
      // 16-byte load per operand, 1 KB contiguous per wave
      auto load_ops = [&](int c) __attribute__((always_inline)) {
        const size_t cid = (size_t)bh * a.N + c0 + c;
        const T* qc = a.Qg + cid * BT * D;
        const T* ac = a.Aqk + cid * BT * BT;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int It = oblock(i);
#pragma unroll
          for (int kg = 0; kg < OKD; ++kg) qf[i][kg] = op_load<T>(qc + qg_frag<T, BT, D>(It, kg, lane));
          // Aqk blocks right of the diagonal block are never written: masked
#pragma unroll
          for (int kg = 0; kg < OKT; ++kg) {
            if constexpr (sizeof(T) == 4) {
              af[i][kg] = kg <= It ? op_load<T>(ac + aqk_frag<T, BT>(It, kg, lane)) : op_zero<T>();
            } else {
              af[i][kg] = 2 * kg <= It ? op_load<T>(ac + aqk_frag<T, BT>(It, 2 * kg, lane))
                                       : op_zero<T>();
            }
          }
        }
      };
      // out(c) rows of own row block i
      auto emit = [&](int c, int i) __attribute__((always_inline)) {
        const ChunkRows cr = chunk_rows(a.cstart, c0 + c, bb, a.T_len, BT);
        float* obase = a.out + cr.row0 * HD + (size_t)hh * D + vs * 16 * NW;
        {
          const int It = oblock(i), t = It * 16 + li;
          const int kgmax = (It * 16 + 15) / TKS;
#pragma unroll
          for (int vt = 0; vt < NW; ++vt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kg = 0; kg < OKD; ++kg)
              mma(acc, op_load<T>(&sHo[(vt * 16 + li) * HO_LD + kg * TKS + lg * TKC]), qf[i][kg]);
            acc *= a.scale;
#pragma unroll
            for (int kg = 0; kg < OKT; ++kg)
              if (kg <= kgmax) {
                Op y = af[i][kg];
                if constexpr (sizeof(T) == 2) {
                  if (2 * kg + 1 > It) {   // block 2kg+1 lies right of the diagonal
#pragma unroll
                    for (int e = 4; e < 8; ++e) y[e] = (T)0.f;
                  }
                }
                mma(acc, op_load<T>(&sVo[(vt * 16 + li) * VO_LD + kg * TKS + lg * TKC]), y);
              }
            if (t < cr.valid) store4(obase + (size_t)t * HD + vt * 16 + 4 * lg, sanitize4(acc));
          }
        }
      };
      // chunk c-1's tiles are in sHo / sVo from B(c) to A(c+1): one row block
      // while the compute waves form W h (B..X), the other during their h update
      if (n > 0) load_ops(0);
      for (int c = 0; c < n; ++c) {
        lds_barrier();  // A(c)
        lds_barrier();  // B(c)
        if (c > 0) emit(c - 1, 0);
        for (int x = 0; x < NXB; ++x) lds_barrier();  // X(c)
        if (c > 0) {
          emit(c - 1, 1);
          load_ops(c);
        }
      }
      lds_barrier();  // A(n)
      lds_barrier();  // B(n)
      if (n > 0) {
        emit(n - 1, 0);
        emit(n - 1, 1);
      }
      return;
    }
  }

  if (wv >= NCW) {
    // ---- producers ----------------------------------------------------------
    // producer p moves W / kg^T pieces [p PP, (p+1) PP) and u^T blocks q = p mod NP
    constexpr int ROWB_W = D * (int)sizeof(T), ROWB_K = BT * (int)sizeof(T);
    constexpr int WPIECES = WBYTES / 1024;
    constexpr int PP = PIECES / NP;
    static_assert(PIECES % NP == 0 && (NW * UB) % NP == 0, "work must split evenly");
    const int p = wv - NCW;
    // parts: 1 the W / kg^T tiles and g_last, 2 the u^T blocks, 3 both
    auto issue = [&](int c, char* base, float* gl, int parts = 3) __attribute__((always_inline)) {
      const size_t cid = (size_t)bh * a.N + c0 + c;
      const char* wsrc = reinterpret_cast<const char*>(a.W + cid * BT * D);
      const char* ksrc = reinterpret_cast<const char*>(a.KgT + cid * D * BT);
#pragma unroll
      for (int i = 0; i < ((parts & 1) ? PP : 0); ++i) {
        const int piece = p * PP + i;                      // wave-uniform
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
      if ((parts & 1) && p == NP - 1 && lane < D / 4) lds_dma16(a.GL + cid * D + lane * 4, gl);
      if (!(parts & 2)) return;
      // u^T[col][t] for compute wave w, piece q: lane (li, lg) of that wave gets
      // the 16 bytes at u^T[16 w + li][16 q + 4 lg] (float32: row block q) or
      // [32 q + 8 lg] (bfloat16: row blocks 2q, 2q+1, chained), at sU[(w UB + q) 64 + lane]
      if (mslice) return;  // M columns: u = 0
      constexpr int EPP = 16 / sizeof(T);              // elements per piece per lane
      const T* usrc = a.UT + cid * D * BT + (size_t)(vs * 16 * NW + li) * BT + EPP * lg;
#pragma unroll
      for (int j = 0; j < NW * UB / NP; ++j) {
        const int q = j * NP + p, w = q / UB, it = q % UB;
        lds_dma16(usrc + (size_t)w * 16 * BT + it * 4 * EPP, &sU[q * 64]);
      }
    };
    // L2 touch of chunk c: one 4-byte DMA into a junk slot per 128-byte line of
    // everything issue(c) will read, spread over the producers.  Issued one
    // chunk ahead of the DMA, it turns the DMA's HBM latency into L2 latency.
    // The W / kg^T lines are read by every column slice of the unit: when the
    // slices share an XCD (one L2) slice v touches only the v-th share of them
    // (a touch per line and workgroup cost the scan a fifth of its time), every
    // slice its own u^T rows.
    constexpr int LINE = 128;
    constexpr int LW = WBYTES / LINE;                       // lines per W / kg^T tile
    constexpr int LUR = BT * (int)sizeof(T) / LINE;         // lines per u^T row
    constexpr int LU = 16 * NW * LUR;                       // this workgroup's u^T rows
    constexpr int LG = (D * 4 + LINE - 1) / LINE;           // g_last
    // At chunk 64 the output waves' q_g and Aqk tiles are touched too, shared
    // among the slices like W / kg^T (the touch count assumes that sharing;
    // without it, lines past the count are left to the loads themselves): a
    // step there (about 1.7 us) is shorter than the HBM latency of the operand
    // loads issued one step ahead (fused scan 0.265 -> 0.217 ms).  A chunk-128
    // step lasts long enough, and the extra touches cost more than they save
    // (0.205 -> 0.213 ms).
    constexpr bool TQA = NO > 0 && BT == 64;
    constexpr int LQ = TQA ? BT * D * (int)sizeof(T) / LINE : 0;    // q_g
    constexpr int LA = TQA ? BT * BT * (int)sizeof(T) / LINE : 0;   // Aqk
    constexpr int LSH = 2 * LW + LQ + LA;                   // lines shared by the slices
    constexpr int LTOT = TQA ? (LSH + NVS - 1) / NVS + LU + LG   // at most (one slice)
                             : LSH + LU + LG;
    constexpr int NTP = ((LTOT + 63) / 64 + NP - 1) / NP;   // touch instructions per producer
    const int vsl = vs + (mslice ? NVS : 0);                // slice index within the unit
    const int lws = one_xcd ? (LSH + NSL - 1) / NSL : LSH;  // shared lines touched here
    const int lw0 = one_xcd ? vsl * lws : 0;
    const int ltot = lws + LU + LG;
    auto touch = [&](int c) __attribute__((always_inline)) {
      const size_t cid = (size_t)bh * a.N + c0 + c;
      const char* wsrc = reinterpret_cast<const char*>(a.W + cid * BT * D);
      const char* ksrc = reinterpret_cast<const char*>(a.KgT + cid * D * BT);
      const char* qsrc = reinterpret_cast<const char*>(a.Qg + cid * BT * D);
      const char* asrc = reinterpret_cast<const char*>(a.Aqk + cid * BT * BT);
      const char* usrc =
          reinterpret_cast<const char*>(a.UT + cid * D * BT + (size_t)vs * 16 * NW * BT);
      const char* gsrc = reinterpret_cast<const char*>(a.GL + cid * D);
#pragma unroll
      for (int j = 0; j < NTP; ++j) {
        int l = (j * NP + p) * 64 + lane;
        l = l < ltot ? l : ltot - 1;
        const int lw = min(lw0 + l, LSH - 1);                   // shared line
        const char* sh = lw < LW ? wsrc + lw * LINE
                       : lw < 2 * LW ? ksrc + (lw - LW) * LINE
                       : lw < 2 * LW + LQ ? qsrc + (lw - 2 * LW) * LINE
                       : asrc + (lw - 2 * LW - LQ) * LINE;
        const char* src = l < lws ? sh
                        : l < lws + LU ? usrc + (l - lws) * LINE
                        : gsrc + (l - lws - LU) * LINE;
        lds_dma4(src, sJunk);
      }
    };
    // In flight at the top of chunk c: issue(c), then touch(c+1) if c+1 < n.
    auto wait_chunk = [&](int c) __attribute__((always_inline)) {
      if (c + 1 < n) wait_vmcnt<NTP>();
      else wait_vmcnt<0>();
    };
    // The producers' data ordering is the explicit vmcnt wait; a plain barrier
    // (no fence) keeps the compiler from also waiting for the L2 touches.
    auto barrier = []() __attribute__((always_inline)) {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    // g_last -> e^{g_last} in place, once per chunk, by the producer that moved it
    auto exp_gl = [&](float* gl) __attribute__((always_inline)) {
      if (p == NP - 1) {
#pragma unroll
        for (int i = 0; i < (D + 63) / 64; ++i)
          if (i * 64 + lane < D) gl[i * 64 + lane] = __expf(gl[i * 64 + lane]);
      }
    };
    if constexpr (NBUF == 1) {
      // One tile buffer: W and u^T of chunk c+1 move in once barrier X(c) has
      // passed (the compute waves are done with W(c) and u^T(c)), kg^T and g_last
      // once E(c) has passed, so each move hides behind the other product of the
      // chain (kg^T v_new of chunk c, then W h of chunk c+1).  Every producer
      // moves the same counts: its share of the W pieces and u^T blocks, then its
      // share of the kg^T pieces and of g_last, which it exponentiates itself.
      constexpr int PPW = WPIECES / NP, PPK = (PIECES - WPIECES) / NP, GQ = D / NP;
      static_assert(WPIECES % NP == 0 && (PIECES - WPIECES) % NP == 0 && NXB == 1 &&
                        GQ % 4 == 0 && GQ <= 64,
                    "single-buffer split: equal shares per producer, one X barrier");
      auto piece_dma = [&](const char* wsrc, const char* ksrc, int piece) __attribute__((always_inline)) {
        char* dst = sbuf0 + piece * 1024;
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
      };
      auto issue_w = [&](int c) __attribute__((always_inline)) {
        const size_t cid = (size_t)bh * a.N + c0 + c;
        const char* wsrc = reinterpret_cast<const char*>(a.W + cid * BT * D);
#pragma unroll
        for (int i = 0; i < PPW; ++i) piece_dma(wsrc, nullptr, p * PPW + i);
        if (mslice) return;  // M columns: u = 0
        constexpr int EPP = 16 / sizeof(T);
        const T* usrc = a.UT + cid * D * BT + (size_t)(vs * 16 * NW + li) * BT + EPP * lg;
#pragma unroll
        for (int j = 0; j < NW * UB / NP; ++j) {
          const int q = j * NP + p, w = q / UB, it = q % UB;
          lds_dma16(usrc + (size_t)w * 16 * BT + it * 4 * EPP, &sU[q * 64]);
        }
      };
      auto issue_k = [&](int c) __attribute__((always_inline)) {
        const size_t cid = (size_t)bh * a.N + c0 + c;
        const char* ksrc = reinterpret_cast<const char*>(a.KgT + cid * D * BT);
#pragma unroll
        for (int i = 0; i < PPK; ++i) piece_dma(nullptr, ksrc, WPIECES + p * PPK + i);
        if (lane < GQ / 4) lds_dma16(a.GL + cid * D + p * GQ + lane * 4, sGL0 + p * GQ);
      };
      auto exp_q = [&]() __attribute__((always_inline)) {
        if (lane < GQ) sGL0[p * GQ + lane] = __expf(sGL0[p * GQ + lane]);
      };
      if (n > 0) {
        issue_w(0);
        issue_k(0);
      }
      if (n > 1) touch(1);
      for (int c = 0; c < n; ++c) {
        // in flight here (c > 0): W / u^T of chunk c, then kg^T / g_last of chunk
        // c (PPK + 1), then touch(c+1) if c+1 < n (NTP)
        const bool tch = c + 1 < n;
        if (c == 0) {
          if (tch) wait_vmcnt<NTP>();
          else wait_vmcnt<0>();
          exp_q();
        } else {
          if (tch) wait_vmcnt<PPK + 1 + NTP>();
          else wait_vmcnt<PPK + 1>();
        }
        barrier();  // A(c): W(c), u^T(c) resident
        barrier();  // B(c)
        if (c > 0) {
          if (tch) wait_vmcnt<NTP>();
          else wait_vmcnt<0>();
          exp_q();
        }
        barrier();  // X(c): kg^T(c), e^{g_last(c)} resident; W(c) no longer read
        if (c + 1 < n) issue_w(c + 1);
        barrier();  // E(c): kg^T(c) no longer read
        if (c + 1 < n) {
          issue_k(c + 1);
          if (c + 2 < n) touch(c + 2);
        }
      }
      return;
    }
    if (n > 0) issue(0, sbuf0, sGL0);
    if (n > 1) touch(1);
    // float32: the next chunk's W / kg^T / g_last move once A(c) has passed (their
    // buffer was last read in chunk c-1), its u^T once B(c) has (one u^T buffer,
    // read between A(c) and B(c)); the touch comes last, so waiting for all but
    // the touch waits for both.  The MFMA-bound float32 step gains the head start
    // (training scan 0.458 -> 0.437 ms); the latency-bound bfloat16 steps lost
    // (0.210 -> 0.229 ms at chunk 128) and issue everything after B(c).
    constexpr int EARLY = F32 ? 1 : 0;
    for (int c = 0; c < n; c += 2) {
      wait_chunk(c);
      exp_gl(sGL0);
      barrier();  // A(c)
      if (EARLY && c + 1 < n) issue(c + 1, sbuf1, sGL1, 1);
      barrier();  // B(c)
      if (c + 1 < n) {
        issue(c + 1, sbuf1, sGL1, EARLY ? 2 : 3);
        if (c + 2 < n) touch(c + 2);
        for (int x = 0; x < NXB; ++x) barrier();  // X(c)
        wait_chunk(c + 1);
        exp_gl(sGL1);
        barrier();  // A(c+1)
        if (EARLY && c + 2 < n) issue(c + 2, sbuf0, sGL0, 1);
        barrier();  // B(c+1)
        if (c + 2 < n) issue(c + 2, sbuf0, sGL0, EARLY ? 2 : 3);
        if (c + 3 < n) touch(c + 3);
        for (int x = 0; x < NXB; ++x) barrier();  // X(c+1)
      } else {
        for (int x = 0; x < NXB; ++x) barrier();  // X(c)
      }
    }
    if constexpr (NO > 0) {
      barrier();  // A(n)
      barrier();  // B(n)
    }
    return;
  }

  // ---- compute waves ----------------------------------------------------------
  const int wcol = wv % NW, ks = wv / NW;          // column slice, k-half (K-split)
  const int col = vs * 16 * NW + wcol * 16 + li;
  // element offset of logical (row r, element e) in a tile whose rows hold `re` elements
  auto swz = [](int r, int e, int re) {
    constexpr int EPC = 16 / sizeof(T);           // elements per 16-byte chunk
    const int nchunk = re / EPC;
    const int m = (nchunk < 16 ? nchunk : 16) - 1;
    const int j = e / EPC;
    return r * re + ((j ^ (r & m)) * EPC) + (e % EPC);
  };

  // entry state: h0 (or 0) for a plain pass and for segment 0 of the summary
  // pass, 0 for later segments of the summary pass, the identity for M slices,
  // the combined entry state in the final segmented pass
  f32x4 h[NDH];   // row tiles at = ks NDH + i of this slice's h
  const float* hsrc = a.cu ? (a.h0 ? a.h0 + ((size_t)sg * a.H + bh) * D * D : nullptr)
                    : (a.S > 1 && !a.summary) ? a.hin + ((size_t)unit) * D * D
                    : (sg == 0 && !mslice && a.h0) ? a.h0 + (size_t)bh * D * D : nullptr;
  if (mslice) {
#pragma unroll
    for (int i = 0; i < NDH; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        h[i][r] = ((ks * NDH + i) * 16 + 4 * lg + r == col) ? 1.f : 0.f;
  } else if (hsrc) {
#pragma unroll
    for (int i = 0; i < NDH; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        h[i][r] = sanitize(hsrc[(size_t)((ks * NDH + i) * 16 + 4 * lg + r) * D + col]);
  } else {
#pragma unroll
    for (int i = 0; i < NDH; ++i) h[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bool write_tiles = !a.summary;
  // segmented passes: whether a clip of the state bound (NaN included)
  const bool track = a.sat != nullptr && !mslice;
  bool bound = false;

  // One chunk: v_new = u - W h, h <- e^{gl} h + kg^T v_new, with chunk c in `cur`.
  // output waves: the pieces of chunk c-1's h^T / v_new^T this wave puts into
  // sHo / sVo between barriers A(c) and B(c)
  using HP = typename std::conditional<F32, f32x4, bf16x4>::type;
  constexpr int NVP = F32 ? NB / KS : NB / 2 / KS;
  HP hp[NO > 0 ? NDH : 1];
  Op vp[NO > 0 ? NVP : 1];
  auto put_tiles = [&]() __attribute__((always_inline)) {
    const int lc = wcol * 16 + li;
#pragma unroll
    for (int i = 0; i < NDH; ++i)
      *reinterpret_cast<HP*>(&sHo[lc * HO_LD + (ks * NDH + i) * 16 + 4 * lg]) = hp[i];
#pragma unroll
    for (int j = 0; j < NVP; ++j) {
      if constexpr (F32) store4(&sVo[lc * VO_LD + (ks * NVP + j) * 16 + 4 * lg], vp[j]);
      else *reinterpret_cast<Op*>(&sVo[lc * VO_LD + (ks * NVP + j) * 32 + 8 * lg]) = vp[j];
    }
  };

  auto step = [&](int c, const char* cur, const float* eglc) __attribute__((always_inline)) {
    const size_t cid = (size_t)bh * a.N + c0 + c;
    __syncthreads();  // A(c)
    f32x4 vn[NB];
#pragma unroll
    for (int q = 0; q < UB; ++q) {
      const uint4 pc = sU[(wcol * UB + q) * 64 + lane];
      if constexpr (F32) {
        vn[q] = mslice ? f32x4{0.f, 0.f, 0.f, 0.f} : __builtin_bit_cast(f32x4, pc);
      } else {
        const bf16x8 e = __builtin_bit_cast(bf16x8, pc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          vn[2 * q][r] = mslice ? 0.f : (float)e[r];
          vn[2 * q + 1][r] = mslice ? 0.f : (float)e[4 + r];
        }
      }
    }
    if constexpr (NO > 0) {
      if (c > 0) put_tiles();
    }
    __syncthreads();  // B(c)
    const T* sW = reinterpret_cast<const T*>(cur);
    const T* sK = reinterpret_cast<const T*>(cur + WBYTES);

    T* hT = a.HT + cid * D * D + (size_t)col * D;
    if (!write_tiles || NO > 0) {
    } else if constexpr (F32) {
#pragma unroll
      for (int i = 0; i < NDH; ++i) store4(hT + (ks * NDH + i) * 16 + 4 * lg, h[i]);
    } else {
#pragma unroll
      for (int p = 0; p < NDH / 2; ++p)
        *reinterpret_cast<Op*>(hT + (ks * NDH / 2 + p) * 32 + 8 * lg) =
            op_from_c(h[2 * p], h[2 * p + 1], (Op*)nullptr);
    }

    // v_new -= W h.  The NB row blocks are independent accumulators: the k-step
    // loop is outermost, so consecutive MFMAs never wait on each other, and the
    // next k-step's W operands are read while this one's MFMAs run.
    {
      constexpr int NKD = F32 ? NDH : NDH / 2;   // k-steps over this wave's d
      Op hb[NKD];
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk) {
        if constexpr (F32) hb[kk] = h[kk];
        else hb[kk] = op_from_c(h[2 * kk], h[2 * kk + 1], (Op*)nullptr);
      }
      auto wop = [&](int it, int kk) __attribute__((always_inline)) {
        const int r = it * 16 + li;
        if constexpr (F32) return load4f(&sW[swz(r, (ks * NDH + kk) * 16 + 4 * lg, D)]);
        else return op_load<T>(&sW[swz(r, (ks * NKD + kk) * 32 + 8 * lg, D)]);
      };
      f32x4 acc[NB];
      if constexpr (F32) {
        // split form: h split once per chunk; the W tile holds the split pairs
        // (chunks 2p, 2p+1 of a lane are one pair), all row blocks independent
        static_assert(NKD % 2 == 0, "pairs of k-groups");
        Split8 hs[NKD / 2];
#pragma unroll
        for (int p = 0; p < NKD / 2; ++p) hs[p] = split8(hb[2 * p], hb[2 * p + 1]);
#pragma unroll
        for (int it = 0; it < NB; ++it) acc[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < NKD / 2; ++p)
#pragma unroll
          for (int it = 0; it < NB; ++it)
            mma3(acc[it], split_read(wop(it, 2 * p), wop(it, 2 * p + 1)), hs[p]);
      } else {
        // bfloat16: one accumulator chain at a time (a chain of dependent
        // 16x16x32 MFMAs issues faster than interleaved accumulators); the next
        // row block's W operands are read while this one's chain runs
        Op wc[NKD], wn[NKD];
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk) wc[kk] = wop(0, kk);
#pragma unroll
        for (int it = 0; it < NB; ++it) {
          if (it + 1 < NB) {
#pragma unroll
            for (int kk = 0; kk < NKD; ++kk) wn[kk] = wop(it + 1, kk);
          }
          acc[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < NKD; ++kk) mma(acc[it], wc[kk], hb[kk]);
#pragma unroll
          for (int kk = 0; kk < NKD; ++kk) wc[kk] = wn[kk];
        }
      }
      if constexpr (KS > 1) {
        // exchange the parts; every wave of the slice sums them in the order of
        // the k-parts, so all form the same v_new
        f32x4* xb = sX;
        if constexpr (!XSX) {
          lds_barrier();  // X1(c): every compute wave is done with the W tile
          xb = reinterpret_cast<f32x4*>(const_cast<char*>(cur));
        }
#pragma unroll
        for (int it = 0; it < NB; ++it) xb[(wv * NB + it) * 64 + lane] = acc[it];
        lds_barrier();  // X(c), X2(c)
#pragma unroll
        for (int it = 0; it < NB; ++it) {
          f32x4 sum = ks == 0 ? acc[it] : xb[(wcol * NB + it) * 64 + lane];
#pragma unroll
          for (int q = 1; q < KS; ++q)
            sum += ks == q ? acc[it] : xb[((q * NW + wcol) * NB + it) * 64 + lane];
          vn[it] -= sum;
        }
      } else {
#pragma unroll
        for (int it = 0; it < NB; ++it) vn[it] -= acc[it];
      }
    }
    T* vT = a.VnT + cid * D * BT + (size_t)col * BT;
    if constexpr (NO > 0) {
      // h_c and v_new of chunk c, kept for the output waves (put into LDS at the
      // start of chunk c+1): h^T in natural d order (lane (li, lg) holds
      // d = 16 i + 4 lg + r of row tile i), v_new^T in chained order
#pragma unroll
      for (int i = 0; i < NDH; ++i) {
        if constexpr (F32) hp[i] = h[i];
        else hp[i] = HP{(T)h[i][0], (T)h[i][1], (T)h[i][2], (T)h[i][3]};
      }
#pragma unroll
      for (int j = 0; j < NVP; ++j) {
        if constexpr (F32) vp[j] = vn[ks * NVP + j];
        else vp[j] = op_from_c(vn[2 * (ks * NVP + j)], vn[2 * (ks * NVP + j) + 1], (Op*)nullptr);
      }
    } else if (!write_tiles) {
    } else if constexpr (F32) {
#pragma unroll
      for (int it = ks * (NB / KS); it < (ks + 1) * (NB / KS); ++it)
        store4(vT + it * 16 + 4 * lg, vn[it]);
    } else {
#pragma unroll
      for (int p = ks * (NB / 2 / KS); p < (ks + 1) * (NB / 2 / KS); ++p)
        *reinterpret_cast<Op*>(vT + p * 32 + 8 * lg) = op_from_c(vn[2 * p], vn[2 * p + 1], (Op*)nullptr);
    }

    // h <- e^{g_last} h + kg^T v_new (the row tiles of h are independent
    // accumulators)
    {
      constexpr int NKT = F32 ? NB : NB / 2;     // k-steps over t
#pragma unroll
      for (int i = 0; i < NDH; ++i) {
        const f32x4 egl = load4f(eglc + (ks * NDH + i) * 16 + 4 * lg);
#pragma unroll
        for (int r = 0; r < 4; ++r) h[i][r] *= egl[r];
      }
      auto kop = [&](int i, int kk) __attribute__((always_inline)) {
        const int r = (ks * NDH + i) * 16 + li;
        if constexpr (F32) return load4f(&sK[swz(r, kk * 16 + 4 * lg, BT)]);
        else return op_load<T>(&sK[swz(r, kk * 32 + 8 * lg, BT)]);
      };
      if constexpr (F32) {
        // split form: v_new split once per chunk; the kg^T tile holds the split
        // pairs, all row tiles of h independent
        static_assert(NKT % 2 == 0, "pairs of k-groups");
        Split8 vs2[NKT / 2];
#pragma unroll
        for (int p = 0; p < NKT / 2; ++p) vs2[p] = split8(vn[2 * p], vn[2 * p + 1]);
#pragma unroll
        for (int p = 0; p < NKT / 2; ++p)
#pragma unroll
          for (int at = 0; at < NDH; ++at)
            mma3(h[at], split_read(kop(at, 2 * p), kop(at, 2 * p + 1)), vs2[p]);
      } else {
        // bfloat16: one chain per row tile of h, as for W h above
        Op vb[NKT], kc2[NKT], kn2[NKT];
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk) {
          vb[kk] = op_from_c(vn[2 * kk], vn[2 * kk + 1], (Op*)nullptr);
          kc2[kk] = kop(0, kk);
        }
#pragma unroll
        for (int at = 0; at < NDH; ++at) {
          if (at + 1 < NDH) {
#pragma unroll
            for (int kk = 0; kk < NKT; ++kk) kn2[kk] = kop(at + 1, kk);
          }
#pragma unroll
          for (int kk = 0; kk < NKT; ++kk) mma(h[at], kc2[kk], vb[kk]);
#pragma unroll
          for (int kk = 0; kk < NKT; ++kk) kc2[kk] = kn2[kk];
        }
      }
      if (!mslice) {
        if (track) {
#pragma unroll
          for (int at = 0; at < NDH; ++at)
#pragma unroll
            for (int r2 = 0; r2 < 4; ++r2) bound = bound || !(fabsf(h[at][r2]) <= g_clip);
        }
#pragma unroll
        for (int at = 0; at < NDH; ++at)
#pragma unroll
          for (int r2 = 0; r2 < 4; ++r2) h[at][r2] = sanitize(h[at][r2]);
      }
    }
  };

  if constexpr (NBUF == 1) {
    for (int c = 0; c < n; ++c) {
      step(c, sbuf0, sGL0);
      __syncthreads();  // E(c)
    }
  } else {
    for (int c = 0; c < n; c += 2) {
      step(c, sbuf0, sGL0);
      if (c + 1 < n) step(c + 1, sbuf1, sGL1);
    }
  }
  if constexpr (NO > 0) {
    __syncthreads();  // A(n): the output waves are done with chunk n-2's tiles
    if (n > 0) put_tiles();
    __syncthreads();  // B(n)
  }
  if (track && __ballot(bound) != 0 && lane == 0) *a.sat = 1;
  float* hout = a.cu ? a.h_final + ((size_t)sg * a.H + bh) * D * D
              : a.summary ? a.seg + ((size_t)unit * 2 + (mslice ? 1 : 0)) * D * D
              : (sg == a.S - 1) ? a.h_final + (size_t)bh * D * D : nullptr;
  if (hout) {
#pragma unroll
    for (int i = 0; i < NDH; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        hout[(size_t)((ks * NDH + i) * 16 + 4 * lg + r) * D + col] = h[i][r];
  }
}

// ---------------------------------------------------------------------------
// Segment entry states of a segmented state scan: hin_0 = h0 (or 0), hin_1 =
// e_0 (segment 0's end state, computed from h0), hin_{s+1} = M_s hin_s + e_s
// (e_s from h = 0), sanitized like every chunk state.  The columns of h are
// independent: one workgroup per (b,h) and 16-column slice, serial over the
// segments; wave w produces the row tiles w, w+4, ...  The slice of the current
// state sits transposed in LDS as the chained operand of the next product.
template <int D>
__global__ void __launch_bounds__(256) seg_combine(const float* seg, const float* h0, float* hin,
                                                   int S, int* sat) {
  constexpr int NDT = D / 16;
  __shared__ __align__(16) float sHT[16 * (D + 4)];   // current state, [col][row]
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int bh = blockIdx.x / NDT, c0 = (blockIdx.x % NDT) * 16;
  const size_t DD = (size_t)D * D;
  const float* segb = seg + (size_t)bh * S * 2 * DD;   // [s][2][D][D]
  float* hinb = hin + (size_t)bh * S * DD;             // [s][D][D]
  // hin_0 and hin_1
  for (int i = tid; i < D * 16; i += 256) {
    const int r = i / 16, cc = i % 16;
    const size_t o = (size_t)r * D + c0 + cc;
    hinb[o] = h0 ? sanitize(h0[(size_t)bh * DD + o]) : 0.f;
    const float e0 = segb[o];
    hinb[DD + o] = e0;
    sHT[cc * (D + 4) + r] = e0;
  }
  __syncthreads();
  bool bound = false;   // a clip of an entry state bound (see StateArgs::sat)
  for (int s = 1; s + 1 < S; ++s) {
    const float* M = segb + ((size_t)s * 2 + 1) * DD;
    const float* e = segb + (size_t)s * 2 * DD;
    f32x4 acc[(NDT + 3) / 4];
#pragma unroll
    for (int j = 0; j < (NDT + 3) / 4; ++j) {
      const int at = wv + 4 * j;
      acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (at < NDT) {
#pragma unroll
        for (int kt = 0; kt < NDT; ++kt)
          mma(acc[j], load4f(M + (size_t)(at * 16 + li) * D + kt * 16 + 4 * lg),
              load4f(&sHT[li * (D + 4) + kt * 16 + 4 * lg]));
      }
    }
    __syncthreads();  // every wave has read the current state
#pragma unroll
    for (int j = 0; j < (NDT + 3) / 4; ++j) {
      const int at = wv + 4 * j;
      if (at < NDT) {
        // acc[j] holds (M h)^T: lane (li, lg) has rows at*16 + 4lg + r of column li
        f32x4 nh;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t o = (size_t)(at * 16 + 4 * lg + r) * D + c0 + li;
          const float x = acc[j][r] + e[o];
          bound = bound || !(fabsf(x) <= g_clip);
          nh[r] = sanitize(x);
          hinb[(size_t)(s + 1) * DD + o] = nh[r];
        }
        store4(&sHT[li * (D + 4) + at * 16 + 4 * lg], nh);
      }
    }
    __syncthreads();
  }
  if (__ballot(bound) != 0 && lane == 0) *sat = 1;
}

// ---------------------------------------------------------------------------
template <typename T>
struct OutArgs {
  const T* Qg;
  const T* Aqk;
  const T* HT;
  const T* VnT;
  int T_len, H, N;
  float scale;
  float* out;
  const int* cstart;  // variable-length batch chunk table (see PrepArgs)
};

// o = scale qg h_c + Aqk v_new per chunk (gdn2_fwd.py:349-353), computed as
// o^T tiles so each lane stores 4 consecutive floats of an output row.  One
// workgroup per chunk and slice of out_cols() value columns: float32 at
// D = 128 in 64-column slices (a 32 KB h^T slice: two workgroups per CU;
// whole 128 columns, one per CU, took 1.5x as long), at D = 256 in 32-column
// slices (the same 32 KB), bfloat16 in slices of up to 128 columns.
template <typename T, int D>
constexpr int out_cols() {
  return sizeof(T) == 4 ? (D < 128 ? D : 8192 / D) : (D < 128 ? D : 128);
}

template <typename T, int BT, int D>
__global__ void __launch_bounds__(256) fwd_out(OutArgs<T> a) {
  using Op = typename Tr<T>::Op;
  constexpr int KC = Tr<T>::KC, KS = Tr<T>::KS;
  constexpr int DVS = out_cols<T, D>();   // value columns per workgroup
  constexpr int NSL = D / DVS;
  constexpr int NB = BT / 16, NBW = (NB + 3) / 4, NDT = DVS / 16;
  constexpr int NKD = D / KS, NKT = BT / KS;
  constexpr int PADT = 16 / sizeof(T);
  constexpr int H_LD = D + PADT, V_LD = BT + PADT;
  __shared__ __align__(16) T sH[DVS * H_LD];
  __shared__ __align__(16) T sV[DVS * V_LD];

  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  // a chunk's column slices on one XCD: its q_g and Aqk are fetched once into that L2
  const UnitPart up = xcd_split(blockIdx.x, gridDim.x, NSL);
  const int cid = up.unit, sl = up.part;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;

  // All global loads are issued before the first LDS store: the qg / Aqk
  // operand rows of both own row blocks, then the h^T and v_new^T tiles.
  // h^T and v_new^T are stored in chained order over d and t (kpos), so qg and
  // Aqk are read in the matching chained pattern.  Aqk blocks right of the
  // diagonal block are never written: masked per 16-token block.
  Op qf[NBW][NKD], af[NBW][NKT];
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int It = own_block<NB>(wv, i);
    const int t = It * 16 + li;
    const T* qrow = a.Qg + (size_t)cid * BT * D + (size_t)t * D;
    const T* arow = a.Aqk + (size_t)cid * BT * BT + (size_t)t * BT;
#pragma unroll
    for (int kg = 0; kg < NKD; ++kg) qf[i][kg] = op_chained(qrow + kg * KS, lg);
#pragma unroll
    for (int kg = 0; kg < NKT; ++kg) {
      if constexpr (sizeof(T) == 4) {
        const int s0 = kg * KS + lg * KC;
        af[i][kg] = (s0 <= It * 16 + 15) ? op_load<T>(arow + s0) : op_zero<T>();
      } else {
        const bf16x4 z = {(T)0.f, (T)0.f, (T)0.f, (T)0.f};
        const bf16x4 lo = (2 * kg <= It)
            ? *reinterpret_cast<const bf16x4*>(arow + kg * 32 + 4 * lg) : z;
        const bf16x4 hi = (2 * kg + 1 <= It)
            ? *reinterpret_cast<const bf16x4*>(arow + kg * 32 + 16 + 4 * lg) : z;
        af[i][kg] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
  }
  {
    constexpr int EPV = 16 / sizeof(T);                  // elements per 16-byte piece
    constexpr int NH = DVS * D / EPV / 256, NV = DVS * BT / EPV / 256;
    static_assert(DVS * D % (EPV * 256) == 0 && DVS * BT % (EPV * 256) == 0,
                  "tiles split evenly");
    uint4 rh[NH], rv[NV];
    // rows [sl DVS, (sl+1) DVS) of h^T [col][d] and v_new^T [col][t]
    const uint4* gh = reinterpret_cast<const uint4*>(a.HT + ((size_t)cid * D + sl * DVS) * D);
    const uint4* gv = reinterpret_cast<const uint4*>(a.VnT + ((size_t)cid * D + sl * DVS) * BT);
#pragma unroll
    for (int u = 0; u < NH; ++u) rh[u] = gh[tid + 256 * u];
#pragma unroll
    for (int u = 0; u < NV; ++u) rv[u] = gv[tid + 256 * u];
#pragma unroll
    for (int u = 0; u < NH; ++u) {
      const int i = tid + 256 * u, r = i / (D / EPV), cc = (i % (D / EPV)) * EPV;
      *reinterpret_cast<uint4*>(&sH[r * H_LD + cc]) = rh[u];
    }
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int i = tid + 256 * u, r = i / (BT / EPV), cc = (i % (BT / EPV)) * EPV;
      *reinterpret_cast<uint4*>(&sV[r * V_LD + cc]) = rv[u];
    }
  }
  __syncthreads();

  const size_t HD = (size_t)a.H * D;
  const ChunkRows cr = chunk_rows(a.cstart, c, bb, a.T_len, BT);
  float* obase = a.out + cr.row0 * HD + (size_t)hh * D + sl * DVS;
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int It = own_block<NB>(wv, i);
    const int t = It * 16 + li;
    const int kgmax = (It * 16 + 15) / KS;
#pragma unroll
    for (int vt = 0; vt < NDT; ++vt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kg = 0; kg < NKD; ++kg)
        mma(acc, op_load<T>(&sH[(vt * 16 + li) * H_LD + kg * KS + lg * KC]), qf[i][kg]);
      acc *= a.scale;
#pragma unroll
      for (int kg = 0; kg < NKT; ++kg)
        if (kg <= kgmax)
          mma(acc, op_load<T>(&sV[(vt * 16 + li) * V_LD + kg * KS + lg * KC]), af[i][kg]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = sanitize(acc[r]);
      if (t < cr.valid) store4(obase + (size_t)t * HD + vt * 16 + 4 * lg, acc);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers (called from gdn2_api.cpp).
template <typename T, typename TG, int BT, int D, typename TI>
hipError_t launch_fwd(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                      const void* v, const void* w, const void* b, const void* g,
                      const float* h0, float scale, float* out, float* h_final, char* ws,
                      float* a_dbg, int flags, const Varlen* vl) {
  const int N = vl ? vl->total_chunks : (T_len + BT - 1) / BT;
  const size_t NC = (size_t)B * H * N;
  // the segment count follows flags only (the workspace was sized from them): the
  // final pass of an inference forward is the 32-column scan with output waves
  constexpr int NO = state_out_waves<T, BT, D>();
  const bool fuse_ws = NO > 0 && !(flags & 1);
  const int S_ws = vl ? 1
                      : state_segments((long long)B * H, N, D, (int)sizeof(T), (flags >> 8) & 0xff,
                                       fuse_ws ? 32 : seg_pass_cols(sizeof(T), D));
  // Inference (no residuals kept): the scan forms the outputs itself where its
  // variant has output waves (state_out_waves), fwd_out is not launched and the
  // h^T / v_new^T tiles have no region (a variable-length workspace keeps them:
  // its size does not depend on flags)
  const bool fuse = fuse_ws && !a_dbg;
  const size_t seg_units = S_ws > 1 ? (size_t)B * H * S_ws : 0;
  const FwdLayout L = fwd_layout(NC, BT, D, sizeof(T), seg_units, !(flags & kFwdNoARegion),
                                 !fuse || vl != nullptr);
  T* W = reinterpret_cast<T*>(ws + L.W);
  T* UT = reinterpret_cast<T*>(ws + L.UT);
  T* KgT = reinterpret_cast<T*>(ws + L.KgT);
  T* Qg = reinterpret_cast<T*>(ws + L.Qg);
  T* Aqk = reinterpret_cast<T*>(ws + L.Aqk);
  float* GL = reinterpret_cast<float*>(ws + L.GL);
  T* HT = reinterpret_cast<T*>(ws + L.HT);
  T* VnT = reinterpret_cast<T*>(ws + L.VnT);
  // segmented scan: its saturation flag, in the last slot of SEG
  int* sat = seg_units ? reinterpret_cast<int*>(ws + L.SEG + seg_flag_offset(seg_units, D))
                       : nullptr;
  launch_mark(st);
  if (NC > 0) {
    PrepArgs<T, TG, TI> pa{(const TI*)q, (const TI*)k, (const TI*)v, (const TI*)w, (const TI*)b,
                       (const TG*)g, T_len, H, N, (long long)NC, scale, W, UT, KgT, Qg, Aqk, GL,
                       a_dbg ? a_dbg : ((flags & 1) ? reinterpret_cast<float*>(ws + L.A)
                                                    : nullptr),
                       (flags & 2) ? 1 : 0, vl ? vl->cstart : nullptr, fuse ? 1 : 0, sat};
    hipLaunchKernelGGL((fwd_prep<T, TG, BT, D, TI>), dim3(NC), dim3(64 * prep_waves(BT)), 0, st,
                       pa);
  }
  launch_mark(st);
  constexpr int SW = 2;  // compute waves (16 value columns each) per state workgroup
  constexpr int SP = 4;  // producer waves (DMA issue: 4 beat 2 by 14 % on float32 scans)
  constexpr int SK = state_ksplit<T, BT, D>();   // compute waves per column slice
  constexpr int NVS = D / (16 * SW);
  const size_t BH = (size_t)B * H;
  const int S = S_ws;
  constexpr int NTH = 64 * (SW * SK + SP), NTHO = 64 * (SW * SK + SP + NO);
  if (vl) {
    // one unit per (head, sequence)
    StateArgs<T> va{W,  UT,      KgT,     GL,     h0,           N,  vl->nseq, 0, 0, nullptr,
                    nullptr, HT, VnT, h_final, vl->cu_chunks, H, Qg, Aqk, out, scale, T_len,
                    vl->cstart};
    if (vl->nseq > 0) {
      if (fuse)
        hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK, NO>), dim3(BH * vl->nseq * NVS),
                           dim3(NTHO), 0, st, va);
      else
        hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK>), dim3(BH * vl->nseq * NVS),
                           dim3(NTH), 0, st, va);
    }
  } else if (S > 1) {
    // Segmented passes (several workgroups per CU's worth of units): bfloat16 at
    // D >= 128 takes 64 columns per workgroup (four compute waves, no K-split),
    // so the summary pass, which doubles the units with the M slices, fits the
    // device in one round (1.1x faster than 32-column workgroups in two rounds)
    constexpr int GW = seg_pass_cols(sizeof(T), D) / 16;
    constexpr int GK = GW == SW ? SK : 1;
    constexpr int GVS = D / (16 * GW);
    const int Lseg = (N + S - 1) / S;
    float* seg = reinterpret_cast<float*>(ws + L.SEG);          // [bh][S][2][D][D]
    float* hin = seg + BH * S * 2 * (size_t)D * D;               // [bh][S][D][D]
    StateArgs<T> sum{W, UT, KgT, GL, h0, N, S, Lseg, 1, nullptr, seg, HT, VnT, h_final,
                     nullptr, H, Qg, Aqk, out, scale, T_len, nullptr, sat, nullptr};
    hipLaunchKernelGGL((fwd_state<T, BT, D, GW, SP, GK>), dim3(BH * S * 2 * GVS),
                       dim3(64 * (GW * GK + SP)), 0, st, sum);
    hipLaunchKernelGGL((seg_combine<D>), dim3(BH * (D / 16)), dim3(256), 0, st, seg, h0, hin,
                       S, sat);
    StateArgs<T> fin{W, UT, KgT, GL, h0, N, S, Lseg, 0, hin, nullptr, HT, VnT, h_final,
                     nullptr, H, Qg, Aqk, out, scale, T_len, nullptr, sat, nullptr};
    if (fuse)   // final pass with output waves: 32-column workgroups
      hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK, NO>), dim3(BH * S * NVS), dim3(NTHO),
                         0, st, fin);
    else
      hipLaunchKernelGGL((fwd_state<T, BT, D, GW, SP, GK>), dim3(BH * S * GVS),
                         dim3(64 * (GW * GK + SP)), 0, st, fin);
    // A clip of the state bound somewhere in the segmented passes: the segments'
    // affine combination does not hold, and the serial scan (the plain pass below)
    // recomputes everything the final pass wrote; otherwise its workgroups return
    // at once
    StateArgs<T> ser{W, UT, KgT, GL, h0, N, 1, N, 0, nullptr, nullptr, HT, VnT, h_final,
                     nullptr, H, Qg, Aqk, out, scale, T_len, nullptr, nullptr, sat};
    if (fuse)
      hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK, NO>), dim3(BH * NVS), dim3(NTHO), 0,
                         st, ser);
    else
      hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK>), dim3(BH * NVS), dim3(NTH), 0, st,
                         ser);
  } else {
    StateArgs<T> sa{W, UT, KgT, GL, h0, N, 1, N, 0, nullptr, nullptr, HT, VnT, h_final,
                    nullptr, H, Qg, Aqk, out, scale, T_len, nullptr};
    if (fuse)
      hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK, NO>), dim3(BH * NVS), dim3(NTHO), 0,
                         st, sa);
    else
      hipLaunchKernelGGL((fwd_state<T, BT, D, SW, SP, SK>), dim3(BH * NVS), dim3(NTH), 0, st,
                         sa);
  }
  launch_mark(st);
  if (NC > 0 && !fuse) {
    OutArgs<T> oa{Qg, Aqk, HT, VnT, T_len, H, N, scale, out, vl ? vl->cstart : nullptr};
    hipLaunchKernelGGL((fwd_out<T, BT, D>), dim3(NC * (D / out_cols<T, D>())), dim3(256), 0,
                       st, oa);
  }
  launch_mark(st);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The reference's forward stages one at a time: float32 tiles at chunk 64, the
// reference's (B,H,N,BT,.) layouts.

// Kernel A (build_chunk_scores_pallas): Aqk, Akk [cid][64][64].
template <typename TG, int D, typename TI>
hipError_t launch_stage_scores(hipStream_t st, int B, int T_len, int H, const void* q,
                               const void* k, const void* b, const void* g, float scale,
                               float* aqk, float* akk) {
  const int N = T_len / 64;
  const size_t NC = (size_t)B * H * N;
  if (NC > 0) {
    PrepArgs<float, TG, TI> pa{};
    pa.q = (const TI*)q;
    pa.k = (const TI*)k;
    pa.b = (const TI*)b;
    pa.g = (const TG*)g;
    pa.T_len = T_len;
    pa.H = H;
    pa.N = N;
    pa.NC = (long long)NC;
    pa.scale = scale;
    pa.Aqk = aqk;
    pa.akk_out = akk;
    hipLaunchKernelGGL((fwd_prep<float, TG, 64, D, TI, kPrepScores>), dim3(NC),
                       dim3(64 * prep_waves(64)), 0, st, pa);
  }
  return hipGetLastError();
}

// Kernel B (wy_solve_pallas): A = (I + Akk)^{-1} per [64][64] chunk tile, from
// the strictly lower part of Akk.
hipError_t launch_stage_solve(hipStream_t st, size_t nchunks, const float* akk, float* a_out) {
  if (nchunks > 0) {
    PrepArgs<float, float, float> pa{};
    pa.T_len = 64;
    pa.H = 1;
    pa.N = 1;
    pa.NC = (long long)nchunks;
    pa.a_in = akk;
    pa.a_dbg = a_out;
    hipLaunchKernelGGL((fwd_prep<float, float, 64, 64, float, kPrepSolve>), dim3(nchunks),
                       dim3(64 * prep_waves(64)), 0, st, pa);
  }
  return hipGetLastError();
}

// Kernel C (recompute_wy_pallas): w_pseudo, u, kg, qg [cid][64][D] and gc_last
// [cid][D] from the inputs and a given A [cid][64][64].
template <typename TG, int D, typename TI>
hipError_t launch_stage_wy(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                           const void* v, const void* w, const void* b, const void* g,
                           const float* A, float* w_pseudo, float* u, float* kg, float* qg,
                           float* gc_last) {
  const int N = T_len / 64;
  const size_t NC = (size_t)B * H * N;
  if (NC > 0) {
    PrepArgs<float, TG, TI> pa{};
    pa.q = (const TI*)q;
    pa.k = (const TI*)k;
    pa.v = (const TI*)v;
    pa.w = (const TI*)w;
    pa.b = (const TI*)b;
    pa.g = (const TG*)g;
    pa.T_len = T_len;
    pa.H = H;
    pa.N = N;
    pa.NC = (long long)NC;
    pa.W = w_pseudo;
    pa.UT = u;
    pa.KgT = kg;
    pa.Qg = qg;
    pa.GL = gc_last;
    pa.a_in = A;
    hipLaunchKernelGGL((fwd_prep<float, TG, 64, D, TI, kPrepWy>), dim3(NC),
                       dim3(64 * prep_waves(64)), 0, st, pa);
  }
  return hipGetLastError();
}

// Kernel D (gdn2_inter_chunk_combine(_with_state)): the serial state scan and the
// outputs over given per-chunk tiles.  u and kg are transposed into the scan's
// [D][BT] layout in `ws` (combine_layout); out is (B, N*64, H, D); h_pre_all
// [cid][D][D] (h entering the chunk, [dk][dv]) and v_new_all [cid][64][D] are
// written when not null.
template <int D>
hipError_t launch_stage_combine(hipStream_t st, int B, int N, int H, const float* aqk,
                                const float* w_pseudo, const float* u, const float* kg,
                                const float* qg, const float* gc_last, const float* h0,
                                float scale, float* out, float* h_final, float* h_pre_all,
                                float* v_new_all, char* ws) {
  constexpr int BT = 64;
  const size_t NC = (size_t)B * H * N;
  const CombineLayout L = combine_layout(NC, BT, D);
  float* UT = reinterpret_cast<float*>(ws + L.UT);
  float* KgT = reinterpret_cast<float*>(ws + L.KgT);
  float* Wsp = reinterpret_cast<float*>(ws + L.W);
  float* HT = reinterpret_cast<float*>(ws + L.HT);
  float* VnT = reinterpret_cast<float*>(ws + L.VnT);
  const int T_len = N * BT;
  transpose_all(st, u, UT, NC, BT, D);
  transpose_all(st, kg, KgT, NC, BT, D);
  // the scan's float32 tiles in the split pair layout, as fwd_prep writes them
  split_runs(st, KgT, KgT, NC * D * BT / 32);
  split_runs(st, w_pseudo, Wsp, NC * BT * D / 32);
  constexpr int SW = 2, SP = 4, SK = state_ksplit<float, BT, D>();
  constexpr int NVS = D / (16 * SW);
  StateArgs<float> sa{Wsp, UT, KgT, gc_last, h0, N, 1, N, 0, nullptr, nullptr, HT, VnT,
                      h_final, nullptr, H, qg, aqk, out, scale, T_len, nullptr};
  hipLaunchKernelGGL((fwd_state<float, BT, D, SW, SP, SK>), dim3((size_t)B * H * NVS),
                     dim3(64 * (SW * SK + SP)), 0, st, sa);
  if (NC > 0) {
    OutArgs<float> oa{qg, aqk, HT, VnT, T_len, H, N, scale, out, nullptr};
    hipLaunchKernelGGL((fwd_out<float, BT, D>), dim3(NC * (D / out_cols<float, D>())),
                       dim3(256), 0, st, oa);
  }
  if (h_pre_all) transpose_all(st, HT, h_pre_all, NC, D, D);
  if (v_new_all) transpose_all(st, VnT, v_new_all, NC, D, BT);
  return hipGetLastError();
}

#define GDN2_INST_STAGE(TG, D, TI)                                                            \
  template hipError_t launch_stage_scores<TG, D, TI>(hipStream_t, int, int, int, const void*,  \
                                                     const void*, const void*, const void*,    \
                                                     float, float*, float*);                   \
  template hipError_t launch_stage_wy<TG, D, TI>(hipStream_t, int, int, int, const void*,      \
                                                 const void*, const void*, const void*,        \
                                                 const void*, const void*, const float*,       \
                                                 float*, float*, float*, float*, float*);
GDN2_INST_STAGE(float, 64, float)
GDN2_INST_STAGE(float, 128, float)
GDN2_INST_STAGE(float, 256, float)
GDN2_INST_STAGE(float, 64, bf16_t)
GDN2_INST_STAGE(float, 128, bf16_t)
GDN2_INST_STAGE(float, 256, bf16_t)
GDN2_INST_STAGE(bf16_t, 64, bf16_t)
GDN2_INST_STAGE(bf16_t, 128, bf16_t)
GDN2_INST_STAGE(bf16_t, 256, bf16_t)
#define GDN2_INST_COMBINE(D)                                                                   \
  template hipError_t launch_stage_combine<D>(hipStream_t, int, int, int, const float*,        \
                                              const float*, const float*, const float*,        \
                                              const float*, const float*, const float*, float, \
                                              float*, float*, float*, float*, char*);
GDN2_INST_COMBINE(64)
GDN2_INST_COMBINE(128)
GDN2_INST_COMBINE(256)

#define GDN2_INST_FWD(T, TG, BT, D, TI)                                                      \
  template hipError_t launch_fwd<T, TG, BT, D, TI>(hipStream_t, int, int, int, const void*, \
                                                   const void*, const void*, const void*,   \
                                                   const void*, const void*, const float*,  \
                                                   float, float*, float*, char*, float*, int, \
                                                   const Varlen*);

GDN2_INST_FWD(float, float, 64, 64, float)
GDN2_INST_FWD(float, float, 64, 128, float)
GDN2_INST_FWD(bf16_t, float, 64, 64, bf16_t)
GDN2_INST_FWD(bf16_t, float, 64, 128, bf16_t)
GDN2_INST_FWD(bf16_t, float, 128, 64, bf16_t)
GDN2_INST_FWD(bf16_t, float, 128, 128, bf16_t)
GDN2_INST_FWD(bf16_t, bf16_t, 64, 64, bf16_t)
GDN2_INST_FWD(bf16_t, bf16_t, 64, 128, bf16_t)
GDN2_INST_FWD(bf16_t, bf16_t, 128, 64, bf16_t)
GDN2_INST_FWD(bf16_t, bf16_t, 128, 128, bf16_t)
GDN2_INST_FWD(float, float, 64, 256, float)
GDN2_INST_FWD(bf16_t, float, 64, 256, bf16_t)
GDN2_INST_FWD(bf16_t, bf16_t, 64, 256, bf16_t)
// float32 arithmetic on bfloat16 inputs (GDN2_BF16_F32)
GDN2_INST_FWD(float, float, 64, 64, bf16_t)
GDN2_INST_FWD(float, float, 64, 128, bf16_t)
GDN2_INST_FWD(float, float, 64, 256, bf16_t)
GDN2_INST_FWD(float, bf16_t, 64, 64, bf16_t)
GDN2_INST_FWD(float, bf16_t, 64, 128, bf16_t)
GDN2_INST_FWD(float, bf16_t, 64, 256, bf16_t)

// This translation unit's clip bound on the current device (gdn2_set_clip).
hipError_t set_clip_fwd(float c) { return set_unit_clip(c); }

}  // namespace gdn2
