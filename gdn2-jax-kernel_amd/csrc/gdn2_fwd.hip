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
// masked.  All exponents are formed from in-block partial sums, so they never
// subtract two large prefix sums.  This is exact math; the reference's +-20
// clip of gc_i - gc_j (gdn2_fwd.py:125) is not applied (it changes results by
// < exp(-20) * |q||k| in the documented input domain).

#include "gdn2_common.h"
#include "gdn2_layout.h"

namespace gdn2 {

template <typename T, typename TG>
struct PrepArgs {
  const T *q, *k, *v, *w, *b;
  const TG* g;
  int T_len, H, N;
  float scale;
  T* W;
  float* UT;
  T* KgT;
  T* Qg;
  T* Aqk;
  float* GL;
  float* a_dbg;  // optional A = (I + Akk)^{-1} output (BT x BT fp32 per chunk)
};

// Own row blocks of wave `wv`: {wv} and, for 8 blocks, {7 - wv} -- equal work
// for the triangular loops.
template <int NB>
__device__ __forceinline__ int own_block(int wv, int i) {
  return i == 0 ? wv : NB - 1 - wv;
}

template <typename T, typename TG, int BT, int D>
__global__ void __launch_bounds__(256) fwd_prep(PrepArgs<T, TG> a) {
  using Op = typename Tr<T>::Op;
  constexpr int KC = Tr<T>::KC, KS = Tr<T>::KS;
  constexpr int NB = BT / 16;             // 16-token row blocks
  constexpr int NBW = (NB + 3) / 4;       // row blocks per wave
  constexpr int NKD = D / KS;             // k-groups over channels
  constexpr int NKT = BT / KS;            // k-groups over tokens
  constexpr int DQ = NKD * KC;            // channels owned per lane (= D/4)
  constexpr int PADT = 16 / sizeof(T);
  constexpr int KH_LD = D + PADT;         // sKh  [t][d]
  constexpr int TT_LD = BT + PADT;        // sKbdT, sWVT [d][t]
  constexpr int A_LD = BT + 4;            // sA   [t][s] fp32
  constexpr int R0 = (BT * KH_LD > D * TT_LD) ? BT * KH_LD : D * TT_LD;

  __shared__ __align__(16) T sR0[R0];         // khat [t][d]; later (w v)^T [d][t]
  __shared__ __align__(16) T sKbdT[D * TT_LD];
  __shared__ __align__(16) float sA[BT * A_LD];
  __shared__ __align__(16) float sTot[NB * D];  // per-block sums of g
  __shared__ __align__(16) float sETot[NB * D]; // exp of those
  __shared__ __align__(16) float sPre[NB * D];  // sum of the blocks before m
  __shared__ __align__(16) float sSuf[NB * D];  // sum of the blocks after m

  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int cid = blockIdx.x;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  const size_t HD = (size_t)a.H * D;
  const size_t tok0 = ((size_t)bb * a.T_len + (size_t)c * BT) * HD + (size_t)hh * D;
  auto rowp = [&](int t) { return tok0 + (size_t)t * HD; };
  auto chan = [&](int x) { return (x / KC) * KS + lg * KC + (x % KC); };

  for (int i = tid; i < BT * A_LD / 4; i += 256)
    reinterpret_cast<f32x4*>(sA)[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- 1. in-block inclusive cumsum of g (lanes li = tokens) ----------------
  float loc[NBW][DQ];
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int I = own_block<NB>(wv, i);
    const size_t off = rowp(I * 16 + li);
#pragma unroll
    for (int j = 0; j < NKD; ++j) load_f<KC>(a.g + off + j * KS + lg * KC, &loc[i][j * KC]);
#pragma unroll
    for (int x = 0; x < DQ; ++x) {
      float s = loc[i][x];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        float y = __shfl_up(s, o, 16);
        if (li >= o) s += y;
      }
      loc[i][x] = s;
    }
    if (li == 15) {
#pragma unroll
      for (int x = 0; x < DQ; ++x) sTot[I * D + chan(x)] = loc[i][x];
    }
  }
  __syncthreads();
  for (int i = tid; i < NB * D; i += 256) sETot[i] = __expf(sTot[i]);
  if (tid < D) {
    float run = 0.f;
#pragma unroll
    for (int m = 0; m < NB; ++m) { sPre[m * D + tid] = run; run += sTot[m * D + tid]; }
    run = 0.f;
#pragma unroll
    for (int m = NB - 1; m >= 0; --m) { sSuf[m * D + tid] = run; run += sTot[m * D + tid]; }
    a.GL[(size_t)cid * D + tid] = sPre[(NB - 1) * D + tid] + sTot[(NB - 1) * D + tid];
  }
  __syncthreads();

  // ---- 2. per-token factors, qg/kg/kbd/khat, diagonal score blocks ----------
  float aq[NBW][DQ], ak[NBW][DQ];
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int I = own_block<NB>(wv, i);
    const int t = I * 16 + li;
    const size_t off = rowp(t);
    float qv[DQ], kv[DQ], bv[DQ];
#pragma unroll
    for (int j = 0; j < NKD; ++j) {
      load_f<KC>(a.q + off + j * KS + lg * KC, &qv[j * KC]);
      load_f<KC>(a.k + off + j * KS + lg * KC, &kv[j * KC]);
      load_f<KC>(a.b + off + j * KS + lg * KC, &bv[j * KC]);
    }
    float dq[DQ], dk[DQ], db[DQ], qg[DQ];
    T* kgT = a.KgT + (size_t)cid * D * BT;
#pragma unroll
    for (int x = 0; x < DQ; ++x) {
      const int ch = chan(x);
      const float pre = sPre[I * D + ch], suf = sSuf[I * D + ch];
      const float tot = sTot[I * D + ch];
      const float lc = loc[i][x];
      const float lcm = __shfl(lc, 7, 16);
      const float egc = __expf(pre + lc);
      const float eloc = __expf(lc);
      const float bk = bv[x] * kv[x];
      qg[x] = sanitize(qv[x] * egc);
      sKbdT[ch * TT_LD + t] = from_f<T>(bk * egc);
      kgT[(size_t)ch * BT + t] = from_f<T>(sanitize(kv[x] * __expf(suf + (tot - lc))));
      sR0[t * KH_LD + ch] = from_f<T>(kv[x] * __expf(tot - lc));
      aq[i][x] = qv[x] * eloc;
      ak[i][x] = bk * eloc;
      const float edq = __expf(lc - lcm), edk = __expf(lcm - lc);
      dq[x] = qv[x] * edq;
      db[x] = bk * edq;
      dk[x] = kv[x] * edk;
    }
    T* qgp = a.Qg + (size_t)cid * BT * D + (size_t)t * D;
#pragma unroll
    for (int j = 0; j < NKD; ++j) {
      Op o = op_from<T>(&qg[j * KC]);
      *reinterpret_cast<Op*>(qgp + j * KS + lg * KC) = o;
    }
    // diagonal block: X = k rows (j), Y = q / bk rows (i) -> lane holds [i=li][j=4lg+r]
    f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NKD; ++j) {
      Op xo = op_from<T>(&dk[j * KC]);
      mma(accq, xo, op_from<T>(&dq[j * KC]));
      mma(acck, xo, op_from<T>(&db[j * KC]));
    }
    f32x4 sq, sk;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int jj = 4 * lg + r;
      sq[r] = (jj <= li) ? sanitize(a.scale * accq[r]) : 0.f;
      sk[r] = (jj < li) ? sanitize(acck[r]) : 0.f;
    }
    store4(a.Aqk + (size_t)cid * BT * BT + (size_t)t * BT + I * 16 + 4 * lg, sq);
    store4(&sA[t * A_LD + I * 16 + 4 * lg], sk);
  }
  __syncthreads();

  // ---- 3. off-diagonal score blocks (I > J) on MFMA --------------------------
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int I = own_block<NB>(wv, i);
    const int t = I * 16 + li;
    float F[DQ];
#pragma unroll
    for (int x = 0; x < DQ; ++x) F[x] = 1.f;
    for (int J = I - 1; J >= 0; --J) {
      f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NKD; ++j) {
        float yq[KC], yk[KC];
#pragma unroll
        for (int e = 0; e < KC; ++e) {
          yq[e] = aq[i][j * KC + e] * F[j * KC + e];
          yk[e] = ak[i][j * KC + e] * F[j * KC + e];
        }
        Op xo = op_load<T>(&sR0[(J * 16 + li) * KH_LD + j * KS + lg * KC]);
        mma(accq, xo, op_from<T>(yq));
        mma(acck, xo, op_from<T>(yk));
      }
      f32x4 sq, sk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sq[r] = sanitize(a.scale * accq[r]);
        sk[r] = sanitize(acck[r]);
      }
      store4(a.Aqk + (size_t)cid * BT * BT + (size_t)t * BT + J * 16 + 4 * lg, sq);
      store4(&sA[t * A_LD + J * 16 + 4 * lg], sk);
#pragma unroll
      for (int x = 0; x < DQ; ++x) F[x] *= sETot[J * D + chan(x)];
    }
  }
  __syncthreads();

  // ---- 4. A = (I + Akk)^{-1}: diagonal blocks by substitution ---------------
  if (lg < NBW) {
    const int I = own_block<NB>(wv, lg);
    const int j = li;
    const float* blk = &sA[(I * 16) * A_LD + I * 16];
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float s = (r == j) ? 1.f : 0.f;
#pragma unroll
      for (int kk = 0; kk < r; ++kk) s -= blk[r * A_LD + kk] * x[kk];
      x[r] = sanitize(s);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sA[(I * 16 + r) * A_LD + I * 16 + j] = x[r];
  }
  __syncthreads();

  // ---- 4b. off-diagonal blocks, one column chain per (wave, column) ---------
  //   X_IJ = -X_II * sum_{K=J}^{I-1} L_IK X_KJ, X_KJ kept in C layout.
  f32x4 X[NBW][NB];
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int J = own_block<NB>(wv, i);
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      X[i][I] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (I > J) {
        f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int K = 0; K < NB; ++K) {
          if (K >= J && K < I) {
            f32x4 y;
            if (K == J) {
#pragma unroll
              for (int r = 0; r < 4; ++r) y[r] = sA[(J * 16 + 4 * lg + r) * A_LD + J * 16 + li];
            } else {
              y = X[i][K];
            }
            const f32x4 xo = load4f(&sA[(I * 16 + li) * A_LD + K * 16 + 4 * lg]);
            mma(S, xo, y);
          }
        }
        const f32x4 xii = load4f(&sA[(I * 16 + li) * A_LD + I * 16 + 4 * lg]);
        f32x4 R = {0.f, 0.f, 0.f, 0.f};
        mma(R, xii, S);
#pragma unroll
        for (int r = 0; r < 4; ++r) X[i][I][r] = sanitize(-R[r]);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int J = own_block<NB>(wv, i);
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      if (I > J) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sA[(I * 16 + 4 * lg + r) * A_LD + J * 16 + li] = X[i][I][r];
      }
    }
  }
  // ---- 5. (w v)^T into LDS ----------------------------------------------------
  T* sWVT = sR0;
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int I = own_block<NB>(wv, i);
    const int t = I * 16 + li;
    const size_t off = rowp(t);
    float wv_[DQ], vv[DQ];
#pragma unroll
    for (int j = 0; j < NKD; ++j) {
      load_f<KC>(a.w + off + j * KS + lg * KC, &wv_[j * KC]);
      load_f<KC>(a.v + off + j * KS + lg * KC, &vv[j * KC]);
    }
#pragma unroll
    for (int x = 0; x < DQ; ++x) sWVT[chan(x) * TT_LD + t] = from_f<T>(wv_[x] * vv[x]);
  }
  __syncthreads();

  if (a.a_dbg) {
    float* dst = a.a_dbg + (size_t)cid * BT * BT;
    for (int i = tid; i < BT * BT; i += 256) dst[i] = sA[(i / BT) * A_LD + (i % BT)];
  }

  // ---- 6. w_pseudo = A (b k e^gc), u = A (w v) ------------------------------
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int I = own_block<NB>(wv, i);
    const int kgmax = (I * 16 + 15) / KS;
    Op af[NKT];
#pragma unroll
    for (int kg = 0; kg < NKT; ++kg) {
      float tmp[KC];
#pragma unroll
      for (int e = 0; e < KC; e += 4) {
        f32x4 v4 = load4f(&sA[(I * 16 + li) * A_LD + kg * KS + lg * KC + e]);
        tmp[e] = v4[0]; tmp[e + 1] = v4[1]; tmp[e + 2] = v4[2]; tmp[e + 3] = v4[3];
      }
      af[kg] = op_from<T>(tmp);
    }
    T* Wc = a.W + (size_t)cid * BT * D;
    float* Uc = a.UT + (size_t)cid * D * BT;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      f32x4 accw = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kg = 0; kg < NKT; ++kg) {
        if (kg <= kgmax) {
          mma(accw, op_load<T>(&sKbdT[(dt * 16 + li) * TT_LD + kg * KS + lg * KC]), af[kg]);
          mma(accu, af[kg], op_load<T>(&sWVT[(dt * 16 + li) * TT_LD + kg * KS + lg * KC]));
        }
      }
      f32x4 sw, su;
#pragma unroll
      for (int r = 0; r < 4; ++r) { sw[r] = sanitize(accw[r]); su[r] = sanitize(accu[r]); }
      store4(Wc + (size_t)(I * 16 + li) * D + dt * 16 + 4 * lg, sw);
      store4(Uc + (size_t)(dt * 16 + li) * BT + I * 16 + 4 * lg, su);
    }
  }
}

// ---------------------------------------------------------------------------
template <typename T>
struct StateArgs {
  const T* W;
  const float* UT;
  const T* KgT;
  const float* GL;
  const float* h0;  // nullable, (B,H,D,D)
  int N;
  T* HT;
  T* VnT;
  float* h_final;
};

// One workgroup = one (b,h) and 64 value columns; wave wv owns 16 columns.
// The next chunk's W, kg^T (whole workgroup, registers) and u^T, gc_last
// (per wave) are fetched while the current chunk is computed.
template <typename T, int BT, int D>
__global__ void __launch_bounds__(256) fwd_state(StateArgs<T> a) {
  using Op = typename Tr<T>::Op;
  constexpr int NB = BT / 16, NDT = D / 16;
  constexpr int EPV = 16 / sizeof(T);
  constexpr int W_LD = D + EPV, K_LD = BT + EPV;
  constexpr int NVS = D / 64;
  constexpr bool F32 = sizeof(T) == 4;
  constexpr int PW = BT * D / EPV / 256;  // uint4 per thread for W (same for kg^T)
  __shared__ __align__(16) T sW[BT * W_LD];
  __shared__ __align__(16) T sK[D * K_LD];

  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int bh = blockIdx.x / NVS, vs = blockIdx.x % NVS;
  const int v0 = vs * 64 + wv * 16;
  const int col = v0 + li;

  f32x4 h[NDT];
#pragma unroll
  for (int at = 0; at < NDT; ++at)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      h[at][r] = a.h0 ? sanitize(a.h0[((size_t)bh * D + at * 16 + 4 * lg + r) * D + col]) : 0.f;

  uint4 pw[PW], pk[PW];
  f32x4 un[NB], gn[NDT];
#define GDN2_STATE_FETCH(c_)                                                          \
  {                                                                                   \
    const size_t fcid = (size_t)bh * a.N + (c_);                                      \
    const uint4* ws = reinterpret_cast<const uint4*>(a.W + fcid * BT * D);            \
    const uint4* ks = reinterpret_cast<const uint4*>(a.KgT + fcid * D * BT);          \
    _Pragma("unroll") for (int i = 0; i < PW; ++i) {                                  \
      pw[i] = ws[tid + 256 * i];                                                      \
      pk[i] = ks[tid + 256 * i];                                                      \
    }                                                                                 \
    const float* up = a.UT + fcid * D * BT + (size_t)col * BT;                        \
    _Pragma("unroll") for (int it = 0; it < NB; ++it) un[it] = load4f(up + it * 16 + 4 * lg); \
    const float* glc = a.GL + fcid * D;                                               \
    _Pragma("unroll") for (int at = 0; at < NDT; ++at) gn[at] = load4f(glc + at * 16 + 4 * lg); \
  }
#define GDN2_STATE_COMMIT()                                                           \
  {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < PW; ++i) {                                  \
      const int iw = tid + 256 * i;                                                   \
      const int rw = iw / (D / EPV), cw = iw % (D / EPV);                             \
      *reinterpret_cast<uint4*>(&sW[rw * W_LD + cw * EPV]) = pw[i];                   \
      const int rk = iw / (BT / EPV), ck = iw % (BT / EPV);                           \
      *reinterpret_cast<uint4*>(&sK[rk * K_LD + ck * EPV]) = pk[i];                   \
    }                                                                                 \
  }
  if (a.N > 0) {
    GDN2_STATE_FETCH(0)
    GDN2_STATE_COMMIT()
  }
  __syncthreads();

  for (int c = 0; c < a.N; ++c) {
    const size_t cid = (size_t)bh * a.N + c;
    f32x4 vn[NB], gl[NDT];
#pragma unroll
    for (int it = 0; it < NB; ++it) vn[it] = un[it];
#pragma unroll
    for (int at = 0; at < NDT; ++at) gl[at] = gn[at];
    if (c + 1 < a.N) GDN2_STATE_FETCH(c + 1)

    T* hT = a.HT + cid * D * D + (size_t)col * D;
#pragma unroll
    for (int at = 0; at < NDT; ++at) store4(hT + at * 16 + 4 * lg, h[at]);

#pragma unroll
    for (int it = 0; it < NB; ++it) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (F32) {
#pragma unroll
        for (int at = 0; at < NDT; ++at)
          mma(acc, op_chained(&sW[(it * 16 + li) * W_LD + at * 16], lg), h[at]);
      } else {
#pragma unroll
        for (int p = 0; p < NDT / 2; ++p)
          mma(acc, op_chained(&sW[(it * 16 + li) * W_LD + p * 32], lg),
              op_from_c(h[2 * p], h[2 * p + 1], (Op*)nullptr));
      }
      vn[it] -= acc;
    }
    T* vT = a.VnT + cid * D * BT + (size_t)col * BT;
#pragma unroll
    for (int it = 0; it < NB; ++it) store4(vT + it * 16 + 4 * lg, vn[it]);

#pragma unroll
    for (int at = 0; at < NDT; ++at) {
#pragma unroll
      for (int r = 0; r < 4; ++r) h[at][r] *= __expf(gl[at][r]);
      if constexpr (F32) {
#pragma unroll
        for (int it = 0; it < NB; ++it)
          mma(h[at], op_chained(&sK[(at * 16 + li) * K_LD + it * 16], lg), vn[it]);
      } else {
#pragma unroll
        for (int p = 0; p < NB / 2; ++p)
          mma(h[at], op_chained(&sK[(at * 16 + li) * K_LD + p * 32], lg),
              op_from_c(vn[2 * p], vn[2 * p + 1], (Op*)nullptr));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) h[at][r] = sanitize(h[at][r]);
    }
    __syncthreads();
    if (c + 1 < a.N) GDN2_STATE_COMMIT()
    __syncthreads();
  }
#pragma unroll
  for (int at = 0; at < NDT; ++at)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      a.h_final[((size_t)bh * D + at * 16 + 4 * lg + r) * D + col] = h[at][r];
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
};

// o = scale qg h_c + Aqk v_new per chunk (gdn2_fwd.py:349-353), computed as
// o^T tiles so each lane stores 4 consecutive floats of an output row.
template <typename T, int BT, int D>
__global__ void __launch_bounds__(256) fwd_out(OutArgs<T> a) {
  using Op = typename Tr<T>::Op;
  constexpr int KC = Tr<T>::KC, KS = Tr<T>::KS;
  constexpr int NB = BT / 16, NBW = (NB + 3) / 4, NDT = D / 16;
  constexpr int NKD = D / KS, NKT = BT / KS;
  constexpr int PADT = 16 / sizeof(T);
  constexpr int H_LD = D + PADT, V_LD = BT + PADT;
  __shared__ __align__(16) T sH[D * H_LD];
  __shared__ __align__(16) T sV[D * V_LD];

  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int cid = blockIdx.x;
  const int c = cid % a.N, bh = cid / a.N, hh = bh % a.H, bb = bh / a.H;
  g2s<T, 256>(sH, H_LD, a.HT + (size_t)cid * D * D, D, D, D, tid);
  g2s<T, 256>(sV, V_LD, a.VnT + (size_t)cid * D * BT, BT, D, BT, tid);
  __syncthreads();

  const size_t HD = (size_t)a.H * D;
  float* obase = a.out + ((size_t)bb * a.T_len + (size_t)c * BT) * HD + (size_t)hh * D;
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int It = own_block<NB>(wv, i);
    const int t = It * 16 + li;
    Op qf[NKD], af[NKT];
    const T* qrow = a.Qg + (size_t)cid * BT * D + (size_t)t * D;
    const T* arow = a.Aqk + (size_t)cid * BT * BT + (size_t)t * BT;
#pragma unroll
    for (int kg = 0; kg < NKD; ++kg) qf[kg] = op_load<T>(qrow + kg * KS + lg * KC);
#pragma unroll
    for (int kg = 0; kg < NKT; ++kg) {
      const int s0 = kg * KS + lg * KC;
      af[kg] = (s0 <= It * 16 + 15) ? op_load<T>(arow + s0) : op_zero<T>();
    }
    const int kgmax = (It * 16 + 15) / KS;
#pragma unroll
    for (int vt = 0; vt < NDT; ++vt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kg = 0; kg < NKD; ++kg)
        mma(acc, op_load<T>(&sH[(vt * 16 + li) * H_LD + kg * KS + lg * KC]), qf[kg]);
      acc *= a.scale;
#pragma unroll
      for (int kg = 0; kg < NKT; ++kg)
        if (kg <= kgmax)
          mma(acc, op_load<T>(&sV[(vt * 16 + li) * V_LD + kg * KS + lg * KC]), af[kg]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = sanitize(acc[r]);
      store4(obase + (size_t)t * HD + vt * 16 + 4 * lg, acc);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers (called from gdn2_api.cpp).
template <typename T, typename TG, int BT, int D>
hipError_t launch_fwd(hipStream_t st, int B, int T_len, int H, const void* q, const void* k,
                      const void* v, const void* w, const void* b, const void* g,
                      const float* h0, float scale, float* out, float* h_final, char* ws,
                      float* a_dbg, int flags) {
  const int N = T_len / BT;
  const size_t NC = (size_t)B * H * N;
  const FwdLayout L = fwd_layout(NC, BT, D, sizeof(T));
  T* W = reinterpret_cast<T*>(ws + L.W);
  float* UT = reinterpret_cast<float*>(ws + L.UT);
  T* KgT = reinterpret_cast<T*>(ws + L.KgT);
  T* Qg = reinterpret_cast<T*>(ws + L.Qg);
  T* Aqk = reinterpret_cast<T*>(ws + L.Aqk);
  float* GL = reinterpret_cast<float*>(ws + L.GL);
  T* HT = reinterpret_cast<T*>(ws + L.HT);
  T* VnT = reinterpret_cast<T*>(ws + L.VnT);
  launch_mark(st);
  if (NC > 0) {
    PrepArgs<T, TG> pa{(const T*)q, (const T*)k, (const T*)v, (const T*)w, (const T*)b,
                       (const TG*)g, T_len, H, N, scale, W, UT, KgT, Qg, Aqk, GL,
                       a_dbg ? a_dbg : ((flags & 1) ? reinterpret_cast<float*>(ws + L.A)
                                                    : nullptr)};
    hipLaunchKernelGGL((fwd_prep<T, TG, BT, D>), dim3(NC), dim3(256), 0, st, pa);
  }
  launch_mark(st);
  StateArgs<T> sa{W, UT, KgT, GL, h0, N, HT, VnT, h_final};
  hipLaunchKernelGGL((fwd_state<T, BT, D>), dim3((size_t)B * H * (D / 64)), dim3(256), 0, st, sa);
  launch_mark(st);
  if (NC > 0) {
    OutArgs<T> oa{Qg, Aqk, HT, VnT, T_len, H, N, scale, out};
    hipLaunchKernelGGL((fwd_out<T, BT, D>), dim3(NC), dim3(256), 0, st, oa);
  }
  launch_mark(st);
  return hipGetLastError();
}

#define GDN2_INST_FWD(T, TG, BT, D)                                                          \
  template hipError_t launch_fwd<T, TG, BT, D>(hipStream_t, int, int, int, const void*,     \
                                               const void*, const void*, const void*,       \
                                               const void*, const void*, const float*,      \
                                               float, float*, float*, char*, float*, int);

GDN2_INST_FWD(float, float, 64, 64)
GDN2_INST_FWD(float, float, 64, 128)
GDN2_INST_FWD(bf16_t, float, 64, 64)
GDN2_INST_FWD(bf16_t, float, 64, 128)
GDN2_INST_FWD(bf16_t, float, 128, 64)
GDN2_INST_FWD(bf16_t, float, 128, 128)
GDN2_INST_FWD(bf16_t, bf16_t, 64, 64)
GDN2_INST_FWD(bf16_t, bf16_t, 64, 128)
GDN2_INST_FWD(bf16_t, bf16_t, 128, 64)
GDN2_INST_FWD(bf16_t, bf16_t, 128, 128)

}  // namespace gdn2
