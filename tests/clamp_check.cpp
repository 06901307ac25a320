// Host check of the chunk-table clamps in gdn2_layout.h (chunk_rows,
// seq_chunks): the functions the kernels read their variable-length tables
// through; and of xcd_split, the kernels' workgroup-to-(chunk, part) map.  For random and adversarial tables, every token row a kernel can
// touch must lie inside the packed (B*T) rows and every chunk range inside
// [0, N).  Built with g++ by tests/test_clamps_cpu.py; prints "ok <cases>".
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "gdn2_layout.h"

using gdn2::chunk_rows;
using gdn2::seq_chunks;

static int fail(const char* what, long long a, long long b, long long c) {
  std::printf("FAIL %s %lld %lld %lld\n", what, a, b, c);
  return 1;
}

// rows the kernels touch for one chunk: row0 + min(t, max(valid - 1, 0)), t < BT
static bool rows_ok(const gdn2::ChunkRows& cr, int BT, long long rows) {
  if (cr.valid < 0 || cr.valid > BT) return false;
  const long long last = cr.valid > 0 ? cr.valid - 1 : 0;
  return (long long)cr.row0 >= 0 && (long long)cr.row0 + last < rows;
}

int main() {
  std::mt19937_64 rng(12345);
  const int specials[] = {INT_MIN, INT_MIN + 1, -7, -1, 0, 1, 63, 64, 65, 127, 128, 129,
                          1 << 29, INT_MAX - 1, INT_MAX};
  long long cases = 0;
  for (int iter = 0; iter < 20000; ++iter) {
    const int BT = (iter & 1) ? 64 : 128;
    const int total = 1 + (int)(rng() % 40);
    const int T = total + (int)(rng() % (total * BT));   // >= 1 token per chunk
    std::vector<int> cs(total + 1), cu(total + 2);
    for (int c = 0; c <= total; ++c) {
      const unsigned kind = rng() % 4;
      cs[c] = kind == 0 ? specials[rng() % 15]
            : kind == 1 ? (int)(rng() % (2 * T + 2)) - 1
                        : (int)std::min<long long>((long long)c * BT, T);
    }
    for (int c = 0; c < total; ++c) {
      const gdn2::ChunkRows cr = chunk_rows(cs.data(), c, 0, T, BT);
      if (!rows_ok(cr, BT, T)) return fail("varlen rows", c, (long long)cr.row0, cr.valid);
      ++cases;
    }
    const int nseq = 1 + (int)(rng() % (total + 1));
    for (int s = 0; s <= nseq; ++s)
      cu[s] = (rng() % 3 == 0) ? specials[rng() % 15] : (int)(rng() % (total + 3)) - 1;
    for (int s = 0; s < nseq; ++s) {
      const gdn2::SeqChunks sc = seq_chunks(cu.data(), s, total);
      if (sc.c0 < 0 || sc.n < 0 || (long long)sc.c0 + sc.n > total)
        return fail("seq chunks", s, sc.c0, sc.n);
      ++cases;
    }
    // equal-length sequences (no table): B batch elements of T tokens
    const int B = 1 + (int)(rng() % 4), N = (T + BT - 1) / BT;
    for (int bb = 0; bb < B; ++bb)
      for (int c = 0; c < N; ++c) {
        const gdn2::ChunkRows cr = chunk_rows(nullptr, c, bb, T, BT);
        if (cr.valid <= 0 || !rows_ok(cr, BT, (long long)B * T) ||
            (long long)cr.row0 + cr.valid > (long long)(bb + 1) * T)
          return fail("equal rows", bb, c, cr.valid);
        ++cases;
      }
  }
  // xcd_split: a bijection of workgroup ids onto (unit, part), and in whole
  // groups of 8 NS ids every part of a unit on the same XCD (id mod 8)
  for (int NS : {1, 2, 4, 8}) {
    for (int n = 1; n <= 300; ++n) {
      const int nwg = NS * n;
      const int full = nwg / (8 * NS) * (8 * NS);
      std::vector<int> seen((size_t)nwg, -1);
      for (int id = 0; id < nwg; ++id) {
        const gdn2::UnitPart up = gdn2::xcd_split(id, nwg, NS);
        if (up.unit < 0 || up.unit >= n || up.part < 0 || up.part >= NS)
          return fail("xcd_split range", NS, nwg, id);
        int& s = seen[(size_t)up.unit * NS + up.part];
        if (s >= 0) return fail("xcd_split twice", NS, nwg, id);
        s = id;
        ++cases;
      }
      for (int u = 0; u < n; ++u)
        for (int p = 1; p < NS; ++p) {
          const int a = seen[(size_t)u * NS], b = seen[(size_t)u * NS + p];
          if (a < full && b < full && a % 8 != b % 8) return fail("xcd_split xcd", NS, nwg, u);
        }
    }
  }
  std::printf("ok %lld\n", cases);
  return 0;
}
