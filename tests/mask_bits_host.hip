// Host driver for tests/test_mask_bits.py: evaluates the kernels' 64-element
// visibility words (row_valid_bits / col_valid_bits in gki_common.cuh, the
// same functions the attention kernels call) on the CPU.
//
// stdin, repeated per geometry:
//   G n_q n_kv causal sink window bm bn n_queries
//   <n_qb * n_kb block-mask ints>
//   n_queries lines "r q_row k0 partial" or "c kv q0 partial"
// stdout: one 16-digit hex word per query.
#include <cstdio>
#include <vector>

#include "gki_common.cuh"

int main() {
  char tag[4];
  while (std::scanf("%3s", tag) == 1) {
    gki::Geom g{};
    int n_queries = 0;
    if (std::scanf("%d %d %d %d %d %d %d %d", &g.n_q, &g.n_kv, &g.causal, &g.sink, &g.window, &g.bm,
                   &g.bn, &n_queries) != 8)
      return 2;
    g.q_off = g.n_kv - g.n_q;
    g.n_qb = (g.n_q + g.bm - 1) / g.bm;
    g.n_kb = (g.n_kv + g.bn - 1) / g.bn;
    std::vector<int32_t> mask((size_t)g.n_qb * g.n_kb);
    for (auto& m : mask)
      if (std::scanf("%d", &m) != 1) return 2;
    g.mask = mask.data();
    for (int i = 0; i < n_queries; ++i) {
      char kind[4];
      int a, b, partial;
      if (std::scanf("%3s %d %d %d", kind, &a, &b, &partial) != 4) return 2;
      const uint64_t w = kind[0] == 'r' ? gki::row_valid_bits(g, a, b, partial != 0)
                                        : gki::col_valid_bits(g, a, b, partial != 0);
      std::printf("%016llx\n", (unsigned long long)w);
    }
  }
  return 0;
}
