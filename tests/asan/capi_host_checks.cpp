// Host-side checks of the C ABI, built with AddressSanitizer on the host code
// (see tests/test_host_asan.py). Calls only entry points and argument
// combinations that return before any kernel launch, so it needs no GPU:
//  * gki_dkdv_items on random column lists, with output arrays sized exactly
//    to the counts the first call reports (an out-of-bounds write trips ASan),
//    checked against the work-list invariants;
//  * gki_rolling_stream against a brute-force count of the positions the last
//    n_q queries of a StreamingLLM cache can see;
//  * gki_fwd_order on random row lists into an exactly sized table: a
//    permutation that keeps each XCD's contiguous share, heaviest first;
//  * every launching entry point rejecting bad arguments with an error code
//    and a message, before it touches the device.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "gki_bsa.h"

static int g_fail = 0;
#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      ++g_fail;                                            \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                   \
      std::fprintf(stderr, "\n");                          \
    }                                                      \
  } while (0)

static void check_work_lists(std::mt19937& rng) {
  for (int trial = 0; trial < 2000; ++trial) {
    const int n_kt = 1 + (int)(rng() % 300);
    const int group = 1 + (int)(rng() % 16);
    const int bh_kv = 1 + (int)(rng() % 8);
    const int max_chunk = (rng() % 3 == 0) ? 1 + (int)(rng() % 64) : 0;
    const int max_len = (rng() % 4 == 0) ? 400 : 40;
    std::vector<int32_t> col_ptr(n_kt + 1, 0);
    for (int kt = 0; kt < n_kt; ++kt) col_ptr[kt + 1] = col_ptr[kt] + (int32_t)(rng() % (max_len + 1));
    int32_t ni = -1, ns = -1, np = -1;
    int rc = gki_dkdv_items(col_ptr.data(), n_kt, group, bh_kv, max_chunk, nullptr, &ni, nullptr, &ns, &np);
    CHECK(rc == 0, "counting call rc %d (%s)", rc, gki_last_error());
    if (rc) continue;
    std::vector<int32_t> items(4 * (size_t)ni), split(3 * (size_t)ns);
    int32_t ni2 = -1, ns2 = -1, np2 = -1;
    rc = gki_dkdv_items(col_ptr.data(), n_kt, group, bh_kv, max_chunk, items.data(), &ni2,
                        ns ? split.data() : nullptr, &ns2, &np2);
    CHECK(rc == 0 && ni2 == ni && ns2 == ns && np2 == np, "filling call disagrees with the counts");
    // every column's walk of len * group iterations is covered once, in order,
    // by consecutive items; split columns own consecutive partial slots
    int item = 0, slot = 0, si = 0;
    for (int kt = 0; kt < n_kt; ++kt) {
      const int64_t n_it = (int64_t)(col_ptr[kt + 1] - col_ptr[kt]) * group;
      int64_t next = 0;
      const int first = item;
      while (item < ni && items[4 * item] == kt) {
        CHECK(items[4 * item + 1] == next, "item %d of column %d starts at %d, expected %lld", item, kt,
              items[4 * item + 1], (long long)next);
        CHECK(items[4 * item + 2] >= items[4 * item + 1], "item %d is reversed", item);
        if (max_chunk > 0)
          CHECK(items[4 * item + 2] - items[4 * item + 1] <= max_chunk || item == first,
                "item %d longer than the chunk", item);
        next = items[4 * item + 2];
        ++item;
      }
      const int parts = item - first;
      CHECK(parts >= 1 && next == n_it, "column %d: %d items end at %lld of %lld", kt, parts,
            (long long)next, (long long)n_it);
      if (parts == 1) {
        CHECK(items[4 * first + 3] == -1, "unsplit column %d has a partial slot", kt);
      } else {
        CHECK(si < ns && split[3 * si] == kt && split[3 * si + 1] == slot && split[3 * si + 2] == parts,
              "split entry of column %d", kt);
        for (int c = 0; c < parts; ++c)
          CHECK(items[4 * (first + c) + 3] == slot + c, "slot of item %d of column %d", c, kt);
        slot += parts;
        ++si;
      }
    }
    CHECK(item == ni && si == ns && slot == np, "work list has extra entries");
  }
}

static void check_rolling_stream(std::mt19937& rng) {
  for (int trial = 0; trial < 3000; ++trial) {
    const int n_q = 1 + (int)(rng() % 4);
    const int sink = (int)(rng() % 8);
    const int window = (int)(rng() % 40);
    const int ring = window + n_q - 1 + (int)(rng() % 5) + (window + n_q - 1 == 0 ? 1 : 0);
    const int64_t length = n_q + (int64_t)(rng() % 120);
    int32_t ns = -1, lo = -1, nt = -1;
    const int rc = gki_rolling_stream(length, n_q, sink, window, ring, &ns, &lo, &nt);
    CHECK(rc == 0, "rolling stream rc %d (%s)", rc, gki_last_error());
    if (rc) continue;
    // brute force: positions any of the last n_q queries sees under the
    // causal StreamingLLM rule (k <= q and (k < S or k >= q - W + 1))
    std::set<int64_t> seen;
    for (int64_t q = length - n_q; q < length; ++q)
      for (int64_t k = 0; k <= q; ++k)
        if (k < sink || k >= q - window + 1) seen.insert(k);
    // the stream: the sinks, then the hull max(S, L - n_q - W + 1) .. L - 1
    // of the rows' windows (each row applies the token rule inside it); for
    // W >= 1 the hull is exactly the union, for W = 0 it adds n_q - 1
    // positions that no row sees
    std::set<int64_t> stream;
    for (int64_t k = 0; k < sink && k < length; ++k) stream.insert(k);
    for (int64_t k = std::max<int64_t>(sink, length - n_q - window + 1); k < length; ++k) stream.insert(k);
    CHECK(nt == (int64_t)stream.size(), "length %lld n_q %d S %d W %d: %d tokens, stream %zu",
          (long long)length, n_q, sink, window, nt, stream.size());
    bool covers = true;
    for (int64_t k : seen) covers &= stream.count(k) > 0;
    CHECK(covers, "stream misses a visible position (length %lld n_q %d S %d W %d)", (long long)length,
          n_q, sink, window);
    if (window >= 1) CHECK(stream == seen, "stream is not exactly the visible set for W >= 1");
    int64_t n_sink_bf = 0;
    for (int64_t k : stream) n_sink_bf += k < sink;
    CHECK(ns == n_sink_bf, "sink count %d, expected %lld", ns, (long long)n_sink_bf);
  }
  // rejected: ring shorter than the window the queries need, bad n_q, length < n_q
  int32_t a, b, c;
  CHECK(gki_rolling_stream(100, 2, 4, 16, 16, &a, &b, &c) != 0, "short ring accepted");
  CHECK(gki_rolling_stream(100, 5, 4, 16, 32, &a, &b, &c) != 0, "n_q 5 accepted");
  CHECK(gki_rolling_stream(1, 2, 4, 16, 32, &a, &b, &c) != 0, "length < n_q accepted");
}

static void check_rejections() {
  alignas(16) static char buf[1024];
  void* p = buf;
  float* f = (float*)buf;
  const int32_t* ip = (const int32_t*)buf;
  auto rejected = [](int rc, const char* what) {
    const std::string msg = gki_last_error();
    CHECK(rc != 0 && !msg.empty(), "%s: rc %d, message '%s'", what, rc, msg.c_str());
  };
  // forward: bad dtype, bad head_dim, null tensors, misaligned pointers, wrong list size
  // (arguments: q, dtype, H, H_kv, head_dim, n_qt, n_qb, scale, sink; the rest fixed)
  auto fwd = [&](void* q, int dtype, int H, int H_kv, int head_dim, int n_qt, int n_qb, float scale,
                 int sink) {
    return gki_bsa_fwd(q, p, p, p, f, dtype, 1, H, H_kv, 64, 64, head_dim, ip, ip, n_qt, nullptr, ip, n_qb,
                       1, 64, 64, scale, 1, sink, 16, nullptr);
  };
  rejected(fwd(p, 7, 1, 1, 64, 1, 1, 0.125f, 4), "fwd dtype 7");
  rejected(fwd(p, 2, 1, 1, 48, 1, 1, 0.125f, 4), "fwd head_dim 48");
  rejected(fwd(nullptr, 2, 1, 1, 64, 1, 1, 0.125f, 4), "fwd null q");
  rejected(fwd(buf + 2, 2, 1, 1, 64, 1, 1, 0.125f, 4), "fwd misaligned q");
  rejected(fwd(p, 2, 1, 1, 64, 3, 1, 0.125f, 4), "fwd schedule rows");
  rejected(fwd(p, 2, 4, 3, 64, 1, 1, 0.125f, 4), "fwd H_kv not dividing H");
  rejected(fwd(p, 2, 1, 1, 64, 1, 2, 0.125f, 4), "fwd mask shape");
  rejected(fwd(p, 2, 1, 1, 64, 1, 1, __builtin_inff(), 4), "fwd infinite scale");
  rejected(fwd(p, 2, 1, 1, 64, 1, 1, 0.125f, -1), "fwd negative sink");
  // backward: inconsistent work list, missing partials, schedule shape
  rejected(gki_bsa_bwd(p, p, p, p, p, f, p, p, p, f, 2, 1, 1, 1, 64, 64, 64, ip, ip, 1, ip, ip, 1, ip, 0,
                       ip, 0, 0, f, nullptr, ip, 1, 1, 64, 64, 0.125f, 1, 4, 16, nullptr), "bwd no items");
  rejected(gki_bsa_bwd(p, p, p, p, p, f, p, p, p, f, 2, 1, 1, 1, 64, 64, 64, ip, ip, 1, ip, ip, 1, ip, 2,
                       nullptr, 1, 1, nullptr, nullptr, ip, 1, 1, 64, 64, 0.125f, 1, 4, 16, nullptr),
           "bwd split without partials");
  rejected(gki_bsa_bwd(p, p, p, p, p, f, p, p, p, f, 2, 1, 1, 1, 64, 64, 64, ip, ip, 2, ip, ip, 1, ip, 1,
                       ip, 0, 0, f, nullptr, ip, 1, 1, 64, 64, 0.125f, 1, 4, 16, nullptr), "bwd schedule rows");
  // decode: too many query rows, bad splits, missing workspace
  rejected(gki_bsa_decode(p, p, p, p, f, 2, 1, 1, 1, 5, 64, 64, ip, 1, ip, 1, 1, 64, 64, 0.125f, 1, 4,
                          16, f, 1, nullptr), "decode n_q 5");
  rejected(gki_bsa_decode(p, p, p, p, f, 2, 1, 1, 1, 1, 64, 64, ip, 1, ip, 1, 1, 1, 64, 0.125f, 1, 4, 16,
                          nullptr, 2, nullptr), "decode without workspace");
  rejected(gki_bsa_decode(p, p, p, p, f, 2, 1, 1, 1, 1, 64, 64, ip, 1, ip, 1, 1, 1, 64, 0.125f, 1, 4, 16,
                          f, 0, nullptr), "decode zero splits");
  rejected(gki_rolling_decode(p, p, p, p, f, 2, 1, 1, 1, 1, 64, 4, 16, 8, 64, 0.125f, f, 1, nullptr),
           "rolling decode short ring");
  rejected(gki_rolling_decode_noalloc(p, p, p, p, f, 2, 64, 64, 64, 4, 128, 4, 2048, 2051, 100000,
                                      0.125f, 64, nullptr),
           "noalloc decode beyond the scratch");
  rejected(gki_rolling_append(p, p, p, p, 2, 1, 1, 64, 4, 0, 0, 1, nullptr), "append zero ring");
  rejected(gki_rolling_append(p, p, p, p, 2, 1, 1, 64, 4, 8, -1, 1, nullptr), "append negative start");
  rejected(gki_decode_tokens(ip, -1, 1, 64, ip, 1, 1, 1, 64, 1, 4, 16, nullptr, nullptr, nullptr),
           "decode tokens null count");
  // accepted without a launch: an empty append
  CHECK(gki_rolling_append(nullptr, nullptr, nullptr, nullptr, 2, 1, 1, 64, 4, 8, 0, 0, nullptr) == 0,
        "empty append rejected: %s", gki_last_error());
  int32_t t[6];
  CHECK(gki_tile_sizes(t, t + 1, t + 2, t + 3, t + 4, t + 5) == 0 && t[3] == 64, "tile sizes");
  CHECK(gki_tile_sizes(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) == 0, "tile sizes, nulls");
  CHECK(gki_bsa_decode_workspace_floats(8, 32, 1, 128, 4) == 8ll * 32 * 4 * 130, "workspace floats");
  const int32_t down[3] = {0, 4, 2};
  int32_t ord[4];
  rejected(gki_fwd_order(down, 2, 2, ord), "order of a decreasing row_ptr");
  rejected(gki_fwd_order(nullptr, 2, 2, ord), "order, null row_ptr");
  rejected(gki_fwd_order(down, 0, 2, ord), "order, no q tiles");
  rejected(gki_fwd_order(down, 1 << 20, 1 << 12, ord), "order, table too large");
  // read probe: null, misaligned, row size, output too small
  uint32_t* up = (uint32_t*)buf;
  const int64_t need = gki_read_probe_words(1);
  CHECK(need > 0 && gki_read_probe_words(0) == 0, "read probe words %lld", (long long)need);
  rejected(gki_read_probe(nullptr, p, 1, 100, 256, 4, 16, up, need, nullptr), "read probe null k");
  rejected(gki_read_probe(buf + 4, p, 1, 100, 256, 4, 16, up, need, nullptr), "read probe misaligned k");
  rejected(gki_read_probe(p, p, 1, 100, 24, 4, 16, up, need, nullptr), "read probe row bytes 24");
  rejected(gki_read_probe(p, p, 1, 100, 256, -1, 16, up, need, nullptr), "read probe negative sink");
  rejected(gki_read_probe(p, p, 1, 100, 256, 4, 16, up, need - 1, nullptr), "read probe output too small");
  rejected(gki_read_probe(p, p, 0, 100, 256, 4, 16, up, need, nullptr), "read probe no slices");
}

static void check_fwd_order(std::mt19937& rng) {
  for (int trial = 0; trial < 500; ++trial) {
    const int n_qt = 1 + (int)(rng() % 200);
    const int bh = 1 + (int)(rng() % 40);
    std::vector<int32_t> row_ptr(n_qt + 1, 0);
    for (int qt = 0; qt < n_qt; ++qt) row_ptr[qt + 1] = row_ptr[qt] + (int32_t)(rng() % 6);
    const int n = n_qt * bh;
    std::vector<int32_t> order(n, -1);
    const int rc = gki_fwd_order(row_ptr.data(), n_qt, bh, order.data());
    CHECK(rc == 0, "gki_fwd_order rc %d (%s)", rc, gki_last_error());
    if (rc) continue;
    // XCD x's share: the n / 8 (+1 for x < n % 8) logical ids after XCD x-1's
    int lo = 0;
    for (int x = 0; x < 8; ++x) {
      const int hi = lo + n / 8 + (x < n % 8 ? 1 : 0);
      std::vector<int32_t> share(order.begin() + lo, order.begin() + hi);
      for (int i = lo; i < hi; ++i) {
        CHECK(order[i] >= lo && order[i] < hi, "unit %d left XCD %d's share", order[i], x);
        if (i > lo) {
          const int la = row_ptr[order[i - 1] % n_qt + 1] - row_ptr[order[i - 1] % n_qt];
          const int lb = row_ptr[order[i] % n_qt + 1] - row_ptr[order[i] % n_qt];
          CHECK(la > lb || (la == lb && order[i - 1] < order[i]), "share of XCD %d out of order", x);
        }
      }
      std::sort(share.begin(), share.end());
      CHECK(std::unique(share.begin(), share.end()) == share.end(), "repeated unit in XCD %d", x);
      lo = hi;
    }
  }
}

int main() {
  std::mt19937 rng(1234);
  check_work_lists(rng);
  check_fwd_order(rng);
  check_rolling_stream(rng);
  check_rejections();
  if (g_fail) {
    std::fprintf(stderr, "%d host check(s) failed\n", g_fail);
    return 1;
  }
  std::printf("host checks passed (abi %d)\n", gki_abi_version());
  return 0;
}
