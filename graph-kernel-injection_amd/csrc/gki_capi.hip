// C ABI of the block-sparse attention library (declared in include/gki_bsa.h).
//
// Every entry point is stateless and asynchronous on the caller's stream: it
// validates its arguments, launches, and returns 0 or a non-zero code whose
// message is available from gki_last_error() (thread-local). The library never
// allocates or frees device memory and keeps no pointer after returning.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "gki_bsa.h"
#include "gki_common.cuh"

namespace gki {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(3, std::string(what) + ": " + hipGetErrorString(err));
  return 0;
}

int fwd_tile_m(int dtype);
int fwd_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                 void* o, float* lse, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
                 const int32_t* wg_order, hipStream_t stream);
int bwd_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                 const void* o, const void* dout, const float* lse, void* dq, void* dk, void* dv,
                 float* delta, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
                 const int32_t* dq_order, const int32_t* col_ptr, const int32_t* col_idx, const KvWork& w,
                 hipStream_t stream);
int decode_tokens_dispatch(const Geom& g, const int32_t* list, int n_ent, int32_t* tok, int32_t* count,
                           hipStream_t stream);
int decode_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                    void* o, float* lse, const int32_t* tok, int n_tokens, float* ws, int n_splits,
                    hipStream_t stream);
void ring_stream(int length, int n_q, int sink, int window, int ring, int* n_sink, int* w_lo, int* base,
                 int* n_tokens);
int decode_ring_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k,
                         const void* v, void* o, float* lse, int ring, float* ws, int n_splits,
                         hipStream_t stream);
int append_dispatch(int dtype, int head_dim, void* kc, void* vc, const void* kn, const void* vn, int BH,
                    int n_new, int start, int sink, int ring, hipStream_t stream);
int64_t read_probe_words(int BH);
int read_probe_dispatch(const void* k, const void* v, int BH, int64_t n_kv, int row_bytes, int n_sink,
                        int64_t w_lo, uint32_t* out, hipStream_t stream);

namespace {

// The kernels move Q / K / V / O (and gradients, K/V caches) in 16-byte chunks
// (vector loads and LDS-DMA); every such tensor must start 16-byte aligned.
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
template <typename... P> inline bool all_aligned16(P... p) { return (aligned16(p) && ...); }

// Softmax scale of any finite sign: the signed scale for the kernels that
// scale each score before the max, and the Q transform plus positive scale
// for the kernels that take the max on unscaled scores (Geom::q_and). The
// words are 32-bit: two 16-bit Q elements or one fp32 element (the fp32
// kernels scale before the max and ignore them).
void set_scale(Geom& g, float scale) {
  g.scale = scale;
  g.scale_log2 = scale * kLog2e;
  g.q_and = scale == 0.f ? 0u : 0xFFFFFFFFu;
  g.q_xor = scale < 0.f ? 0x80008000u : 0u;
  g.qk_scale_log2 = scale == 0.f ? kLog2e : (scale < 0.f ? -scale : scale) * kLog2e;
  g.prescale = 0;   // reference order; make_geom sets it where exact
}

int make_geom(Geom& g, int dtype, int B, int H, int H_kv, int n_q, int n_kv, int head_dim,
              const int32_t* mask, int n_qb, int n_kb, int block_m, int block_n, float scale, int causal,
              int sink, int window) {
  GKI_REQUIRE(dtype == kF32 || dtype == kF16 || dtype == kBF16, 2,
              "unsupported dtype code " + std::to_string(dtype) + " (0=fp32, 1=fp16, 2=bf16)");
  GKI_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128, 2,
              "unsupported head_dim " + std::to_string(head_dim) + " (supported: 16, 32, 64, 128)");
  GKI_REQUIRE(B > 0 && H > 0 && n_q > 0 && n_kv > 0, 1, "B, H, n_q and n_kv must be positive");
  GKI_REQUIRE(H_kv > 0 && H % H_kv == 0, 1,
              "H_kv must be positive and divide H (grouped-query attention)");
  GKI_REQUIRE((int64_t)B * H < (1ll << 31) / 4096, 1, "B * H too large");
  GKI_REQUIRE(block_m > 0 && block_n > 0, 1, "block_m and block_n must be positive");
  GKI_REQUIRE(n_qb == (n_q + block_m - 1) / block_m && n_kb == (n_kv + block_n - 1) / block_n, 1,
              "block mask shape does not match ceil(n_q/block_m) x ceil(n_kv/block_n)");
  GKI_REQUIRE((int64_t)n_qb * n_kb < (1ll << 31), 1,
              "block mask too large (the kernels index it with 32-bit offsets)");
  GKI_REQUIRE(sink >= 0 && window >= 0, 1, "sink_size and window_size must be non-negative");
  GKI_REQUIRE(std::isfinite(scale), 1, "softmax_scale must be finite");
  GKI_REQUIRE((int64_t)n_kv < (1ll << kPartialBit), 1, "n_kv too large");
  GKI_REQUIRE(mask != nullptr, 1, "null block mask");
  g.B = B;
  g.H = H;
  g.H_kv = H_kv;
  g.group = H / H_kv;
  g.n_q = n_q;
  g.n_kv = n_kv;
  g.q_off = n_kv - n_q;
  set_scale(g, scale);
  // 16-bit backward: the power-of-two scale moves into the dP operand (exact
  // products; see Geom::prescale) for |scale| in [2^-4, 1]; the dS cast keeps
  // the reference's place (after the scale) either way.
  int e2 = 0;
  const float mant = std::frexp(scale, &e2);
  g.prescale = dtype != kF32 && std::fabs(mant) == 0.5f && e2 >= -3 && e2 <= 1;
  g.causal = causal ? 1 : 0;
  g.sink = sink;
  g.window = window;
  g.mask = mask;
  g.n_qb = n_qb;
  g.n_kb = n_kb;
  g.bm = block_m;
  g.bn = block_n;
  return 0;
}

// Device-resident scratch of gki_rolling_decode_noalloc (the split partials
// of a decode step), for callers that cannot allocate: code under HIP graph
// capture, tight serving loops. Every GPU the library runs on holds its own
// copy until the process ends. In host code `scratch` names a host-side
// stand-in, never the device array: the device address comes from
// hipGetSymbolAddress, once per device (scratch_on_device).
constexpr int64_t kScratchFloats = int64_t(4) << 20;   // 16 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The scratch address on the device that `stream` launches on (the current
// device for the null stream): looked up on first use per device, with that
// device made current for the lookup and the caller's device restored.
int scratch_on_device(hipStream_t stream, float** out) {
  int cur = -1;
  const hipError_t e0 = hipGetDevice(&cur);
  GKI_REQUIRE(e0 == hipSuccess && cur >= 0, 3,
              std::string("scratch: no current HIP device (") + hipGetErrorString(e0) + ")");
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = -1;
    const hipError_t es = hipStreamGetDevice(stream, &sd);
    GKI_REQUIRE(es == hipSuccess && sd >= 0, 3,
                std::string("scratch: hipStreamGetDevice failed: ") + hipGetErrorString(es));
    dev = (int)sd;
  }
  GKI_REQUIRE(dev < kMaxDevices, 3, "scratch: device index " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) {
      const hipError_t es = hipSetDevice(dev);
      GKI_REQUIRE(es == hipSuccess, 3, std::string("scratch: hipSetDevice failed: ") + hipGetErrorString(es));
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t er = hipSetDevice(cur);
      GKI_REQUIRE(er == hipSuccess, 3,
                  std::string("scratch: restoring the current device failed: ") + hipGetErrorString(er));
    }
    GKI_REQUIRE(e == hipSuccess && p != nullptr, 3,
                std::string("scratch: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = (float*)p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Argument checks of the rolling-cache decode entry points.
int rolling_decode_args(int dtype, int B, int H, int H_kv, int n_q, int head_dim, int sink_size,
                        int window_size, int ring_size, int64_t length, float softmax_scale,
                        const void* q, const void* k_cache, const void* v_cache, void* o, float* lse,
                        int n_splits) {
  GKI_REQUIRE(dtype == kF32 || dtype == kF16 || dtype == kBF16, 2,
              "unsupported dtype code " + std::to_string(dtype) + " (0=fp32, 1=fp16, 2=bf16)");
  GKI_REQUIRE(head_dim == 64 || head_dim == 128, 2,
              "gki_rolling_decode: head_dim must be 64 or 128, got " + std::to_string(head_dim));
  GKI_REQUIRE(B > 0 && H > 0 && (int64_t)B * H < (1ll << 31) / 4096, 1,
              "gki_rolling_decode: B and H must be positive and B * H not too large");
  GKI_REQUIRE(H_kv > 0 && H % H_kv == 0, 1,
              "H_kv must be positive and divide H (grouped-query attention)");
  if (int rc = gki_rolling_stream(length, n_q, sink_size, window_size, ring_size, nullptr, nullptr,
                                  nullptr))
    return rc;
  GKI_REQUIRE(std::isfinite(softmax_scale), 1, "softmax_scale must be finite");
  GKI_REQUIRE(q && k_cache && v_cache && o && lse, 1, "gki_rolling_decode: null pointer");
  GKI_REQUIRE(all_aligned16(q, k_cache, v_cache), 1, "gki_rolling_decode: q and caches must be 16-byte aligned");
  GKI_REQUIRE(n_splits >= 1 && (int64_t)n_splits * B * H < (1ll << 31), 1,
              "gki_rolling_decode: n_splits must be >= 1 and the grid must fit");
  return 0;
}

int rolling_decode_checked(const void* q, const void* k_cache, const void* v_cache, void* o, float* lse,
                           int dtype, int B, int H, int H_kv, int n_q, int head_dim, int sink_size,
                           int window_size, int ring_size, int64_t length, float softmax_scale,
                           float* workspace, int n_splits, void* stream) {
  GKI_REQUIRE(n_splits == 1 || workspace, 1, "gki_rolling_decode: null workspace");
  Geom g{};
  g.B = B;
  g.H = H;
  g.H_kv = H_kv;
  g.group = H / H_kv;
  g.n_q = n_q;
  g.n_kv = (int)length;                 // positions 0 .. length-1; queries are the last n_q
  g.q_off = (int)length - n_q;
  set_scale(g, softmax_scale);
  g.causal = 1;
  g.sink = sink_size;
  g.window = window_size;
  g.mask = nullptr;                     // no stream entry carries the partial flag
  g.n_qb = g.n_kb = g.bm = g.bn = 1;
  return decode_ring_dispatch(dtype, head_dim, g, q, k_cache, v_cache, o, lse, ring_size, workspace,
                              n_splits, (hipStream_t)stream);
}

}  // namespace
}  // namespace gki

using namespace gki;

extern "C" {

int gki_abi_version(void) { return 8; }

const char* gki_last_error(void) { return g_last_error.c_str(); }

int gki_tile_sizes(int32_t* fwd_tile_m_16, int32_t* fwd_tile_m_32, int32_t* bwd_tile_m,
                   int32_t* tile_n, int32_t* decode_tile_m, int32_t* decode_max_q) {
  if (fwd_tile_m_16) *fwd_tile_m_16 = fwd_tile_m(kBF16);
  if (fwd_tile_m_32) *fwd_tile_m_32 = fwd_tile_m(kF32);
  if (bwd_tile_m) *bwd_tile_m = kTileM;
  if (tile_n) *tile_n = kTileN;
  if (decode_tile_m) *decode_tile_m = kDecodeTileM;
  if (decode_max_q) *decode_max_q = kDecodeMaxQ;
  return 0;
}

int gki_bsa_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int32_t dtype,
                int32_t B, int32_t H, int32_t H_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                const int32_t* row_ptr, const int32_t* row_idx, int32_t n_qt, const int32_t* wg_order,
                const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m, int32_t block_n,
                float softmax_scale, int32_t is_causal, int32_t sink_size, int32_t window_size,
                void* stream) {
  Geom g;
  if (int rc = make_geom(g, dtype, B, H, H_kv, n_q, n_kv, head_dim, mask, n_qb, n_kb, block_m, block_n,
                         softmax_scale, is_causal, sink_size, window_size))
    return rc;
  GKI_REQUIRE(q && k && v && o && lse && row_ptr && row_idx, 1, "gki_bsa_fwd: null pointer");
  GKI_REQUIRE(all_aligned16(q, k, v, o), 1, "gki_bsa_fwd: q, k, v, o must be 16-byte aligned");
  const int tm = fwd_tile_m(dtype);
  GKI_REQUIRE(n_qt == (n_q + tm - 1) / tm, 1, "gki_bsa_fwd: schedule row count mismatch");
  GKI_REQUIRE((int64_t)n_qt * B * H < (1ll << 31), 1, "gki_bsa_fwd: grid too large");
  return fwd_dispatch(dtype, head_dim, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, wg_order,
                      (hipStream_t)stream);
}

int gki_fwd_order(const int32_t* row_ptr, int32_t n_qt, int32_t bh, int32_t* order) {
  GKI_REQUIRE(row_ptr && order, 1, "gki_fwd_order: null pointer");
  GKI_REQUIRE(n_qt >= 1 && bh >= 1 && (int64_t)n_qt * bh < (1ll << 31), 1,
              "gki_fwd_order: n_qt and bh must be positive, n_qt * bh < 2^31");
  std::vector<int32_t> len(n_qt);
  for (int qt = 0; qt < n_qt; ++qt) {
    len[qt] = row_ptr[qt + 1] - row_ptr[qt];
    GKI_REQUIRE(len[qt] >= 0, 1, "gki_fwd_order: row_ptr must be non-decreasing");
  }
  // the launch's logical ids are (b * H + h) * n_qt + qt, split into one
  // contiguous range per XCD; each range is reordered on its own (its q tiles
  // stay on that XCD, so neighbouring tiles of a head still share its L2),
  // longest kept-tile list first, ties in logical order
  const int n = n_qt * bh;
  for (int x = 0; x < kXcd; ++x) {
    const int lo = xcd_start(x, n), hi = x + 1 < kXcd ? xcd_start(x + 1, n) : n;
    for (int l = lo; l < hi; ++l) order[l] = l;
    std::stable_sort(order + lo, order + hi,
                     [&](int32_t a, int32_t b) { return len[a % n_qt] > len[b % n_qt]; });
  }
  return 0;
}

int gki_bsa_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                const float* lse, void* dq, void* dk, void* dv, float* delta, int32_t dtype, int32_t B,
                int32_t H, int32_t H_kv, int32_t n_q, int32_t n_kv, int32_t head_dim, const int32_t* row_ptr,
                const int32_t* row_idx, int32_t n_qt, const int32_t* col_ptr, const int32_t* col_idx,
                int32_t n_kt, const int32_t* kv_items, int32_t n_items, const int32_t* kv_split,
                int32_t n_split, int32_t n_pslots, float* kv_partials, const int32_t* dq_order,
                const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m, int32_t block_n,
                float softmax_scale, int32_t is_causal, int32_t sink_size, int32_t window_size,
                void* stream) {
  Geom g;
  if (int rc = make_geom(g, dtype, B, H, H_kv, n_q, n_kv, head_dim, mask, n_qb, n_kb, block_m, block_n,
                         softmax_scale, is_causal, sink_size, window_size))
    return rc;
  GKI_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv && delta, 1, "gki_bsa_bwd: null tensor");
  GKI_REQUIRE(all_aligned16(q, k, v, o, dout, dq, dk, dv), 1,
              "gki_bsa_bwd: q, k, v, o, dout, dq, dk, dv must be 16-byte aligned");
  GKI_REQUIRE(row_ptr && row_idx && col_ptr && col_idx && kv_items, 1, "gki_bsa_bwd: null schedule");
  GKI_REQUIRE(n_qt == (n_q + kTileM - 1) / kTileM && n_kt == (n_kv + kTileN - 1) / kTileN, 1,
              "gki_bsa_bwd: schedule shape mismatch");
  GKI_REQUIRE(((uintptr_t)kv_items & 15) == 0, 1, "gki_bsa_bwd: kv_items must be 16-byte aligned");
  GKI_REQUIRE(n_items >= n_kt && n_split >= 0 && n_pslots >= n_split && n_split <= n_kt, 1,
              "gki_bsa_bwd: work list inconsistent with the tile count (see gki_dkdv_items)");
  GKI_REQUIRE(n_split == 0 || (kv_split && kv_partials), 1,
              "gki_bsa_bwd: split columns need kv_split and kv_partials");
  GKI_REQUIRE((int64_t)n_qt * B * H < (1ll << 31), 1, "gki_bsa_bwd: dQ grid too large");
  GKI_REQUIRE((int64_t)n_items * B * H_kv < (1ll << 31) &&
                  (int64_t)n_split * B * H_kv * (head_dim / 8) < (1ll << 31), 1,
              "gki_bsa_bwd: dK/dV grid too large");
  GKI_REQUIRE(((uintptr_t)kv_partials & 15) == 0, 1, "gki_bsa_bwd: kv_partials must be 16-byte aligned");
  KvWork w{kv_items, n_items, kv_split, n_split, n_pslots, kv_partials};
  return bwd_dispatch(dtype, head_dim, g, q, k, v, o, dout, lse, dq, dk, dv, delta, row_ptr, row_idx,
                      n_qt, dq_order, col_ptr, col_idx, w, (hipStream_t)stream);
}

int gki_dkdv_items(const int32_t* col_ptr, int32_t n_kt, int32_t group, int32_t bh_kv,
                   int32_t max_chunk, int32_t* items, int32_t* n_items, int32_t* split,
                   int32_t* n_split, int32_t* n_pslots) {
  GKI_REQUIRE(col_ptr && n_items && n_split && n_pslots, 1, "gki_dkdv_items: null pointer");
  GKI_REQUIRE(n_kt >= 1 && group >= 1 && bh_kv >= 1, 1,
              "gki_dkdv_items: n_kt, group and bh_kv must be positive");
  int64_t total = 0;
  for (int kt = 0; kt < n_kt; ++kt) {
    const int64_t len = (int64_t)col_ptr[kt + 1] - col_ptr[kt];
    GKI_REQUIRE(len >= 0 && len * group < (1ll << 30), 1, "gki_dkdv_items: bad column list");
    total += len;
  }
  total *= (int64_t)group * bh_kv;
  // iterations per item: at least kDkdvMinChunk, and few enough that the whole
  // grid has about kDkdvTargetItems items of work when columns are long; at
  // most max_chunk when positive (more, shorter items: cuts columns at any
  // length, e.g. to test the split path on short sequences)
  int64_t chunk = std::max<int64_t>(kDkdvMinChunk, (total + kDkdvTargetItems - 1) / kDkdvTargetItems);
  if (max_chunk > 0) chunk = std::min<int64_t>(chunk, max_chunk);
  int32_t ni = 0, ns = 0, np = 0;
  for (int kt = 0; kt < n_kt; ++kt) {
    const int64_t n_it = ((int64_t)col_ptr[kt + 1] - col_ptr[kt]) * group;
    const int64_t parts = std::max<int64_t>(1, (n_it + chunk - 1) / chunk);
    if (parts == 1) {
      if (items) {
        int32_t* it = items + 4 * ni;
        it[0] = kt, it[1] = 0, it[2] = (int32_t)n_it, it[3] = -1;
      }
      ++ni;
      continue;
    }
    if (split) {
      int32_t* sp = split + 3 * ns;
      sp[0] = kt, sp[1] = np, sp[2] = (int32_t)parts;
    }
    ++ns;
    for (int64_t c = 0; c < parts; ++c) {
      if (items) {
        int32_t* it = items + 4 * ni;
        it[0] = kt, it[1] = (int32_t)(n_it * c / parts), it[2] = (int32_t)(n_it * (c + 1) / parts);
        it[3] = np + (int32_t)c;
      }
      ++ni;
    }
    np += (int32_t)parts;
  }
  *n_items = ni;
  *n_split = ns;
  *n_pslots = np;
  return 0;
}

int64_t gki_bsa_decode_workspace_floats(int32_t B, int32_t H, int32_t n_q, int32_t head_dim,
                                        int32_t n_splits) {
  return (int64_t)B * H * n_splits * n_q * (head_dim + 2);
}

int gki_decode_tokens(const int32_t* tile_list, int32_t n_tiles, int32_t n_q, int32_t n_kv,
                      const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m, int32_t block_n,
                      int32_t is_causal, int32_t sink_size, int32_t window_size, int32_t* tokens,
                      int32_t* n_tokens, void* stream) {
  Geom g;
  if (int rc = make_geom(g, kBF16, 1, 1, 1, n_q, n_kv, 64, mask, n_qb, n_kb, block_m, block_n, 1.f,
                         is_causal, sink_size, window_size))
    return rc;
  GKI_REQUIRE(n_tokens && (n_tiles == 0 || (tile_list && tokens)), 1, "gki_decode_tokens: null pointer");
  GKI_REQUIRE(n_tiles >= 0, 1, "gki_decode_tokens: negative tile count");
  return decode_tokens_dispatch(g, tile_list, n_tiles, tokens, n_tokens, (hipStream_t)stream);
}

int gki_bsa_decode(const void* q, const void* k, const void* v, void* o, float* lse, int32_t dtype,
                   int32_t B, int32_t H, int32_t H_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                   const int32_t* tokens, int32_t n_tokens, const int32_t* mask, int32_t n_qb,
                   int32_t n_kb, int32_t block_m, int32_t block_n, float softmax_scale,
                   int32_t is_causal, int32_t sink_size, int32_t window_size, float* workspace,
                   int32_t n_splits, void* stream) {
  Geom g;
  if (int rc = make_geom(g, dtype, B, H, H_kv, n_q, n_kv, head_dim, mask, n_qb, n_kb, block_m, block_n,
                         softmax_scale, is_causal, sink_size, window_size))
    return rc;
  GKI_REQUIRE(q && k && v && o && lse, 1, "gki_bsa_decode: null pointer");
  GKI_REQUIRE(all_aligned16(q, k, v), 1, "gki_bsa_decode: q, k, v must be 16-byte aligned");
  GKI_REQUIRE(n_splits == 1 || workspace, 1, "gki_bsa_decode: null workspace");
  GKI_REQUIRE(n_q <= kDecodeMaxQ, 2, "gki_bsa_decode: n_q exceeds the decode kernel's row limit");
  GKI_REQUIRE(n_tokens >= 0 && (n_tokens == 0 || tokens), 1, "gki_bsa_decode: bad token list");
  GKI_REQUIRE(n_splits >= 1 && (int64_t)n_splits * B * H < (1ll << 31), 1,
              "gki_bsa_decode: n_splits must be >= 1 and the grid must fit");
  return decode_dispatch(dtype, head_dim, g, q, k, v, o, lse, tokens, n_tokens, workspace, n_splits,
                         (hipStream_t)stream);
}

int gki_rolling_stream(int64_t length, int32_t n_q, int32_t sink_size, int32_t window_size,
                       int32_t ring_size, int32_t* n_sink, int32_t* window_lo, int32_t* n_tokens) {
  GKI_REQUIRE(n_q >= 1 && n_q <= kDecodeMaxQ, 2, "gki_rolling_stream: n_q must be in [1, 4]");
  GKI_REQUIRE(length >= n_q && length < (1ll << kPartialBit), 1,
              "gki_rolling_stream: length must be in [n_q, 2^30)");
  GKI_REQUIRE(sink_size >= 0 && window_size >= 0, 1,
              "gki_rolling_stream: sink_size and window_size must be non-negative");
  GKI_REQUIRE(ring_size >= 1 && (int64_t)ring_size >= (int64_t)window_size + n_q - 1, 1,
              "gki_rolling_stream: ring_size must be >= window_size + n_q - 1 (and >= 1)");
  int ns, lo, base, nt;
  ring_stream((int)length, n_q, sink_size, window_size, ring_size, &ns, &lo, &base, &nt);
  if (n_sink) *n_sink = ns;
  if (window_lo) *window_lo = lo;
  if (n_tokens) *n_tokens = nt;
  return 0;
}

int gki_rolling_append(void* k_cache, void* v_cache, const void* k_new, const void* v_new, int32_t dtype,
                       int32_t B, int32_t H, int32_t head_dim, int32_t sink_size, int32_t ring_size,
                       int64_t start_pos, int32_t n_new, void* stream) {
  GKI_REQUIRE(dtype == kF32 || dtype == kF16 || dtype == kBF16, 2,
              "unsupported dtype code " + std::to_string(dtype) + " (0=fp32, 1=fp16, 2=bf16)");
  GKI_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128, 2,
              "unsupported head_dim " + std::to_string(head_dim) + " (supported: 16, 32, 64, 128)");
  GKI_REQUIRE(B > 0 && H > 0 && (int64_t)B * H < (1ll << 31) / 4096, 1,
              "gki_rolling_append: B and H must be positive and B * H not too large");
  GKI_REQUIRE(sink_size >= 0 && ring_size >= 1, 1,
              "gki_rolling_append: sink_size must be >= 0 and ring_size >= 1");
  GKI_REQUIRE(start_pos >= 0 && n_new >= 0 && start_pos + n_new < (1ll << kPartialBit), 1,
              "gki_rolling_append: positions must lie in [0, 2^30)");
  GKI_REQUIRE(n_new == 0 || (k_cache && v_cache && k_new && v_new), 1, "gki_rolling_append: null pointer");
  GKI_REQUIRE(n_new == 0 || all_aligned16(k_cache, v_cache, k_new, v_new), 1,
              "gki_rolling_append: caches and new rows must be 16-byte aligned");
  if (n_new == 0) return 0;
  return append_dispatch(dtype, head_dim, k_cache, v_cache, k_new, v_new, B * H, n_new, (int)start_pos,
                         sink_size, ring_size, (hipStream_t)stream);
}

int gki_rolling_decode(const void* q, const void* k_cache, const void* v_cache, void* o, float* lse,
                       int32_t dtype, int32_t B, int32_t H, int32_t H_kv, int32_t n_q, int32_t head_dim,
                       int32_t sink_size, int32_t window_size, int32_t ring_size, int64_t length,
                       float softmax_scale, float* workspace, int32_t n_splits, void* stream) {
  if (int rc = rolling_decode_args(dtype, B, H, H_kv, n_q, head_dim, sink_size, window_size, ring_size,
                                   length, softmax_scale, q, k_cache, v_cache, o, lse, n_splits))
    return rc;
  return rolling_decode_checked(q, k_cache, v_cache, o, lse, dtype, B, H, H_kv, n_q, head_dim, sink_size,
                                window_size, ring_size, length, softmax_scale, workspace, n_splits,
                                stream);
}

int gki_rolling_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, void* o,
                               float* lse, int32_t dtype, int32_t B, int32_t H, int32_t H_kv,
                               int32_t n_q, int32_t head_dim, int32_t sink_size, int32_t window_size,
                               int32_t ring_size, int64_t length, float softmax_scale, int32_t n_splits,
                               void* stream) {
  if (int rc = rolling_decode_args(dtype, B, H, H_kv, n_q, head_dim, sink_size, window_size, ring_size,
                                   length, softmax_scale, q, k_cache, v_cache, o, lse, n_splits))
    return rc;
  float* ws = nullptr;
  if (n_splits > 1) {
    const int64_t need = gki_bsa_decode_workspace_floats(B, H, n_q, head_dim, n_splits);
    GKI_REQUIRE(need <= kScratchFloats, 1,
                "gki_rolling_decode_noalloc: n_splits * B * H * n_q * (head_dim + 2) = " +
                    std::to_string(need) + " floats exceeds the library scratch of " +
                    std::to_string(kScratchFloats) + " floats (16 MiB); use fewer splits or "
                    "gki_rolling_decode with a workspace");
    if (int rc = scratch_on_device((hipStream_t)stream, &ws)) return rc;
  }
  return rolling_decode_checked(q, k_cache, v_cache, o, lse, dtype, B, H, H_kv, n_q, head_dim, sink_size,
                                window_size, ring_size, length, softmax_scale, ws, n_splits, stream);
}

int64_t gki_read_probe_words(int32_t bh) { return bh > 0 ? read_probe_words(bh) : 0; }

int gki_read_probe(const void* k, const void* v, int32_t bh, int64_t n_kv, int32_t row_bytes,
                   int32_t sink_size, int32_t window_size, uint32_t* out, int64_t out_words, void* stream) {
  GKI_REQUIRE(k && v && out, 1, "gki_read_probe: null pointer");
  GKI_REQUIRE(all_aligned16(k, v), 1, "gki_read_probe: k and v must be 16-byte aligned");
  GKI_REQUIRE(bh >= 1 && bh <= (1 << 26) && n_kv >= 1 && row_bytes >= 16 && row_bytes % 16 == 0, 1,
              "gki_read_probe: bh and n_kv must be positive, row_bytes a positive multiple of 16");
  GKI_REQUIRE(sink_size >= 0 && window_size >= 0, 1, "gki_read_probe: sink_size and window_size must be >= 0");
  GKI_REQUIRE(out_words >= read_probe_words(bh), 1,
              "gki_read_probe: out must hold gki_read_probe_words(bh) words");
  const int n_sink = (int)std::min<int64_t>(sink_size, n_kv);
  const int64_t w_lo = std::max<int64_t>(n_sink, n_kv - window_size);
  return read_probe_dispatch(k, v, bh, n_kv, row_bytes, n_sink, w_lo, out, (hipStream_t)stream);
}

}  // extern "C"
