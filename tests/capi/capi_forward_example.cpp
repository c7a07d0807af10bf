// The C-ABI forward from a C++ caller with no Python and no torch: device
// buffers from hipMalloc, the StreamingLLM block mask, the forward kernel's
// tile classes and CSR list built by the library on the GPU, the workgroup
// order from a host copy of the row pointers, then gki_bsa_fwd (the sequence a
// C / cgo / JNI binding follows). The output and LSE are compared with a
// double-precision attention over the token rule computed here on the host and
// with an index-order launch (same bits); a schedule of the wrong size must be
// rejected.
// Built by graph-kernel-injection_amd/build.py, run by
// tests/test_gpu_capi_example.py on an MI355X.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "gki_bsa.h"

#define HIP_OK(x)                                                           \
  do {                                                                      \
    hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                 \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));   \
      return 2;                                                             \
    }                                                                       \
  } while (0)
#define GKI_OK(x)                                                           \
  do {                                                                      \
    if ((x) != 0) {                                                         \
      std::fprintf(stderr, "%s failed: %s\n", #x, gki_last_error());        \
      return 3;                                                             \
    }                                                                       \
  } while (0)

// fp32 -> bf16, round to nearest even (inputs here are finite)
static uint16_t to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float from_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

int main() {
  const int B = 1, H = 2, N = 300, D = 64, S = 4, W = 64, BM = 64, BN = 64;
  const float scale = 0.125f;   // 1 / sqrt(64)
  const size_t elems = (size_t)B * H * N * D;

  // inputs: a fixed linear congruential sequence mapped to [-2, 2), rounded to bf16
  std::vector<uint16_t> hq(elems), hk(elems), hv(elems);
  uint32_t state = 12345u;
  auto next = [&]() {
    state = state * 1664525u + 1013904223u;
    return (float)((state >> 8) & 0xFFFF) / 16384.f - 2.f;
  };
  for (auto* t : {&hq, &hk, &hv})
    for (auto& x : *t) x = to_bf16(next());

  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  int32_t tm16 = 0, tm32 = 0, tmb = 0, tn = 0, tmd = 0, maxq = 0;
  GKI_OK(gki_tile_sizes(&tm16, &tm32, &tmb, &tn, &tmd, &maxq));
  const int nqb = (N + BM - 1) / BM, nkb = (N + BN - 1) / BN;
  const int nqt = (N + tm16 - 1) / tm16, nkt = (N + tn - 1) / tn;

  void *q, *k, *v, *o;
  float* lse;
  int32_t *mask, *tiles, *rc, *cc, *row_ptr, *col_ptr, *row_idx;
  HIP_OK(hipMalloc(&q, elems * 2));
  HIP_OK(hipMalloc(&k, elems * 2));
  HIP_OK(hipMalloc(&v, elems * 2));
  HIP_OK(hipMalloc(&o, elems * 2));
  HIP_OK(hipMalloc((void**)&lse, (size_t)B * H * N * 4));
  HIP_OK(hipMalloc((void**)&mask, (size_t)nqb * nkb * 4));
  HIP_OK(hipMalloc((void**)&tiles, (size_t)nqt * nkt * 4));
  HIP_OK(hipMalloc((void**)&rc, (size_t)nqt * 4));
  HIP_OK(hipMalloc((void**)&cc, (size_t)nkt * 4));
  HIP_OK(hipMalloc((void**)&row_ptr, (size_t)(nqt + 1) * 4));
  HIP_OK(hipMalloc((void**)&col_ptr, (size_t)(nkt + 1) * 4));
  HIP_OK(hipMemcpy(q, hq.data(), elems * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(k, hk.data(), elems * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(v, hv.data(), elems * 2, hipMemcpyHostToDevice));

  // block mask -> the forward kernel's tile classes -> CSR over its q tiles
  GKI_OK(gki_streaming_mask(mask, N, N, S, W, BM, BN, stream));
  GKI_OK(gki_tile_mask(mask, nqb, nkb, BM, BN, N, N, tm16, tn, 1, S, W, tiles, stream));
  GKI_OK(gki_block_list_counts(tiles, nqt, nkt, rc, cc, row_ptr, col_ptr, stream));
  int32_t nnz = 0;
  HIP_OK(hipMemcpyAsync(&nnz, row_ptr + nqt, 4, hipMemcpyDeviceToHost, stream));
  HIP_OK(hipStreamSynchronize(stream));
  HIP_OK(hipMalloc((void**)&row_idx, (size_t)(nnz > 0 ? nnz : 1) * 4));
  GKI_OK(gki_block_list_fill(tiles, nqt, nkt, row_ptr, col_ptr, row_idx, nullptr, stream));

  // the workgroup order (heaviest q tiles first on each XCD), from a host copy
  // of the row pointers
  std::vector<int32_t> h_row_ptr(nqt + 1), h_order((size_t)nqt * B * H);
  HIP_OK(hipMemcpy(h_row_ptr.data(), row_ptr, (nqt + 1) * 4, hipMemcpyDeviceToHost));
  GKI_OK(gki_fwd_order(h_row_ptr.data(), nqt, B * H, h_order.data()));
  int32_t* order;
  HIP_OK(hipMalloc((void**)&order, h_order.size() * 4));
  HIP_OK(hipMemcpy(order, h_order.data(), h_order.size() * 4, hipMemcpyHostToDevice));

  // a schedule for another tile count is rejected before anything launches
  if (gki_bsa_fwd(q, k, v, o, lse, 2, B, H, H, N, N, D, row_ptr, row_idx, nqt + 1, order, mask, nqb,
                  nkb, BM, BN, scale, 1, S, W, stream) == 0) {
    std::fprintf(stderr, "a wrong-size schedule was accepted\n");
    return 4;
  }
  GKI_OK(gki_bsa_fwd(q, k, v, o, lse, 2, B, H, H, N, N, D, row_ptr, row_idx, nqt, order, mask, nqb, nkb,
                     BM, BN, scale, 1, S, W, stream));
  std::vector<uint16_t> ho(elems), ho_idx(elems);
  std::vector<float> hl((size_t)B * H * N), hl_idx(hl.size());
  HIP_OK(hipMemcpyAsync(ho.data(), o, elems * 2, hipMemcpyDeviceToHost, stream));
  HIP_OK(hipMemcpyAsync(hl.data(), lse, hl.size() * 4, hipMemcpyDeviceToHost, stream));
  // the same launch in index order (no table) gives the same bits
  GKI_OK(gki_bsa_fwd(q, k, v, o, lse, 2, B, H, H, N, N, D, row_ptr, row_idx, nqt, nullptr, mask, nqb, nkb,
                     BM, BN, scale, 1, S, W, stream));
  HIP_OK(hipMemcpyAsync(ho_idx.data(), o, elems * 2, hipMemcpyDeviceToHost, stream));
  HIP_OK(hipMemcpyAsync(hl_idx.data(), lse, hl.size() * 4, hipMemcpyDeviceToHost, stream));
  HIP_OK(hipStreamSynchronize(stream));
  if (ho != ho_idx || std::memcmp(hl.data(), hl_idx.data(), hl.size() * 4) != 0) {
    std::fprintf(stderr, "the ordered launch differs from the index-order launch\n");
    return 5;
  }

  // host reference: softmax over the keys the token rule leaves each row
  // (k <= q and (k < S or k >= q - W + 1); the streaming block mask keeps a
  // superset of them), in double
  double max_o = 0, max_lse = 0;
  int bad = 0;
  for (int h = 0; h < B * H; ++h) {
    const size_t base = (size_t)h * N * D;
    for (int i = 0; i < N; ++i) {
      std::vector<double> s;
      std::vector<int> keys;
      double mx = -1e300;
      for (int j = 0; j <= i; ++j) {
        if (!(j < S || j >= i - W + 1)) continue;
        double dot = 0;
        for (int d = 0; d < D; ++d)
          dot += (double)from_bf16(hq[base + (size_t)i * D + d]) * from_bf16(hk[base + (size_t)j * D + d]);
        s.push_back(dot * scale);
        keys.push_back(j);
        mx = std::max(mx, dot * scale);
      }
      double l = 0;
      for (double& x : s) l += (x = std::exp(x - mx));
      const double lse_ref = mx + std::log(l);
      const double lse_got = (double)hl[(size_t)h * N + i];   // natural log, as the reference
      max_lse = std::max(max_lse, std::fabs(lse_got - lse_ref));
      if (std::fabs(lse_got - lse_ref) > 2.5e-3) ++bad;
      for (int d = 0; d < D; ++d) {
        double ref = 0;
        for (size_t t = 0; t < keys.size(); ++t)
          ref += s[t] / l * from_bf16(hv[base + (size_t)keys[t] * D + d]);
        const double got = from_bf16(ho[base + (size_t)i * D + d]);
        const double err = std::fabs(got - ref);
        max_o = std::max(max_o, err);
        if (!(err <= 2e-2 + 1e-2 * std::fabs(ref))) ++bad;
      }
    }
  }
  std::printf("abi %d, %d kept forward tiles: max |dO| %.3e, max |dLSE| %.3e, %d out of tolerance\n",
              gki_abi_version(), nnz, max_o, max_lse, bad);
  for (void* p : {q, k, v, o, (void*)lse, (void*)mask, (void*)tiles, (void*)rc, (void*)cc,
                  (void*)row_ptr, (void*)col_ptr, (void*)row_idx, (void*)order})
    HIP_OK(hipFree(p));
  HIP_OK(hipStreamDestroy(stream));
  if (bad) return 1;
  std::printf("capi forward example passed\n");
  return 0;
}
