// Block masks and GPU-resident kept-block lists.
//
// * streaming_mask_kernel restates `make_streaming_mask`
//   (sparse_triton_kernel.py:104-181): keep (i, j) iff
//   q_hi > k_lo  and  (k_lo < S  or  k_hi - 1 >= q_lo - W + 1), with
//   q_lo = i*bm + (n_kv - n_q), q_hi = q_lo + bm, k_lo = j*bn, k_hi = k_lo + bn
//   (unclipped, ceil-div grid). Bit-exact with the reference formula.
// * dense_mask_kernel restates `make_dense_mask` (sparse_triton_kernel.py:184-210).
// * tile_mask_kernel maps a mask of any (bm, bn) granularity onto the kernels'
//   fixed tm x tn tiles, taking the token rule into account when causal:
//   0 = nothing to compute, 1 = the lifted mask keeps every element the token
//   rule allows, 2 = partially kept (the kernel then looks the mask up per
//   element).
// * The list kernels turn a {0,1,2} matrix into CSR (rows -> ascending columns)
//   and CSC (columns -> ascending rows) int32 lists, entry = index | (v==2)<<30.
//   Applied to a 0/1 block mask they give exactly `mask.nonzero()` order.
#include "gki_common.cuh"

namespace gki {
namespace {

__global__ void streaming_mask_kernel(int32_t* __restrict__ mask, int64_t n_q, int64_t n_kv,
                                      int64_t sink, int64_t window, int64_t bm, int64_t bn,
                                      int n_qb, int n_kb) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n_qb * n_kb) return;
  const int64_t i = idx / n_kb, j = idx - i * n_kb;
  const int64_t q_lo = i * bm + (n_kv - n_q);
  const int64_t q_hi = q_lo + bm;
  const int64_t k_lo = j * bn;
  const int64_t k_hi = k_lo + bn;
  const bool causal_block = q_hi > k_lo;
  const bool sink_block = k_lo < sink;
  const bool window_block = (k_hi - 1) >= (q_lo - window + 1);
  mask[idx] = (causal_block && (sink_block || window_block)) ? 1 : 0;
}

__global__ void dense_mask_kernel(int32_t* __restrict__ mask, int64_t bm, int64_t bn, int n_qb,
                                  int n_kb, int causal) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n_qb * n_kb) return;
  const int64_t i = idx / n_kb, j = idx - i * n_kb;
  mask[idx] = (!causal || (j * bn < (i + 1) * bm)) ? 1 : 0;
}

// Tile (a, b) of tm x tn is visited (1) if some in-bounds element is kept by the
// lifted block mask and allowed by the token rule (when causal), and partial
// (2) if additionally some in-bounds element allowed by the token rule is NOT
// kept by the lifted mask, so the kernel must consult the mask per element.
__global__ void tile_mask_kernel(const int32_t* __restrict__ mask, int n_qb, int n_kb, int bm, int bn,
                                 int n_q, int n_kv, int tm, int tn, int n_qt, int n_kt, int causal,
                                 int sink, int window, int32_t* __restrict__ tmask) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n_qt * n_kt) return;
  const int a = (int)(idx / n_kt), b = (int)(idx - (int64_t)a * n_kt);
  const int qr0 = a * tm, qr1 = min((a + 1) * tm, n_q) - 1;
  const int kc0 = b * tn, kc1 = min((b + 1) * tn, n_kv) - 1;
  const long off = (long)n_kv - n_q;
  bool visited = false, partial = false;
  if (qr0 <= qr1 && kc0 <= kc1) {
    for (int r = qr0 / bm; r <= qr1 / bm; ++r) {
      const int rq0 = max(qr0, r * bm), rq1 = min(qr1, (r + 1) * bm - 1);
      for (int c = kc0 / bn; c <= kc1 / bn; ++c) {
        const int ck0 = max(kc0, c * bn), ck1 = min(kc1, (c + 1) * bn - 1);
        if (causal && !any_visible(rq0 + off, rq1 + off, ck0, ck1, sink, window)) continue;
        if (mask[(size_t)r * n_kb + c] != 0)
          visited = true;
        else
          partial = true;
      }
    }
  }
  tmask[idx] = visited ? (partial ? 2 : 1) : 0;
}

__global__ __launch_bounds__(256) void row_count_kernel(const int32_t* __restrict__ m, int n_cols,
                                                        int32_t* __restrict__ cnt) {
  __shared__ int part[4];
  const int r = blockIdx.x;
  int c = 0;
  for (int j = threadIdx.x; j < n_cols; j += 256) c += m[(size_t)r * n_cols + j] != 0;
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) cnt[r] = part[0] + part[1] + part[2] + part[3];
}

__global__ __launch_bounds__(256) void col_count_kernel(const int32_t* __restrict__ m, int n_rows,
                                                        int n_cols, int32_t* __restrict__ cnt) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n_cols) return;
  int c = 0;
  for (int r = 0; r < n_rows; ++r) c += m[(size_t)r * n_cols + j] != 0;
  cnt[j] = c;
}

// Single-workgroup inclusive scan into ptr[1..n], ptr[0] = 0.
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* __restrict__ cnt, int n,
                                                    int32_t* __restrict__ ptr) {
  __shared__ int wsum[16];
  __shared__ int carry;
  if (threadIdx.x == 0) {
    carry = 0;
    ptr[0] = 0;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int base = 0; base < n; base += 1024) {
    const int i = base + threadIdx.x;
    int v = i < n ? cnt[i] : 0;
    // inclusive wave scan
    for (int off = 1; off < 64; off <<= 1) {
      const int u = __shfl_up(v, off);
      if (lane >= off) v += u;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    int before = carry;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    if (i < n) ptr[i + 1] = before + v;
    __syncthreads();
    if (threadIdx.x == 1023) carry = before + v;
    __syncthreads();
  }
}

// Stream compaction of one row (grid = rows) or one column (grid = cols).
template <bool kCols>
__global__ __launch_bounds__(256) void fill_kernel(const int32_t* __restrict__ m, int n_rows,
                                                   int n_cols, const int32_t* __restrict__ ptr,
                                                   int32_t* __restrict__ idx) {
  __shared__ int wcnt[4];
  __shared__ int carry;
  const int line = blockIdx.x;
  const int len = kCols ? n_rows : n_cols;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) carry = ptr[line];
  __syncthreads();
  for (int base = 0; base < len; base += 256) {
    const int k = base + threadIdx.x;
    int v = 0;
    if (k < len) v = kCols ? m[(size_t)k * n_cols + line] : m[(size_t)line * n_cols + k];
    const bool keep = v != 0;
    const unsigned long long bal = __ballot(keep);
    const int below = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wcnt[wave] = __popcll(bal);
    __syncthreads();
    int off = carry;
    for (int w = 0; w < wave; ++w) off += wcnt[w];
    if (keep) idx[off + below] = k | ((v == 2 ? 1 : 0) << kPartialBit);
    __syncthreads();
    if (threadIdx.x == 0) carry += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    __syncthreads();
  }
}

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace
}  // namespace gki

using namespace gki;

extern "C" {

int gki_streaming_mask(int32_t* mask, int64_t n_q, int64_t n_kv, int64_t sink, int64_t window,
                       int64_t block_m, int64_t block_n, void* stream) {
  GKI_REQUIRE(mask != nullptr, 1, "gki_streaming_mask: null mask pointer");
  GKI_REQUIRE(n_q > 0 && n_kv > 0, 1, "n_q and n_kv must be positive");
  GKI_REQUIRE(block_m > 0 && block_n > 0, 1, "block_m and block_n must be positive");
  GKI_REQUIRE(sink >= 0 && window >= 0, 1, "sink_size and window_size must be non-negative");
  const int64_t n_qb = (n_q + block_m - 1) / block_m, n_kb = (n_kv + block_n - 1) / block_n;
  GKI_REQUIRE(n_qb * n_kb < (1ll << 31), 1, "block mask too large");
  hipLaunchKernelGGL(streaming_mask_kernel, dim3(blocks_for(n_qb * n_kb, 256)), dim3(256), 0,
                     (hipStream_t)stream, mask, n_q, n_kv, sink, window, block_m, block_n, (int)n_qb,
                     (int)n_kb);
  return check_launch("gki_streaming_mask");
}

int gki_dense_mask(int32_t* mask, int64_t n_q, int64_t n_kv, int64_t block_m, int64_t block_n,
                   int32_t causal, void* stream) {
  GKI_REQUIRE(mask != nullptr, 1, "gki_dense_mask: null mask pointer");
  GKI_REQUIRE(block_m > 0 && block_n > 0 && n_q % block_m == 0 && n_kv % block_n == 0, 1,
              "block_m / block_n must divide n_q / n_kv");
  const int64_t n_qb = n_q / block_m, n_kb = n_kv / block_n;
  if (n_qb * n_kb == 0) return 0;
  hipLaunchKernelGGL(dense_mask_kernel, dim3(blocks_for(n_qb * n_kb, 256)), dim3(256), 0,
                     (hipStream_t)stream, mask, block_m, block_n, (int)n_qb, (int)n_kb, causal);
  return check_launch("gki_dense_mask");
}

int gki_tile_mask(const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m, int32_t block_n,
                  int32_t n_q, int32_t n_kv, int32_t tile_m, int32_t tile_n, int32_t is_causal,
                  int32_t sink_size, int32_t window_size, int32_t* tile_mask, void* stream) {
  GKI_REQUIRE(mask && tile_mask, 1, "gki_tile_mask: null pointer");
  GKI_REQUIRE(n_q > 0 && n_kv > 0 && block_m > 0 && block_n > 0 && tile_m > 0 && tile_n > 0, 1,
              "gki_tile_mask: sizes must be positive");
  GKI_REQUIRE(n_qb == (n_q + block_m - 1) / block_m && n_kb == (n_kv + block_n - 1) / block_n, 1,
              "gki_tile_mask: mask shape does not match ceil(n/block)");
  GKI_REQUIRE(sink_size >= 0 && window_size >= 0, 1, "gki_tile_mask: negative sink/window");
  const int n_qt = (n_q + tile_m - 1) / tile_m, n_kt = (n_kv + tile_n - 1) / tile_n;
  hipLaunchKernelGGL(tile_mask_kernel, dim3(blocks_for((int64_t)n_qt * n_kt, 256)), dim3(256), 0,
                     (hipStream_t)stream, mask, n_qb, n_kb, block_m, block_n, n_q, n_kv, tile_m,
                     tile_n, n_qt, n_kt, is_causal ? 1 : 0, sink_size, window_size, tile_mask);
  return check_launch("gki_tile_mask");
}

int gki_block_list_counts(const int32_t* m, int32_t n_rows, int32_t n_cols, int32_t* row_cnt,
                          int32_t* col_cnt, int32_t* row_ptr, int32_t* col_ptr, void* stream) {
  GKI_REQUIRE(m && row_cnt && col_cnt && row_ptr && col_ptr, 1, "gki_block_list_counts: null pointer");
  GKI_REQUIRE(n_rows > 0 && n_cols > 0, 1, "gki_block_list_counts: empty matrix");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(row_count_kernel, dim3(n_rows), dim3(256), 0, s, m, n_cols, row_cnt);
  hipLaunchKernelGGL(col_count_kernel, dim3(blocks_for(n_cols, 256)), dim3(256), 0, s, m, n_rows,
                     n_cols, col_cnt);
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, s, row_cnt, n_rows, row_ptr);
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, s, col_cnt, n_cols, col_ptr);
  return check_launch("gki_block_list_counts");
}

int gki_block_list_fill(const int32_t* m, int32_t n_rows, int32_t n_cols, const int32_t* row_ptr,
                        const int32_t* col_ptr, int32_t* row_idx, int32_t* col_idx, void* stream) {
  GKI_REQUIRE(m && row_ptr && col_ptr, 1, "gki_block_list_fill: null pointer");
  GKI_REQUIRE(n_rows > 0 && n_cols > 0, 1, "gki_block_list_fill: empty matrix");
  hipStream_t s = (hipStream_t)stream;
  if (row_idx)
    hipLaunchKernelGGL(fill_kernel<false>, dim3(n_rows), dim3(256), 0, s, m, n_rows, n_cols, row_ptr,
                       row_idx);
  if (col_idx)
    hipLaunchKernelGGL(fill_kernel<true>, dim3(n_cols), dim3(256), 0, s, m, n_rows, n_cols, col_ptr,
                       col_idx);
  return check_launch("gki_block_list_fill");
}

}  // extern "C"
