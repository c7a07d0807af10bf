// Block-sparse StreamingLLM attention: decode-step kernels for gfx950.
//
// The reference has no decode kernel: its harness runs `_fwd_kernel` with
// BLOCK_M = 1 (benchmark.py:802-804), which gate-loads every one of the n_kb
// mask entries and does a 1-row tl.dot per kept tile. Here the decode step
// (n_q <= 4 query rows at the end of the KV cache, q_offset = n_kv - n_q) is a
// bandwidth-bound split-KV pass:
//   * decode_tokens_kernel (once per mask, cached by the host) expands the kept
//     kv tiles of the single decode q tile into exactly the positions some query
//     row can see (per tile its sink run and its window run): S + W positions
//     per head for n_q = 1;
//   * decode_kernel: workgroup (bh, split) takes an equal slice of that stream
//     and its 12 waves (8 for several rows) take the slice's rounds of 4
//     token-row passes in turn (wave w: rounds w, w + 12, ..., so the workgroup
//     sweeps its rows in address order; 16-byte non-temporal K and V loads,
//     D/8 lanes per row), double-buffered: the next round's loads are issued
//     before the current one is consumed (scores, wave-local online softmax,
//     P V), so every CU keeps HBM busy through its compute. No barrier until
//     the end, where the waves merge in LDS. With one split per head the workgroup writes O and
//     LSE itself; otherwise it writes (acc[D], m, l) to a workspace and
//   * combine_kernel (one wave per row) merges the splits:
//     O = sum acc_s 2^(m_s-M) / sum l_s 2^(m_s-M), LSE = (M + log2 L) ln 2
//     (the partials' max is in base 2; the LSE is natural, as the forward
//     stores it), with the (O = 0, LSE = 0) sentinel for empty rows.
// Cross-workgroup merging goes through a second launch on purpose: publishing
// partials across XCDs inside one kernel needs agent-scope fences, which on
// gfx950 write back and invalidate L2.
// Numerics follow the reference forward: fp32 scores scaled after the dot, P
// cast to V's dtype before P V, token mask causal & (sink | window).
#include <atomic>
#include <string>
#include <type_traits>

#include "gki_common.cuh"

namespace gki {
namespace {

// Slack of the decode's lazy reference max, in log2 units: p = exp2(s - m) <= 2^8.
constexpr float kDecodeSlack = 8.f;


// The tokens of kv tile `kt` that some of the n_q rows can see, as at most two
// ascending runs [lo1, hi1), [lo2, hi2): the sink run and the window run (one
// run when they touch; the whole in-bounds tile when not causal). The stream is
// exactly the union of the rows' visible positions, so for a single query row
// no token in it needs the token rule.
__device__ inline void tile_runs(const Geom& g, int kt, int& lo1, int& hi1, int& lo2, int& hi2) {
  const int lo = kt * kTileN, hi = min(lo + kTileN, g.n_kv);
  lo1 = lo;
  hi1 = hi;
  lo2 = hi2 = 0;
  if (!g.causal || lo >= hi) return;
  const int qa = g.q_off, qb = g.n_kv - 1;          // absolute positions of rows 0 and n_q-1
  const int a_hi = min(hi, qb + 1);
  const int s_hi = min(a_hi, g.sink);               // sink run [lo, s_hi)
  const int w_lo = max(lo, qa - g.window + 1);      // window run [w_lo, a_hi)
  const bool has_s = lo < s_hi, has_w = w_lo < a_hi;
  if (has_s && has_w && w_lo <= s_hi) {             // they touch: one run
    hi1 = max(s_hi, a_hi);
  } else if (has_s) {
    hi1 = s_hi;
    if (has_w) {
      lo2 = w_lo;
      hi2 = a_hi;
    }
  } else if (has_w) {
    lo1 = w_lo;
    hi1 = a_hi;
  } else {
    hi1 = lo;                                       // nothing visible
  }
}

// One workgroup: tile list -> token positions (| partial << 30) and their count.
__global__ __launch_bounds__(256) void decode_tokens_kernel(Geom g, const int32_t* __restrict__ list,
                                                            int n_ent, int32_t* __restrict__ tok,
                                                            int32_t* __restrict__ count) {
  __shared__ int red[4];
  __shared__ int carry;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int c = 0; c < n_ent; c += 256) {
    const int e = c + threadIdx.x;
    int lo1 = 0, hi1 = 0, lo2 = 0, hi2 = 0, flag = 0;
    if (e < n_ent) {
      const int ent = list[e];
      tile_runs(g, ent & kIdxMask, lo1, hi1, lo2, hi2);
      flag = (ent >> kPartialBit) & 1;
    }
    const int len1 = hi1 - lo1, len = len1 + (hi2 - lo2);
    int inc = len;
    for (int off = 1; off < 64; off <<= 1) {
      const int u = __shfl_up(inc, off);
      if (lane >= off) inc += u;
    }
    if (lane == 63) red[wave] = inc;
    __syncthreads();
    int start = carry;
    for (int w = 0; w < wave; ++w) start += red[w];
    start += inc - len;
    for (int t = 0; t < len; ++t)
      tok[start + t] = (t < len1 ? lo1 + t : lo2 + (t - len1)) | (flag << kPartialBit);
    __syncthreads();
    if (threadIdx.x == 0) carry += red[0] + red[1] + red[2] + red[3];
    __syncthreads();
  }
  if (threadIdx.x == 0) *count = carry;
}

// Waves per decode workgroup: 12 (3 per SIMD, 168 VGPRs each) for one query
// row; 8 (2 per SIMD, 256 VGPRs) for up to four rows, whose per-row scores,
// query and accumulators would not fit 168 registers.
template <int NQ> constexpr int decode_waves() { return NQ == 1 ? 12 : 8; }

// Token sources of the decode kernel: entry(t) is the t-th entry of the token
// stream (position | partial << 30), row(e) the K / V row that holds it.
//   ListTokens: the explicit stream of gki_decode_tokens over a full cache
//     (row = position).
//   RingTokens: a rolling cache of `sink` sink slots followed by a ring of
//     `ring` slots (position p >= sink lives in slot sink + (p - sink) mod ring).
//     The stream is computed, not loaded: positions 0 .. n_sink-1, then w_lo,
//     w_lo + 1, ... -- the same ascending positions the full-cache stream holds.
struct ListTokens {
  const int32_t* __restrict__ tok;
  __device__ inline int entry(int t) const { return tok[t]; }
  __device__ inline int row(int e) const { return e & kIdxMask; }
};

struct RingTokens {
  int n_sink, w_lo, sink, ring;
  int base;                               // (w_lo - sink) mod ring
  __device__ inline int entry(int t) const { return t < n_sink ? t : w_lo + (t - n_sink); }
  __device__ inline int row(int e) const {
    const int p = e & kIdxMask;
    const int j = base + (p - w_lo);      // in [base, base + ring) for window positions
    return p < sink ? p : sink + (j >= ring ? j - ring : j);
  }
};

// One round of a wave: NU passes of TPW token rows, LPT lanes per row, one
// 16-byte K and V chunk per lane and pass.
template <typename T, int D, int NU>
struct DecodeRound {
  using S = typename T::storage;
  static constexpr int VEC = 16 / sizeof(S);
  static constexpr int LPT = D / VEC;
  static constexpr int TPW = 64 / LPT;
  static constexpr int RT = NU * TPW;
  int pj[NU];
  uint4 kr[NU], vr[NU];
  // Token positions of round t0 for this lane's row (one dword load per pass).
  // Rows past the wave's slice read the slice's last entry, flagged by the
  // sign bit: every load stays in range and unconditional (no branch, so no
  // wait is forced on the loads in flight) and the row is masked when consumed.
  template <typename Src>
  __device__ static inline void positions(const Src& src, int t0, int w1, int tk, int (&pos)[NU]) {
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int t = t0 + u * TPW + tk;
      const int v = src.entry(t < w1 ? t : w1 - 1);
      pos[u] = t < w1 ? v : (v | (1 << 31));
    }
  }
  template <typename Src>
  __device__ inline void fetch(const Src& src, const int (&pos)[NU], int ch, const S* __restrict__ K,
                               const S* __restrict__ V, size_t kb) {
#pragma unroll
    for (int u = 0; u < NU; ++u) pj[u] = pos[u];
#pragma unroll
    for (int u = 0; u < NU; ++u) kr[u] = ld_nt16(K + kb + (size_t)src.row(pj[u]) * D + ch * VEC);
#pragma unroll
    for (int u = 0; u < NU; ++u) vr[u] = ld_nt16(V + kb + (size_t)src.row(pj[u]) * D + ch * VEC);
  }
};

// A lane's slice of the workgroup's query rows and its dot product with one
// 16-byte K chunk: 16-bit inputs stay packed and go through v_dot2_f32_* (the
// products are exact in fp32, accumulation in fp32); fp32 inputs use FMAs.
template <typename T, int NQ>
struct DecodeQ {
  uint4 raw[NQ];
  __device__ inline float dot(int r, const uint4& k) const {
    float p = T::dot2(raw[r].x, k.x, 0.f);
    p = T::dot2(raw[r].y, k.y, p);
    p = T::dot2(raw[r].z, k.z, p);
    return T::dot2(raw[r].w, k.w, p);
  }
};
template <int NQ>
struct DecodeQ<F32, NQ> {
  uint4 raw[NQ];
  __device__ inline float dot(int r, const uint4& k) const {
    const float* q = (const float*)&raw[r];
    const float* kf = (const float*)&k;
    float p = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) p += q[i] * kf[i];
    return p;
  }
};

// Row r of the workgroup is query row qrow[r] (qrow = n_q marks an unused row,
// which elem_valid rejects).
// EXACT: every row sits at the same position (n_q == 1) and the stream holds
// exactly the positions it can see, so a token is valid unless it is padding
// or its tile's block-mask entry (partial tiles only) drops it -- one test per
// token instead of the token rule per (row, token).
template <typename T, int D, int NQ, int NU, bool EXACT>
__device__ inline void decode_consume(const Geom& g, const DecodeRound<T, D, NU>& rd,
                                      const int (&qrow)[NQ], const DecodeQ<T, NQ>& qv,
                                      float (&m)[NQ], float (&l)[NQ],
                                      float (&acc)[NQ][16 / sizeof(typename T::storage)]) {
  using S = typename T::storage;
  using R = DecodeRound<T, D, NU>;
  constexpr int VEC = R::VEC, LPT = R::LPT;
  float sc[NQ][NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    bool ok_u = rd.pj[u] >= 0;                // sign bit: padding row of the round
    if constexpr (EXACT) {
      if (ok_u && ((rd.pj[u] >> kPartialBit) & 1))
        ok_u = g.mask[(size_t)((g.n_q - 1) / g.bm) * g.n_kb + (rd.pj[u] & kIdxMask) / g.bn] != 0;
    }
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      float part = qv.dot(r, rd.kr[u]);
      part = group_sum<LPT>(part);             // the LPT lanes of a token row
      bool ok = ok_u;
      if constexpr (!EXACT) {
        if (ok) ok = elem_valid(g, qrow[r], rd.pj[u] & kIdxMask, (rd.pj[u] >> kPartialBit) & 1);
      }
      sc[r][u] = ok ? part * g.scale_log2 : kNegInf;
    }
  }
#pragma unroll
  for (int r = 0; r < NQ; ++r) {
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < NU; ++u) mx = fmaxf(mx, sc[r][u]);
    // Lazy reference max (wave-uniform): it moves, to the exact running max,
    // only when some score of the round exceeds it by the slack, so p stays
    // below 2^slack and the rescale (a cross-lane max, one exp2, VEC + 1
    // multiplies) is skipped in almost every round. acc / l is exact for any
    // reference max.
    if (__any(mx > m[r] + kDecodeSlack)) {
      mx = cross_group_max<LPT>(mx);           // scores are uniform within a token row
      const float m_new = fmaxf(m[r], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[r] - m_new);   // m = -inf: 0
      m[r] = m_new;
      l[r] *= alpha;
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[r][i] *= alpha;
    }
    const float mu = m[r] == kNegInf ? 0.f : m[r];
    float rs = 0.f;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const float p = __builtin_amdgcn_exp2f(sc[r][u] - mu);
      rs += p;
      const float pv = T::is_f32 ? p : T::to_float(T::from_float(p));   // P -> V dtype
      // a padding row re-reads a real V row: zero it so 0 * inf cannot appear
      const uint4 vz = rd.pj[u] >= 0 ? rd.vr[u] : make_uint4(0, 0, 0, 0);
      const S* e = (const S*)&vz;
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[r][i] += pv * T::to_float(e[i]);
    }
    l[r] += rs;
  }
}

// kv_rows: K / V rows per (b, kv head) (n_kv for a full cache, sink + ring
// slots for a rolling one). A workgroup serves gq consecutive q heads of one kv
// head (gq = group when group * n_q <= kDecodeMaxQ, else 1): its n_rows =
// gq * n_q rows are rows bhq0 * n_q + r of Q / O / LSE, r = head * n_q + query
// row, and share every K / V load. Workgroups run in the logical order (kv
// stream, split, q head of the stream's group), XCD-remapped: when the q heads
// of a group get one workgroup each (gq = 1), those reading one K / V slice are
// neighbours on one XCD and share its L2 (one HBM read per slice, not group).
template <typename T, int D, int NQ, typename Src, bool EXACT>
__global__ __launch_bounds__(64 * decode_waves<NQ>()) void decode_kernel(
    Geom g, const typename T::storage* __restrict__ Q, const typename T::storage* __restrict__ K,
    const typename T::storage* __restrict__ V, typename T::storage* __restrict__ O,
    float* __restrict__ LSE, float* __restrict__ ws, Src src, int kv_rows, int n_tokens,
    int n_splits, int gq) {
  constexpr int NU = NQ == 1 ? 4 : 3;   // passes per round; two rounds in flight (double-buffered)
  using R = DecodeRound<T, D, NU>;
  constexpr int VEC = R::VEC, LPT = R::LPT, RT = R::RT;
  constexpr int NW = decode_waves<NQ>();
  __shared__ float wm[NW][NQ], wl[NW][NQ];
  __shared__ float wacc[NW][NQ][D];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lb = xcd_remap(blockIdx.x, gridDim.x);
  const int gh = gq == 1 ? g.group : 1;                    // workgroups per K / V slice
  const int gj = lb % gh, rest = lb / gh;
  const int split = rest % n_splits, wgh = (rest / n_splits) * gh + gj;
  const int n_rows = gq * g.n_q;
  const int bhq0 = wgh * gq;                               // first q head of this workgroup
  const size_t qb = (size_t)bhq0 * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bhq0) * kv_rows * D;
  // this workgroup's slice of the token stream
  const int g0 = (int)(((int64_t)n_tokens * split) / n_splits);
  const int g1 = (int)(((int64_t)n_tokens * (split + 1)) / n_splits);
  // The waves take the slice's rounds of RT tokens in turn (wave w: rounds w,
  // w + NW, ...), so the workgroup sweeps its K / V rows in address order:
  // with the memory-side cache cold this reads 2% faster than one contiguous
  // part per wave (12 concurrent streams per slice), and the same warm.
  constexpr int ST = NW * RT;
  const int w0 = g0 + wave * RT;
  const int w1 = g1;
  const int tk = lane / LPT, ch = lane % LPT;

  DecodeQ<T, NQ> qv;
  int qrow[NQ];
#pragma unroll
  for (int r = 0; r < NQ; ++r) {
    qrow[r] = r < n_rows ? r % g.n_q : g.n_q;
    qv.raw[r] = r < n_rows ? *(const uint4*)(Q + qb + (size_t)r * D + ch * VEC) : make_uint4(0, 0, 0, 0);
  }
  // wave-local online softmax state; m is uniform across the wave, l and acc
  // are per token-row group and summed at the end
  float m[NQ], l[NQ], acc[NQ][VEC];
#pragma unroll
  for (int r = 0; r < NQ; ++r) {
    m[r] = kNegInf;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[r][i] = 0.f;
  }

  // Rounds alternate between two register sets: the K / V loads of round i+1
  // (and the positions of round i+2) are issued before round i is consumed, so
  // HBM streams while the VALU works. Loads complete in order, so each wait
  // covers only the oldest round.
  if (w0 < w1) {
    R ra, rb;
    int pa[NU], pb[NU];
    R::positions(src, w0, w1, tk, pa);
    R::positions(src, w0 + ST, w1, tk, pb);
    ra.fetch(src, pa, ch, K, V, kb);
    for (int t0 = w0; t0 < w1; t0 += 2 * ST) {
      const bool has_b = t0 + ST < w1;
      if (has_b) {
        R::positions(src, t0 + 2 * ST, w1, tk, pa);
        rb.fetch(src, pb, ch, K, V, kb);
      }
      decode_consume<T, D, NQ, NU, EXACT>(g, ra, qrow, qv, m, l, acc);
      if (!has_b) break;
      if (t0 + 2 * ST < w1) {
        R::positions(src, t0 + 3 * ST, w1, tk, pb);
        ra.fetch(src, pa, ch, K, V, kb);
      }
      decode_consume<T, D, NQ, NU, EXACT>(g, rb, qrow, qv, m, l, acc);
    }
  }
  // merge the token-row groups of the wave (same m), then the four waves
#pragma unroll
  for (int r = 0; r < NQ; ++r) {
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[r][i] += __shfl_xor(acc[r][i], off);
    }
    // l was accumulated once per token by every lane of its group
    float lw = l[r];
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) lw += __shfl_xor(lw, off);
    if (lane < LPT) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) wacc[wave][r][ch * VEC + i] = acc[r][i];
    }
    if (lane == 0) {
      wm[wave][r] = m[r];
      wl[wave][r] = lw;
    }
  }
  __syncthreads();
  const size_t row_stride = D + 2;
  float* part = ws + ((size_t)wgh * n_splits + split) * n_rows * row_stride;
  for (int idx = tid; idx < n_rows * D; idx += 64 * NW) {
    const int r = idx / D, d = idx - r * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][r]);
    const float Mu = M == kNegInf ? 0.f : M;
    float L = 0.f, a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float sw = __builtin_amdgcn_exp2f(wm[w][r] - Mu);
      L += wl[w][r] * sw;
      a += wacc[w][r][d] * sw;
    }
    if (n_splits == 1) {
      const bool valid = L > 0.f;
      O[qb + (size_t)r * D + d] = T::from_float(valid ? a / L : 0.f);
      if (d == 0) LSE[(size_t)bhq0 * g.n_q + r] = valid ? lse_natural(M, L) : 0.f;
    } else {
      part[r * row_stride + d] = a;
      if (d == 0) {
        part[r * row_stride + D] = M;
        part[r * row_stride + D + 1] = L;
      }
    }
  }
}

// Merge the n_splits partials of one (b, h, row): one wave per row.
template <typename T, int D>
__global__ __launch_bounds__(64) void combine_kernel(const float* __restrict__ ws,
                                                     typename T::storage* __restrict__ O,
                                                     float* __restrict__ LSE, int n_q, int n_splits) {
  const int row = blockIdx.x;
  const int bh = row / n_q, r = row - bh * n_q;
  const int lane = threadIdx.x;
  const size_t row_stride = D + 2;
  const float* base = ws + (size_t)bh * n_splits * n_q * row_stride + (size_t)r * row_stride;
  const size_t sstride = (size_t)n_q * row_stride;
  // unrolled so that several splits' loads are in flight at once (the
  // partials were just written by other CUs: every load goes past this L2)
  float M = kNegInf;
#pragma unroll 4
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, base[s * sstride + D]);
  const float Mu = M == kNegInf ? 0.f : M;
  float L = 0.f;
  float a[D / 64];
#pragma unroll
  for (int j = 0; j < D / 64; ++j) a[j] = 0.f;
#pragma unroll 4
  for (int s = 0; s < n_splits; ++s) {
    const float* ps = base + s * sstride;
    const float w = __builtin_amdgcn_exp2f(ps[D] - Mu);
    L += ps[D + 1] * w;
#pragma unroll
    for (int j = 0; j < D / 64; ++j) a[j] += ps[lane + 64 * j] * w;
  }
  const bool valid = L > 0.f;
#pragma unroll
  for (int j = 0; j < D / 64; ++j)
    O[(size_t)row * D + lane + 64 * j] = T::from_float(valid ? a[j] / L : 0.f);
  if (lane == 0) LSE[row] = valid ? lse_natural(M, L) : 0.f;
}

template <typename T, int D, int NQ, typename Src>
int launch_decode_t(const Geom& g, const void* q, const void* k, const void* v, void* o, float* lse,
                    const Src& src, int kv_rows, int n_tokens, float* ws, int n_splits, int gq,
                    hipStream_t stream, const char* what) {
  using S = typename T::storage;
  const int n_wgh = g.B * g.H / gq, n_rows = gq * g.n_q;
  // one query position (always so for a single-row workgroup): the stream is
  // exact for every row
  if (NQ == 1 || g.n_q == 1)
    hipLaunchKernelGGL((decode_kernel<T, D, NQ, Src, true>), dim3(n_wgh * n_splits),
                       dim3(64 * decode_waves<NQ>()), 0, stream, g, (const S*)q, (const S*)k,
                       (const S*)v, (S*)o, lse, ws, src, kv_rows, n_tokens, n_splits, gq);
  else if constexpr (NQ > 1)
    hipLaunchKernelGGL((decode_kernel<T, D, NQ, Src, false>), dim3(n_wgh * n_splits),
                       dim3(64 * decode_waves<NQ>()), 0, stream, g, (const S*)q, (const S*)k,
                       (const S*)v, (S*)o, lse, ws, src, kv_rows, n_tokens, n_splits, gq);
  if (n_splits > 1)
    hipLaunchKernelGGL((combine_kernel<T, D>), dim3(n_wgh * n_rows), dim3(64), 0, stream, ws, (S*)o, lse,
                       n_rows, n_splits);
  return check_launch(what);
}

template <typename Src>
int launch_decode(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                  void* o, float* lse, const Src& src, int kv_rows, int n_tokens, float* ws,
                  int n_splits, hipStream_t stream, const char* what) {
  const int gq = decode_heads_per_workgroup(g.group, g.n_q);
#define GKI_DECODE_CASE(TT, DD)                                                                   \
  if (gq * g.n_q == 1)                                                                            \
    return launch_decode_t<TT, DD, 1>(g, q, k, v, o, lse, src, kv_rows, n_tokens, ws, n_splits,   \
                                      gq, stream, what);                                          \
  return launch_decode_t<TT, DD, kDecodeMaxQ>(g, q, k, v, o, lse, src, kv_rows, n_tokens, ws,     \
                                              n_splits, gq, stream, what);
#define GKI_DECODE_DTYPE(TT)                                                                      \
  if (head_dim == 64) {                                                                           \
    GKI_DECODE_CASE(TT, 64)                                                                       \
  }                                                                                               \
  if (head_dim == 128) {                                                                          \
    GKI_DECODE_CASE(TT, 128)                                                                      \
  }                                                                                               \
  return fail(2, "decode kernel supports head_dim 64 and 128, got " + std::to_string(head_dim));
  if (dtype == kF32) {
    GKI_DECODE_DTYPE(F32)
  }
  if (dtype == kF16) {
    GKI_DECODE_DTYPE(F16)
  }
  GKI_DECODE_DTYPE(BF16)
#undef GKI_DECODE_DTYPE
#undef GKI_DECODE_CASE
}

// ---------------------------------------------------------------------------
// Decode on the matrix cores: 16-bit K / V, head_dim 64 or 128, the n_q query
// rows of a group's q heads (2 .. 2 * kDecodeTileM rows per K / V stream). Those
// rows are the B operand of S^T = K Q^T (NB blocks of 16 columns, the unused
// ones zero); with
// several query positions (EXACT false) each row applies the token rule; each wave takes 16 tokens of every 64-token chunk of the
// workgroup's slice of the stream; the chunk's K / V rows are gathered into
// LDS by LDS-DMA (swizzled as the forward's tiles), so no registers hold loads
// in flight and two chunks are requested at once. P^T of the wave's 16 tokens
// is the B operand of O^T += V^T P^T (v_mfma_f32_16x16x16, V^T from one
// transposed LDS read); the row sums add the fp32 P. The four waves' states
// merge through LDS into the same partials / output as decode_kernel.
// ---------------------------------------------------------------------------
// One ds_read_b64_tr_b16: lane (g, c) gets tile[k0 + 4g + e][n0 + c], e = 0..3,
// the K-operand layout of v_mfma_f32_16x16x16_{bf16,f16} for a K-major matrix.
template <int D>
__device__ inline uint2 lds_tr4(const uint16_t* tile, int k0, int n0, int lane) {
  const int g = lane >> 4, l = lane & 15;
  const uint16_t* p = tile + lds_off<D>(k0 + 4 * g + (l >> 2), n0 + 4 * (l & 3));
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p));
}

template <typename T>
__device__ inline floatx4 mfma16k(const uint2& a, const uint2& b, floatx4 c) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
  if constexpr (std::is_same<T, BF16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h16x4, a),
                                                 __builtin_bit_cast(h16x4, b), c, 0, 0, 0);
}

// s_waitcnt vmcnt(N), other counters untouched (N < 64: the field's low four
// bits at 3:0, its high two at 15:14).
template <int N>
__device__ inline void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Chunks in flight per workgroup (LDS ring of K and V tiles): three or four
// measured no faster than two on the grouped-query and four-position steps.
template <int D>
constexpr int decode_mfma_bufs() { return 2; }
// K / V ring, plus the workgroup's query rows (at most 2 * kDecodeTileM) when
// they are staged through LDS (QLDS).
template <int D, bool QLDS>
constexpr int decode_mfma_lds() {
  return 2 * decode_mfma_bufs<D>() * kTileN * D * 2 + (QLDS ? 2 * kDecodeTileM * D * 2 : 0);
}

// Wait until at most k chunks (of 2 * NP LDS-DMA instructions per wave each,
// k <= NBUF) are still in flight: every memory operation issued before them
// has completed.
template <int NP, int NBUF>
__device__ inline void wait_chunks(int k) {
  static_assert(NBUF <= 4 && 8 * NP < 64, "wait_chunks covers up to four chunks in flight");
  if (k <= 0) vm_wait<0>();
  else if (k == 1) vm_wait<2 * NP>();
  else if (k == 2) vm_wait<4 * NP>();
  else if (k == 3) vm_wait<6 * NP>();
  else vm_wait<8 * NP>();
}

template <typename T, int D, bool EXACT, int NB, bool QLDS>
__global__ __launch_bounds__(256) void decode_mfma_kernel(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ LSE,
    float* __restrict__ ws, RingTokens src, int kv_rows, int n_tokens, int n_splits) {
  static_assert(D == 64 || D == 128, "matrix-core decode: head_dim 64 or 128");
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int NP = D / 32;                 // 1 KB LDS blocks per wave and 64-row tile
  constexpr int NBUF = decode_mfma_bufs<D>();
  extern __shared__ __align__(16) uint16_t decode_lds[];
  uint16_t* const sk = decode_lds;                       // [NBUF][64 * D]
  uint16_t* const sv = decode_lds + NBUF * kTileN * D;   // [NBUF][64 * D]
  uint16_t* const sq = decode_lds + 2 * NBUF * kTileN * D;   // [n_rows][D], row-major

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4, col = lane & 15;
  const int lb = xcd_remap(blockIdx.x, gridDim.x);
  const int split = lb % n_splits, wgh = lb / n_splits;     // wgh: one K / V stream
  const int n_rows = g.group * g.n_q;                       // row r: q head r / n_q, query r % n_q
  const int bhq0 = wgh * g.group;
  const size_t qb = (size_t)bhq0 * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bhq0) * kv_rows * D;
  const int g0 = (int)(((int64_t)n_tokens * split) / n_splits);
  const int g1 = (int)(((int64_t)n_tokens * (split + 1)) / n_splits);
  const int n_chunks = (g1 - g0 + kTileN - 1) / kTileN;

  // Q^T operand of column block h: lane (grp, col) holds elements 32ks + 8grp ..
  // +7 of q row 16h + col. QLDS (a split stream: a short slice, where the start
  // weighs): the workgroup's n_rows query rows, contiguous in Q, are staged into
  // LDS by LDS-DMA ahead of the first K / V chunks (1 KB per wave instruction;
  // lanes past the rows re-read the last 16 bytes, landing in LDS no row uses),
  // so their latency overlaps the K / V stream instead of preceding it;
  // otherwise (a long slice) they are loaded into registers first.
  uint4 qf[NB][KS];
  if constexpr (QLDS) {
    const int q_bytes = n_rows * D * 2;
#pragma unroll
    for (int j = wave; j < (2 * kDecodeTileM * D * 2) / 1024; j += 4)
      if (j * 1024 < q_bytes)
        dma_load16((const char*)(Q + qb) + min(j * 1024 + 16 * lane, q_bytes - 16), lds_addr(sq) + j * 1024);
  } else {
#pragma unroll
    for (int h = 0; h < NB; ++h) {
      const int r = 16 * h + col;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[h][ks] = r < n_rows ? q_words(g, *(const uint4*)(Q + qb + (size_t)r * D + 32 * ks + 8 * grp))
                               : make_uint4(0, 0, 0, 0);
    }
    dma_wait();   // the Q loads are complete before any LDS-DMA is in flight
  }
  int my_q[NB];                                             // the lane's query position index
#pragma unroll
  for (int h = 0; h < NB; ++h) my_q[h] = (16 * h + col) % g.n_q;

  // this lane's chunk of LDS block 4p + wave of a tile: row, swizzled column
  int drow[NP], dcol[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int e = (4 * p + wave) * 512 + 8 * lane;
    drow[p] = e / D;
    dcol[p] = (((e % D) >> 3) ^ lds_swz<D>(drow[p])) << 3;
  }
  // gather chunk c of the slice into buffer b (rows past the slice repeat its
  // last token and are masked when consumed)
  auto issue = [&](int c, int b) {
    const int c0 = g0 + c * kTileN;
    const uint32_t lk = lds_addr(sk + b * kTileN * D), lv = lds_addr(sv + b * kTileN * D);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int t = min(c0 + drow[p], g1 - 1);
      const size_t off = kb + (size_t)src.row(src.entry(t)) * D + dcol[p];
      dma_load16(K + off, lk + (4 * p + wave) * 1024);
      dma_load16(V + off, lv + (4 * p + wave) * 1024);
    }
  };

  floatx4 o[NB][DT];
  float lsum[NB], m[NB];                       // per column block: row 16h + col
#pragma unroll
  for (int h = 0; h < NB; ++h) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[h][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    lsum[h] = 0.f;
    m[h] = kNegInf;
  }

#pragma unroll
  for (int c = 0; c < NBUF; ++c)
    if (c < n_chunks) issue(c, c);
  if constexpr (QLDS) {
    // the Q rows have landed once at most the chunks just issued are in flight
    // (vector memory operations complete in order); every wave's share of
    // them is visible after the barrier
    wait_chunks<NP, NBUF>(min(NBUF, n_chunks));
    __syncthreads();
#pragma unroll
    for (int h = 0; h < NB; ++h) {
      const int r = 16 * h + col;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[h][ks] = r < n_rows ? q_words(g, *(const uint4*)(sq + r * D + 32 * ks + 8 * grp))
                               : make_uint4(0, 0, 0, 0);
    }
  }
  for (int c = 0; c < n_chunks; ++c) {
    const int b = c % NBUF;
    // chunk c has landed; the up to NBUF - 1 chunks issued after it may stay in flight
    wait_chunks<NP, NBUF>(min(NBUF - 1, n_chunks - 1 - c));
    __syncthreads();
    const uint16_t* ck = sk + b * kTileN * D;
    const uint16_t* cv = sv + b * kTileN * D;
    floatx4 s[NB];
#pragma unroll
    for (int h = 0; h < NB; ++h) s[h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 a = lds_row8<D>(ck, 16 * wave + col, 32 * ks + 8 * grp);
#pragma unroll
      for (int h = 0; h < NB; ++h) s[h] = T::mfma(a, qf[h][ks], s[h]);
    }
    // lane (grp, col): s[h][i] = score of token t0 + i for q row 16h + col
    const int t0 = g0 + c * kTileN + 16 * wave + 4 * grp;
    uint2 pb[NB];
#pragma unroll
    for (int h = 0; h < NB; ++h) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bool ok = t0 + i < g1;
        if constexpr (!EXACT)   // several query positions: the token rule per row
          ok = ok && elem_tok(g, my_q[h], src.entry(min(t0 + i, g1 - 1)) & kIdxMask);
        s[h][i] = ok ? s[h][i] : kNegInf;
      }
      float mx = fmaxf(fmaxf(s[h][0], s[h][1]), fmaxf(s[h][2], s[h][3]));
      if (__any(mx * g.qk_scale_log2 > m[h] + kDecodeSlack)) {   // unscaled max: Geom::q_and
        mx = wave_max16x4(mx) * g.qk_scale_log2;
        const bool grow = mx > m[h] + kDecodeSlack;
        const float alpha = grow ? __builtin_amdgcn_exp2f(m[h] - mx) : 1.f;
        m[h] = grow ? mx : m[h];
        lsum[h] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[h][dt] *= alpha;
      }
      const float m_use = m[h] == kNegInf ? 0.f : m[h];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        s[h][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[h][i], g.qk_scale_log2, -m_use));
      lsum[h] += (s[h][0] + s[h][1]) + (s[h][2] + s[h][3]);
      pb[h] = make_uint2(pack2<T>(s[h][0], s[h][1]), pack2<T>(s[h][2], s[h][3]));
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint2 a = lds_tr4<D>(cv, 16 * wave, 16 * dt, lane);
#pragma unroll
      for (int h = 0; h < NB; ++h) o[h][dt] = mfma16k<T>(a, pb[h], o[h][dt]);
    }
    __syncthreads();                           // every wave is done with buffer b
    if (c + NBUF < n_chunks) issue(c + NBUF, b);
  }

  // merge the four waves, one column block at a time: lane (grp, col) holds
  // O^T rows 16dt + 4grp + i of q row 16h + col
  const size_t row_stride = D + 2;
  float* part = ws + ((size_t)wgh * n_splits + split) * n_rows * row_stride;
  float* wacc = (float*)sk;                    // [4][16][D] (fits two K buffers)
  float* wml = (float*)sv;                     // [4][16][2]
#pragma unroll
  for (int h = 0; h < NB; ++h) {
    const float lw = wave_sum16x4(lsum[h]);
    __syncthreads();                           // the previous block's readers are done
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) wacc[(wave * 16 + col) * D + 16 * dt + 4 * grp + i] = o[h][dt][i];
    if (grp == 0) {
      wml[(wave * 16 + col) * 2] = m[h];
      wml[(wave * 16 + col) * 2 + 1] = lw;
    }
    __syncthreads();
    const int rows_h = min(16, n_rows - 16 * h);
    for (int idx = tid; idx < rows_h * D; idx += 256) {
      const int rl = idx / D, d = idx - rl * D, r = 16 * h + rl;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * 16 + rl) * 2]);
      const float Mu = M == kNegInf ? 0.f : M;
      float L = 0.f, a = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float sw = __builtin_amdgcn_exp2f(wml[(w * 16 + rl) * 2] - Mu);
        L += wml[(w * 16 + rl) * 2 + 1] * sw;
        a += wacc[(w * 16 + rl) * D + d] * sw;
      }
      if (n_splits == 1) {
        const bool valid = L > 0.f;
        O[qb + (size_t)r * D + d] = T::from_float(valid ? a / L : 0.f);
        if (d == 0) LSE[(size_t)bhq0 * g.n_q + r] = valid ? lse_natural(M, L) : 0.f;
      } else {
        part[r * row_stride + d] = a;
        if (d == 0) {
          part[r * row_stride + D] = M;
          part[r * row_stride + D + 1] = L;
        }
      }
    }
  }
}

// The matrix-core decode serves the group * n_q query rows of a K / V stream
// when they are 2 .. 2 * kDecodeTileM (16-bit, head_dim 64 / 128; one or two
// 16-column blocks), the whole group in one workgroup (one K / V read per
// group); a single row keeps decode_kernel.
inline bool decode_on_mfma(int dtype, int head_dim, const Geom& g) {
  const int rows = g.group * g.n_q;
  return dtype != kF32 && (head_dim == 64 || head_dim == 128) && rows >= 2 &&
         rows <= 2 * kDecodeTileM;
}

template <typename T, int D>
int launch_decode_mfma(const Geom& g, const void* q, const void* k, const void* v, void* o, float* lse,
                       const RingTokens& src, int kv_rows, int n_tokens, float* ws, int n_splits,
                       hipStream_t stream, const char* what) {
  const int n_wgh = g.B * g.H_kv;
  constexpr int lds_q = decode_mfma_lds<D, true>(), lds_r = decode_mfma_lds<D, false>();
  if constexpr (lds_q > 65536 || lds_r > 65536) {
    // above the 64 KB default: opt in once per device and instantiation
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(3, std::string(what) + ": hipGetDevice failed");
    const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
    if (!bit || !(done.load() & bit)) {
      bool ok = true;
#define GKI_MFMA_LDS(EX, NBK, QL, BYTES)                                                            ok = ok && (BYTES <= 65536 || hipFuncSetAttribute((const void*)decode_mfma_kernel<T, D, EX, NBK, QL>,                                                     hipFuncAttributeMaxDynamicSharedMemorySize,                                                           BYTES) == hipSuccess)
      GKI_MFMA_LDS(true, 1, true, lds_q);
      GKI_MFMA_LDS(false, 1, true, lds_q);
      GKI_MFMA_LDS(true, 2, true, lds_q);
      GKI_MFMA_LDS(false, 2, true, lds_q);
      GKI_MFMA_LDS(true, 1, false, lds_r);
      GKI_MFMA_LDS(false, 1, false, lds_r);
      GKI_MFMA_LDS(true, 2, false, lds_r);
      GKI_MFMA_LDS(false, 2, false, lds_r);
#undef GKI_MFMA_LDS
      if (!ok) return fail(3, std::string(what) + ": cannot reserve LDS for the matrix-core decode");
      done.fetch_or(bit);
    }
  }
  const int n_rows = g.group * g.n_q;
  // split streams (short slices) stage their query rows through LDS
#define GKI_MFMA_DECODE(EX, NBK)                                                                   do {                                                                                             if (n_splits > 1)                                                                                hipLaunchKernelGGL((decode_mfma_kernel<T, D, EX, NBK, true>), dim3(n_wgh * n_splits),                            dim3(256), lds_q, stream, g, (const uint16_t*)q, (const uint16_t*)k,                            (const uint16_t*)v, (uint16_t*)o, lse, ws, src, kv_rows, n_tokens,                              n_splits);                                                                else                                                                                             hipLaunchKernelGGL((decode_mfma_kernel<T, D, EX, NBK, false>), dim3(n_wgh * n_splits),                           dim3(256), lds_r, stream, g, (const uint16_t*)q, (const uint16_t*)k,                            (const uint16_t*)v, (uint16_t*)o, lse, ws, src, kv_rows, n_tokens,                              n_splits);                                                              } while (0)
  if (n_rows <= kDecodeTileM) {
    if (g.n_q == 1) GKI_MFMA_DECODE(true, 1);
    else GKI_MFMA_DECODE(false, 1);
  } else {
    if (g.n_q == 1) GKI_MFMA_DECODE(true, 2);
    else GKI_MFMA_DECODE(false, 2);
  }
#undef GKI_MFMA_DECODE
  if (n_splits > 1)
    hipLaunchKernelGGL((combine_kernel<T, D>), dim3(n_wgh * n_rows), dim3(64), 0, stream, ws,
                       (uint16_t*)o, lse, n_rows, n_splits);
  return check_launch(what);
}

// Rolling-cache append: one thread per 16-byte chunk of the rows that survive
// the call. Of the n_new appended positions start .. end-1, only sink positions
// (< sink) and the last `ring` positions >= sink are written: earlier ones would
// be overwritten within the same call, so every slot is written at most once.
// Rows [0, n_a) of the launch are new rows [0, n_a) (sink part), rows
// [n_a, n_a + n_b) are new rows [i_b, i_b + n_b) (ring part).
template <typename T, int D>
__global__ __launch_bounds__(256) void ring_append_kernel(
    typename T::storage* __restrict__ kc, typename T::storage* __restrict__ vc,
    const typename T::storage* __restrict__ kn, const typename T::storage* __restrict__ vn, int BH,
    int n_new, int n_a, int i_b, int n_b, int start, int sink, int ring) {
  using S = typename T::storage;
  constexpr int VEC = 16 / sizeof(S);
  constexpr int CPR = D / VEC;                 // 16-byte chunks per row
  const int rows = n_a + n_b;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)BH * rows * CPR) return;
  const int ch = (int)(idx % CPR);
  const int64_t rr = idx / CPR;
  const int r = (int)(rr % rows);
  const int bh = (int)(rr / rows);
  const int i = r < n_a ? r : i_b + (r - n_a);
  const int p = start + i;
  const int slot = p < sink ? p : sink + (p - sink) % ring;
  const size_t src = ((size_t)bh * n_new + i) * D + ch * VEC;
  const size_t dst = ((size_t)bh * (sink + ring) + slot) * D + ch * VEC;
  *(uint4*)(kc + dst) = *(const uint4*)(kn + src);
  *(uint4*)(vc + dst) = *(const uint4*)(vn + src);
}

template <typename T>
int launch_append_t(int head_dim, void* kc, void* vc, const void* kn, const void* vn, int BH, int n_new,
                    int n_a, int i_b, int n_b, int start, int sink, int ring, hipStream_t stream) {
  using S = typename T::storage;
  constexpr int VEC = 16 / sizeof(S);
  const int64_t total = (int64_t)BH * (n_a + n_b) * (head_dim / VEC);
  if (total == 0) return 0;
  const unsigned grid = (unsigned)((total + 255) / 256);
#define GKI_APPEND_CASE(DD)                                                                       \
  case DD:                                                                                        \
    hipLaunchKernelGGL((ring_append_kernel<T, DD>), dim3(grid), dim3(256), 0, stream, (S*)kc,     \
                       (S*)vc, (const S*)kn, (const S*)vn, BH, n_new, n_a, i_b, n_b, start, sink, \
                       ring);                                                                     \
    break;
  switch (head_dim) {
    GKI_APPEND_CASE(16)
    GKI_APPEND_CASE(32)
    GKI_APPEND_CASE(64)
    GKI_APPEND_CASE(128)
    default: return fail(2, "unsupported head_dim " + std::to_string(head_dim));
  }
#undef GKI_APPEND_CASE
  return check_launch("gki_rolling_append");
}

}  // namespace

int decode_tokens_dispatch(const Geom& g, const int32_t* list, int n_ent, int32_t* tok, int32_t* count,
                           hipStream_t stream) {
  hipLaunchKernelGGL(decode_tokens_kernel, dim3(1), dim3(256), 0, stream, g, list, n_ent, tok, count);
  return check_launch("gki_decode_tokens");
}

int decode_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                    void* o, float* lse, const int32_t* tok, int n_tokens, float* ws,
                    int n_splits, hipStream_t stream) {
  return launch_decode(dtype, head_dim, g, q, k, v, o, lse, ListTokens{tok}, g.n_kv, n_tokens, ws,
                       n_splits, stream, "gki_bsa_decode");
}

// Visible-token stream of the n_q decode rows over a rolling cache of `length`
// positions: sinks [0, min(sink, length)), then the window positions from
// w_lo = max(sink, length - n_q - window + 1) to length - 1.
void ring_stream(int length, int n_q, int sink, int window, int ring, int* n_sink, int* w_lo, int* base,
                 int* n_tokens) {
  *n_sink = length < sink ? length : sink;
  const int lo = length - n_q - window + 1;
  *w_lo = lo > sink ? lo : sink;
  *base = (*w_lo - sink) % ring;
  *n_tokens = *n_sink + (length > *w_lo ? length - *w_lo : 0);
}

int decode_ring_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k,
                         const void* v, void* o, float* lse, int ring, float* ws, int n_splits,
                         hipStream_t stream) {
  RingTokens src;
  int n_tokens;
  ring_stream(g.n_kv, g.n_q, g.sink, g.window, ring, &src.n_sink, &src.w_lo, &src.base, &n_tokens);
  src.sink = g.sink;
  src.ring = ring;
  if (decode_on_mfma(dtype, head_dim, g)) {
    const char* what = "gki_rolling_decode";
    const int rows = g.sink + ring;
    if (dtype == kF16)
      return head_dim == 64
                 ? launch_decode_mfma<F16, 64>(g, q, k, v, o, lse, src, rows, n_tokens, ws, n_splits, stream, what)
                 : launch_decode_mfma<F16, 128>(g, q, k, v, o, lse, src, rows, n_tokens, ws, n_splits, stream, what);
    return head_dim == 64
               ? launch_decode_mfma<BF16, 64>(g, q, k, v, o, lse, src, rows, n_tokens, ws, n_splits, stream, what)
               : launch_decode_mfma<BF16, 128>(g, q, k, v, o, lse, src, rows, n_tokens, ws, n_splits, stream, what);
  }
  return launch_decode(dtype, head_dim, g, q, k, v, o, lse, src, g.sink + ring, n_tokens, ws, n_splits,
                       stream, "gki_rolling_decode");
}

int append_dispatch(int dtype, int head_dim, void* kc, void* vc, const void* kn, const void* vn, int BH,
                    int n_new, int start, int sink, int ring, hipStream_t stream) {
  const int end = start + n_new;
  const int n_a = start < sink ? (end < sink ? end : sink) - start : 0;
  const int keep_lo = end - ring > sink ? end - ring : sink;       // first surviving ring position
  const int b_lo = keep_lo > start ? keep_lo : start;
  const int i_b = b_lo - start;
  const int n_b = end > b_lo ? end - b_lo : 0;
  if (dtype == kF32)
    return launch_append_t<F32>(head_dim, kc, vc, kn, vn, BH, n_new, n_a, i_b, n_b, start, sink, ring, stream);
  if (dtype == kF16)
    return launch_append_t<F16>(head_dim, kc, vc, kn, vn, BH, n_new, n_a, i_b, n_b, start, sink, ring, stream);
  return launch_append_t<BF16>(head_dim, kc, vc, kn, vn, BH, n_new, n_a, i_b, n_b, start, sink, ring, stream);
}

// ---------------------------------------------------------------------------
// Read probe (measurement only): the bytes a single-position StreamingLLM
// decode step reads -- per (b, kv head) slice the sink rows 0 .. n_sink - 1 and
// the window rows w_lo .. n_kv - 1 of K and of V -- streamed with 16-byte
// non-temporal loads and XOR-folded into one word per thread (so no load can be
// dropped), with no other work: the ceiling of that access pattern, timed by
// bench.py beside the decode step. Workgroup (slice, tensor, part): parts
// 0 .. kReadParts - 1 split the window rows into near-equal chunks, the last
// part reads the sink rows; kReadUnroll loads in flight per thread. (Eight
// chunks of 256 threads with four loads each was the fastest of ten layouts
// measured on the c4 rows with the memory-side cache evicted.)
// ---------------------------------------------------------------------------
typedef uint32_t probe_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kReadParts = 8;
constexpr int kReadUnroll = 4;
constexpr int kReadThreads = 256;

__global__ __launch_bounds__(kReadThreads) void read_probe_kernel(
    const probe_u32x4* __restrict__ k, const probe_u32x4* __restrict__ v, int64_t slice16, int64_t sink16,
    int64_t win_lo16, int64_t win16, uint32_t* __restrict__ out) {
  const int part = blockIdx.x % (kReadParts + 1);
  const int t = (blockIdx.x / (kReadParts + 1)) & 1;
  const int64_t s = blockIdx.x / (2 * (kReadParts + 1));
  const probe_u32x4* base = (t ? v : k) + s * slice16;
  int64_t lo = 0, n = sink16;
  if (part < kReadParts) {
    const int64_t c = (win16 + kReadParts - 1) / kReadParts;
    lo = win_lo16 + part * c;
    n = win16 - part * c < c ? win16 - part * c : c;
    n = n > 0 ? n : 0;
  }
  probe_u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t i = threadIdx.x; i < n; i += (int64_t)kReadThreads * kReadUnroll) {
    probe_u32x4 r[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const int64_t j = i + (int64_t)u * kReadThreads;
      r[u] = j < n ? __builtin_nontemporal_load(base + lo + j) : probe_u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= r[u];
  }
  out[(int64_t)blockIdx.x * kReadThreads + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

int64_t read_probe_words(int BH) { return (int64_t)BH * 2 * (kReadParts + 1) * kReadThreads; }

int read_probe_dispatch(const void* k, const void* v, int BH, int64_t n_kv, int row_bytes, int n_sink,
                        int64_t w_lo, uint32_t* out, hipStream_t stream) {
  const int64_t r16 = row_bytes / 16;
  hipLaunchKernelGGL(read_probe_kernel, dim3(BH * 2 * (kReadParts + 1)), dim3(kReadThreads), 0, stream,
                     (const probe_u32x4*)k, (const probe_u32x4*)v, n_kv * r16, (int64_t)n_sink * r16,
                     w_lo * r16, (n_kv - w_lo) * r16, out);
  return check_launch("gki_read_probe");
}

}  // namespace gki
