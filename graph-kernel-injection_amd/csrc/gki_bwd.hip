// Block-sparse StreamingLLM attention: backward kernels for gfx950.
//
// Replaces the reference's three Triton launches in
// `_BlockSparseFlashAttention.backward` (sparse_triton_kernel.py:719-777):
//   * `_bwd_preprocess_kernel` (sparse_triton_kernel.py:354-392),
//       Delta[q] = sum_d fp32(O) * fp32(dO) over the stored O: for 16-bit
//       inputs inside dq_kernel_16, which runs first and stores -Delta for
//       dK/dV; for fp32 inputs delta_kernel, before the other two. For 16-bit
//       inputs the dQ kernel also turns the stored natural LSE into base 2
//       once per row (second half of the row-term workspace), so the 16-bit
//       kernels form P = exp(S scale - LSE) as one exp2 of an fma; the fp32
//       kernels form it as exp2(fma(S, scale, -LSE) log2 e) from the stored
//       LSE, as the fp32 forward computed its exponents.
//   * dkdv_kernel   <- `_bwd_dkdv_kernel` (sparse_triton_kernel.py:394-509):
//       one workgroup per 64-row KV tile, loop over the kept q tiles of its
//       column (CSC list), P = exp(S - LSE), dV += P^T dO,
//       dS = P (dP - Delta) * scale, dK += dS^T Q. No atomics; one store per
//       tile.
//   * dq_kernel     <- `_bwd_dq_kernel` (sparse_triton_kernel.py:511-601):
//       one workgroup per 64-row q tile, loop over its kept kv tiles (CSR),
//       dQ += dS K.
// Casts follow the reference: P^T -> dO dtype for dV, dS -> Q/K dtype for
// dK/dQ, results stored in the input dtype.
//
// MI355X specifics: the dK/dV grid runs a work list in which long column walks
// (the sink column, kept by every q tile; the columns of a large grouped-query
// group) are cut into items of bounded length whose fp32 partials a reduce
// pass sums in a fixed order; items are XCD-remapped so neighbouring tiles of
// one head share L2.
#include "gki_common.cuh"

namespace gki {
namespace {

// ---------------------------------------------------------------------------
// Delta = rowsum(O * dO)
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void delta_kernel(const typename T::storage* __restrict__ O,
                                                    const typename T::storage* __restrict__ dO,
                                                    float* __restrict__ delta, int64_t rows) {
  constexpr int VEC = T::is_f32 ? 4 : 8;
  constexpr int LPR = D / VEC;          // lanes per row (2..32)
  constexpr int RPB = 256 / LPR;        // rows per block
  const int tid = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * RPB + tid / LPR;
  const int ch = tid % LPR;
  float acc = 0.f;
  if (row < rows) {
    const uint4 a = *(const uint4*)(O + row * D + ch * VEC);
    const uint4 b = *(const uint4*)(dO + row * D + ch * VEC);
    if constexpr (T::is_f32) {
      const float* fa = (const float*)&a;
      const float* fb = (const float*)&b;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc += fa[i] * fb[i];
    } else {
      const uint16_t* ha = (const uint16_t*)&a;
      const uint16_t* hb = (const uint16_t*)&b;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += T::to_float(ha[i]) * T::to_float(hb[i]);
    }
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (row < rows && ch == 0) delta[row] = acc;
}

// fp32 gradients accumulate one iteration (64 rows) at a time in a fresh
// accumulator, which is then added to the running sum with its rounding error
// kept exactly (TwoSum) in a compensation term: a long walk (the sink keys of a
// long sequence, |dV| ~ 10 over thousands of rows) then rounds like a short
// one. The result is sum + compensation.
__device__ inline void two_sum_fold(floatx4& sum, floatx4& comp, const floatx4& x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float s = sum[i] + x[i];
    const float bp = s - sum[i];
    const float ap = s - bp;
    comp[i] += (sum[i] - ap) + (x[i] - bp);
    sum[i] = s;
  }
}

template <int D>
struct Stage32 {
  static constexpr int LD = D + 4;
  static constexpr int CPR = D / 4;
  static constexpr int CH = 64 * CPR;
  static constexpr int P = (CH + 255) / 256;
  float4 reg[P];
  __device__ inline void load(const float* base, int r0, int n_rows, int tid) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = tid + 256 * p;
      const int r = c / CPR, ch = c - r * CPR;
      reg[p] = (c < CH && r0 + r < n_rows) ? *(const float4*)(base + (size_t)(r0 + r) * D + ch * 4)
                                           : make_float4(0, 0, 0, 0);
    }
  }
  __device__ inline void store(float* rowmajor, int tid) const {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = tid + 256 * p;
      if (c < CH) {
        const int r = c / CPR, ch = c - r * CPR;
        *(float4*)(&rowmajor[r * LD + ch * 4]) = reg[p];
      }
    }
  }
};

// Work item of workgroup b in the dK / dV grid: the items of one (b, kv head)
// are consecutive, XCD-remapped so that neighbouring kv tiles of a head (which
// share most q tiles) run on one XCD and meet in its L2.
struct KvItem {
  int kt, it0, it1, pslot;
};
__device__ inline KvItem kv_item_of(int b, int BH, const KvWork& w, int& bh) {
  const int wg = xcd_remap(b, w.n_items * BH);
  bh = wg / w.n_items;
  const int4 t = ((const int4*)w.items)[wg - bh * w.n_items];
  return {t.x, t.y, t.z, t.w};
}

// Sum of a split column's fp32 partials, in item order, cast to the storage
// type. A split column's 2 x 64 x D partial floats (dK then dV) are spread
// over D / 8 workgroups, one float4 per thread; the loads of four partials are
// issued together and added in item order (the sum is deterministic).
template <int D>
constexpr int kReduceWgPerTile = 2 * kTileN * D / (256 * 4);

template <typename T, int D>
__global__ __launch_bounds__(256) void dkdv_reduce_kernel(Geom g, KvWork w,
                                                          typename T::storage* __restrict__ dK,
                                                          typename T::storage* __restrict__ dV) {
  constexpr int TILE = kTileN * D;                     // floats of one dK (or dV) tile
  constexpr int STRIDE = 2 * TILE / 4;                 // float4s between two partials
  constexpr int WGT = kReduceWgPerTile<D>;
  const int rest = blockIdx.x / WGT, part = blockIdx.x - rest * WGT;
  const int bh = rest / w.n_split, s = rest - bh * w.n_split;
  const int kt = w.split[3 * s], p0 = w.split[3 * s + 1], np = w.split[3 * s + 2];
  const int idx = (part * 256 + threadIdx.x) * 4;      // first float of this thread
  const float4* src = (const float4*)(w.partials + ((size_t)bh * w.n_pslots + p0) * 2 * TILE + idx);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  int c = 0;
  if constexpr (T::is_f32) {           // compensated (Kahan) sum of the fp32 partials
    float4 comp = make_float4(0.f, 0.f, 0.f, 0.f);
    for (; c < np; ++c) {
      const float4 a = src[(size_t)c * STRIDE];
      const float ya = a.x - comp.x, yb = a.y - comp.y, yc = a.z - comp.z, yd = a.w - comp.w;
      const float ta = acc.x + ya, tb = acc.y + yb, tc = acc.z + yc, td = acc.w + yd;
      comp = make_float4((ta - acc.x) - ya, (tb - acc.y) - yb, (tc - acc.z) - yc, (td - acc.w) - yd);
      acc = make_float4(ta, tb, tc, td);
    }
  }
  for (; c + 4 <= np; c += 4) {
    const float4 a0 = src[(size_t)c * STRIDE], a1 = src[(size_t)(c + 1) * STRIDE];
    const float4 a2 = src[(size_t)(c + 2) * STRIDE], a3 = src[(size_t)(c + 3) * STRIDE];
    acc.x = (((acc.x + a0.x) + a1.x) + a2.x) + a3.x;
    acc.y = (((acc.y + a0.y) + a1.y) + a2.y) + a3.y;
    acc.z = (((acc.z + a0.z) + a1.z) + a2.z) + a3.z;
    acc.w = (((acc.w + a0.w) + a1.w) + a2.w) + a3.w;
  }
  for (; c < np; ++c) {
    const float4 a = src[(size_t)c * STRIDE];
    acc.x += a.x, acc.y += a.y, acc.z += a.z, acc.w += a.w;
  }
  const int which = idx / TILE, rem = idx - which * TILE;   // 4 floats of one row (D % 4 == 0)
  const int row = kt * kTileN + rem / D;
  if (row >= g.n_kv) return;
  typename T::storage* dst = (which ? dV : dK) + (size_t)bh * g.n_kv * D + (size_t)row * D + rem % D;
  dst[0] = T::from_float(acc.x);
  dst[1] = T::from_float(acc.y);
  dst[2] = T::from_float(acc.z);
  dst[3] = T::from_float(acc.w);
}

// ---------------------------------------------------------------------------
// dK / dV, 16-bit. Q and dO tiles row-major in LDS (double-buffered, staged by
// LDS-DMA); the dV += P^T dO and dK += dS^T Q operands dO / Q come from lds_tr8.
// ---------------------------------------------------------------------------
// PRE (Geom::prescale): the scale is already inside the dP accumulator
// (V / dO operands and Delta pre-multiplied by a power-of-two scale, exact),
// so dS = P * acc; otherwise dS = P * (acc * scale). Either way the scaled dS
// is cast, as the reference. A template parameter, so neither form carries a
// branch.
template <typename T, int D, bool PRE>
__global__ __launch_bounds__(256, 2) void dkdv_kernel_16(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO, uint16_t* __restrict__ dK,
    uint16_t* __restrict__ dV, const float* __restrict__ LSE2, const float* __restrict__ Delta,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ col_idx, KvWork w) {
  // LSE2: base-2 LSE rows; Delta: -Delta rows (times the scale when PRE),
  // both written by the dQ kernel, which runs first
  constexpr int KS = (D + 31) / 32;
  constexpr int DT = D / 16;
  using Tile = RowTile<D>;
  __shared__ __align__(16) uint16_t sq[2][64 * D];
  __shared__ __align__(16) uint16_t sdo[2][64 * D];
  __shared__ __align__(16) float slse[2][64];
  __shared__ __align__(16) float sdlt[2][64];

  // one workgroup per (b, kv head, work item): a range of the kv tile's walk
  // over (q head of the group, CSC list entry), accumulated in registers
  const int BH = g.B * g.H_kv;
  int bh;
  const KvItem item = kv_item_of(blockIdx.x, BH, w, bh);
  // an empty column (no kept q tile) only writes zeros: its K / V rows are not read
  const bool has_work = item.it1 > item.it0;
  const int kt = item.kt;
  const size_t kb = (size_t)bh * g.n_kv * D;
  const int bhq0 = (bh / g.H_kv) * g.H + (bh % g.H_kv) * g.group;   // first q head
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int k_w = kt * kTileN + wave * 16;
  const int my_kv = k_w + col;

  uint4 kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = 32 * ks + 8 * grp;
    const bool ok = has_work && my_kv < g.n_kv && d0 < D;
    kf[ks] = ok ? *(const uint4*)(K + kb + (size_t)my_kv * D + d0) : make_uint4(0, 0, 0, 0);
    vf[ks] = ok ? *(const uint4*)(V + kb + (size_t)my_kv * D + d0) : make_uint4(0, 0, 0, 0);
    if constexpr (PRE) vf[ks] = scale8<T>(vf[ks], g.scale);
  }
  floatx4 dk[DT], dv[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dk[i] = dv[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int e_beg = col_ptr[kt], e_end = col_ptr[kt + 1];
  DmaTile<D> dma;
  dma.init(tid);
  // Q / dO tiles: full tiles by LDS-DMA, the ragged last one through registers
  // (rows past n_q zero). LSE / Delta rows by a 4-byte LDS-DMA (waves 0 / 1,
  // one lane per row; rows past n_q re-read row n_q - 1, which only masked
  // elements see).
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto load_tile = [&](int q0, int bhq, int buf) {
    const size_t qb = (size_t)bhq * g.n_q * D;
    if (q0 + kTileM <= g.n_q) {
      dma.load(Q + qb, q0, sq[buf]);
      dma.load(dO + qb, q0, sdo[buf]);
    } else {
      Tile t;
      t.load(Q + qb, q0, g.n_q, tid);
      t.store(sq[buf], tid);
      t.load(dO + qb, q0, g.n_q, tid);
      t.store(sdo[buf], tid);
      dma_wait();   // nothing of this branch pending where it rejoins the DMA path
    }
    if (wave_u < 2) {
      const float* src = (wave_u == 0 ? LSE2 : Delta) + (size_t)bhq * g.n_q + min(q0 + lane, g.n_q - 1);
      dma_load4(src, lds_addr(wave_u == 0 ? slse[buf] : sdlt[buf]));
    }
  };
  // iterations [it0, it1): iteration i visits list entry e_beg + i % L of q
  // head bhq0 + i / L; (e, bhq) advance together
  const int L = e_end - e_beg;
  const int n_it = item.it1 - item.it0;
  const int h0 = L > 0 ? item.it0 / L : 0;
  int e_nx = e_beg + (item.it0 - h0 * L), q_nx = bhq0 + h0;
  if (n_it > 0) load_tile((col_idx[e_nx] & kIdxMask) * kTileM, q_nx, 0);
  dma_wait();
  __syncthreads();

  const int kv_hi_wave = min(k_w + 15, g.n_kv - 1);
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    const int ent = col_idx[e_nx];
    if (++e_nx == e_end) {
      e_nx = e_beg;
      ++q_nx;
    }
    const int q0 = (ent & kIdxMask) * kTileM;
    const bool partial = (ent >> kPartialBit) & 1;
    if (it + 1 < n_it) load_tile((col_idx[e_nx] & kIdxMask) * kTileM, q_nx, buf ^ 1);
    const uint16_t* cq = sq[buf];
    const uint16_t* cdo = sdo[buf];

    const bool need_mask = partial || (q0 + kTileM > g.n_q) || (k_w + 15 >= g.n_kv) ||
                           !tile_all_visible(g, q0, min(q0 + kTileM - 1, g.n_q - 1), k_w, kv_hi_wave);
    // S and dP for the four 16-row q subtiles (rows rho(t, .)); accumulator
    // element i of lane (grp, col) is q row rho(t, 4 grp + i), kv row my_kv
    floatx4 p[4], ds[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // the dP accumulator starts at -Delta of its four q rows (stored negated
      // by the dQ kernel), so it ends as dP - Delta (times the scale when PRE)
      const int qr0 = rho(t, 4 * grp);
      const float4 lse4 = *(const float4*)(&slse[buf][qr0]);
      const float4 ndl4 = *(const float4*)(&sdlt[buf][qr0]);
      floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 dp = floatx4{ndl4.x, ndl4.y, ndl4.z, ndl4.w};
      const int r = rho(t, col);
      mfma_priority_hi<(D <= 64)>();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        const uint4 aq = (d0 < D) ? lds_row8<D>(cq, r, d0) : make_uint4(0, 0, 0, 0);
        const uint4 ad = (d0 < D) ? lds_row8<D>(cdo, r, d0) : make_uint4(0, 0, 0, 0);
        s = T::mfma(aq, kf[ks], s);
        dp = T::mfma(ad, vf[ks], dp);
      }
      mfma_priority_lo<(D <= 64)>();
      const float lv[4] = {lse4.x, lse4.y, lse4.z, lse4.w};          // base-2 LSE
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], g.scale_log2, -lv[i]));
        p[t][i] = pv;
        ds[t][i] = PRE ? pv * dp[i] : pv * (dp[i] * g.scale);
      }
    }
    // Masked elements: P = dS = 0 (a bit select, so an exp that overflowed on
    // an invisible element cannot leak). One uniform branch per tile keeps the
    // selects off the tiles that need no mask.
    if (need_mask) {
      const LaneBits vis(col_valid_bits(g, my_kv, q0, partial), grp);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[t][i] = vis.pick(t, i, p[t][i], 0.f);
          ds[t][i] = vis.pick(t, i, ds[t][i], 0.f);
        }
    }
    mfma_priority_hi<(D <= 64)>();
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint4 ap = pack8<T>(p[2 * st], p[2 * st + 1]);
      const uint4 ad = pack8<T>(ds[2 * st], ds[2 * st + 1]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dv[dt] = T::mfma(ap, lds_tr8<D>(cdo, 32 * st, 16 * dt, lane), dv[dt]);
        dk[dt] = T::mfma(ad, lds_tr8<D>(cq, 32 * st, 16 * dt, lane), dk[dt]);
      }
    }
    mfma_priority_lo<(D <= 64)>();
    dma_wait();        // the next tile's LDS-DMA has landed before the barrier
    __syncthreads();
  }

  // dK/dV accumulators: lane holds rows k_w + 4grp + i, column 16dt + col.
  if (item.pslot >= 0) {             // a split column: fp32 partials for the reduce
    float* pk = w.partials + ((size_t)bh * w.n_pslots + item.pslot) * 2 * (kTileN * D);
    float* pv = pk + kTileN * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wave * 16 + 4 * grp + i;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        pk[r * D + 16 * dt + col] = dk[dt][i];
        pv[r * D + 16 * dt + col] = dv[dt][i];
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = k_w + 4 * grp + i;
    if (row < g.n_kv) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dK[kb + (size_t)row * D + 16 * dt + col] = T::from_float(dk[dt][i]);
        dV[kb + (size_t)row * D + 16 * dt + col] = T::from_float(dv[dt][i]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV, 16-bit, head_dim 64, in quadrants: wave w owns kv rows
// 32 (w & 1) .. +31 of the 64-row kv tile (two 16-row blocks, K / V in
// registers as the B operands) against q rows 32 (w >> 1) .. +31 of each q
// tile (rho subtiles 2 qh, 2 qh + 1). Every Q / dO row read, LSE / Delta read
// and transposed Q / dO read from LDS then feeds the MFMAs of both kv blocks:
// 28 LDS reads per 32 MFMAs per wave and tile instead of 56. The two q
// halves' fp32 dK / dV sums meet once, through LDS, at the end of the item
// (the qh = 0 wave adds the qh = 1 wave's, a fixed order).
// ---------------------------------------------------------------------------
template <typename T, bool PRE>
__global__ __launch_bounds__(256, 3) void dkdv_kernel_q64(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO, uint16_t* __restrict__ dK,
    uint16_t* __restrict__ dV, const float* __restrict__ LSE2, const float* __restrict__ Delta,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ col_idx, KvWork w) {
  // LSE2: base-2 LSE rows; Delta: -Delta rows (times the scale when PRE),
  // both written by the dQ kernel, which runs first
  constexpr int D = 64, KS = 2, DT = 4;
  using Tile = RowTile<D>;
  __shared__ __align__(16) uint16_t sq[2][64 * D];
  __shared__ __align__(16) uint16_t sdo[2][64 * D];
  __shared__ __align__(16) float slse[2][64];
  __shared__ __align__(16) float sdlt[2][64];

  const int BH = g.B * g.H_kv;
  int bh;
  const KvItem item = kv_item_of(blockIdx.x, BH, w, bh);
  // an empty column (no kept q tile) only writes zeros: its K / V rows are not read
  const bool has_work = item.it1 > item.it0;
  const int kt = item.kt;
  const size_t kb = (size_t)bh * g.n_kv * D;
  const int bhq0 = (bh / g.H_kv) * g.H + (bh % g.H_kv) * g.group;   // first q head
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int kh = __builtin_amdgcn_readfirstlane(wave & 1), qh = __builtin_amdgcn_readfirstlane(wave >> 1);
  const int k_w = kt * kTileN + 32 * kh;       // the wave's first kv row

  uint4 kf[2][KS], vf[2][KS];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int my_kv = k_w + 16 * b + col;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 32 * ks + 8 * grp;
      const bool ok = has_work && my_kv < g.n_kv;
      kf[b][ks] = ok ? *(const uint4*)(K + kb + (size_t)my_kv * D + d0) : make_uint4(0, 0, 0, 0);
      vf[b][ks] = ok ? *(const uint4*)(V + kb + (size_t)my_kv * D + d0) : make_uint4(0, 0, 0, 0);
      if constexpr (PRE) vf[b][ks] = scale8<T>(vf[b][ks], g.scale);
    }
  }
  floatx4 dk[2][DT], dv[2][DT];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < DT; ++i) dk[b][i] = dv[b][i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int e_beg = col_ptr[kt], e_end = col_ptr[kt + 1];
  DmaTile<D> dma;
  dma.init(tid);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto load_tile = [&](int q0, int bhq, int buf) {
    const size_t qb = (size_t)bhq * g.n_q * D;
    if (q0 + kTileM <= g.n_q) {
      dma.load(Q + qb, q0, sq[buf]);
      dma.load(dO + qb, q0, sdo[buf]);
    } else {
      Tile t;
      t.load(Q + qb, q0, g.n_q, tid);
      t.store(sq[buf], tid);
      t.load(dO + qb, q0, g.n_q, tid);
      t.store(sdo[buf], tid);
      dma_wait();   // nothing of this branch pending where it rejoins the DMA path
    }
    if (wave_u < 2) {
      const float* src = (wave_u == 0 ? LSE2 : Delta) + (size_t)bhq * g.n_q + min(q0 + lane, g.n_q - 1);
      dma_load4(src, lds_addr(wave_u == 0 ? slse[buf] : sdlt[buf]));
    }
  };
  const int L = e_end - e_beg;
  const int n_it = item.it1 - item.it0;
  const int h0 = L > 0 ? item.it0 / L : 0;
  int e_nx = e_beg + (item.it0 - h0 * L), q_nx = bhq0 + h0;
  if (n_it > 0) load_tile((col_idx[e_nx] & kIdxMask) * kTileM, q_nx, 0);
  dma_wait();
  __syncthreads();

  const int kv_hi_wave = min(k_w + 31, g.n_kv - 1);
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    const int ent = col_idx[e_nx];
    if (++e_nx == e_end) {
      e_nx = e_beg;
      ++q_nx;
    }
    const int q0 = (ent & kIdxMask) * kTileM;
    const bool partial = (ent >> kPartialBit) & 1;
    if (it + 1 < n_it) load_tile((col_idx[e_nx] & kIdxMask) * kTileM, q_nx, buf ^ 1);
    const uint16_t* cq = sq[buf];
    const uint16_t* cdo = sdo[buf];
    const int qw0 = q0 + 32 * qh;              // the wave's first q row
    const bool need_mask = partial || (qw0 + 32 > g.n_q) || (k_w + 31 >= g.n_kv) ||
                           !tile_all_visible(g, qw0, min(qw0 + 31, g.n_q - 1), k_w, kv_hi_wave);
    floatx4 p[2][2], ds[2][2];                 // [subtile 2 qh + u][kv block]
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = 2 * qh + u;
      const int qr0 = rho(t, 4 * grp);
      const float4 lse4 = *(const float4*)(&slse[buf][qr0]);
      const float4 ndl4 = *(const float4*)(&sdlt[buf][qr0]);
      floatx4 sc[2], dp[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        sc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
        dp[b] = floatx4{ndl4.x, ndl4.y, ndl4.z, ndl4.w};
      }
      const int r = rho(t, col);
      mfma_priority_hi<true>();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        const uint4 aq = lds_row8<D>(cq, r, d0);
        const uint4 ad = lds_row8<D>(cdo, r, d0);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          sc[b] = T::mfma(aq, kf[b][ks], sc[b]);
          dp[b] = T::mfma(ad, vf[b][ks], dp[b]);
        }
      }
      mfma_priority_lo<true>();
      const float lv[4] = {lse4.x, lse4.y, lse4.z, lse4.w};
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[b][i], g.scale_log2, -lv[i]));
          p[u][b][i] = pv;
          ds[u][b][i] = PRE ? pv * dp[b][i] : pv * (dp[b][i] * g.scale);
        }
    }
    if (need_mask) {     // masked elements: P = dS = 0 (bit select)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const LaneBits vis(col_valid_bits(g, k_w + 16 * b + col, q0, partial), grp);
        const uint32_t wq = qh ? vis.w[1] : vis.w[0];   // uniform select, not an index
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = __builtin_amdgcn_sbfe((int)wq, 4 * u + i, 1);   // 0 or -1
            p[u][b][i] = __int_as_float(__float_as_int(p[u][b][i]) & m);
            ds[u][b][i] = __int_as_float(__float_as_int(ds[u][b][i]) & m);
          }
      }
    }
    uint4 ap[2], as[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      ap[b] = pack8<T>(p[0][b], p[1][b]);
      as[b] = pack8<T>(ds[0][b], ds[1][b]);
    }
    mfma_priority_hi<true>();
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint4 bo = lds_tr8<D>(cdo, 32 * qh, 16 * dt, lane);
      const uint4 bq = lds_tr8<D>(cq, 32 * qh, 16 * dt, lane);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        dv[b][dt] = T::mfma(ap[b], bo, dv[b][dt]);
        dk[b][dt] = T::mfma(as[b], bq, dk[b][dt]);
      }
    }
    mfma_priority_lo<true>();
    dma_wait();        // the next tile's LDS-DMA has landed before the barrier
    __syncthreads();
  }

  // the q-half sums meet in LDS (the Q / dO buffers are free: every wave passed
  // the loop's last barrier): qh = 1 waves store, qh = 0 waves add theirs first
  floatx4* red = (floatx4*)&sq[0][0] + kh * (4 * DT * 64);
  if (qh == 1) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        red[((2 * b + 0) * DT + dt) * 64 + lane] = dk[b][dt];
        red[((2 * b + 1) * DT + dt) * 64 + lane] = dv[b][dt];
      }
  }
  __syncthreads();
  if (qh == 1) return;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      dk[b][dt] += red[((2 * b + 0) * DT + dt) * 64 + lane];
      dv[b][dt] += red[((2 * b + 1) * DT + dt) * 64 + lane];
    }
  // accumulators: lane holds kv rows k_w + 16 b + 4 grp + i, column 16 dt + col
  if (item.pslot >= 0) {             // a split column: fp32 partials for the reduce
    float* pk = w.partials + ((size_t)bh * w.n_pslots + item.pslot) * 2 * (kTileN * D);
    float* pv = pk + kTileN * D;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 32 * kh + 16 * b + 4 * grp + i;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          pk[r * D + 16 * dt + col] = dk[b][dt][i];
          pv[r * D + 16 * dt + col] = dv[b][dt][i];
        }
      }
    return;
  }
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = k_w + 16 * b + 4 * grp + i;
      if (row < g.n_kv) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dK[kb + (size_t)row * D + 16 * dt + col] = T::from_float(dk[b][dt][i]);
          dV[kb + (size_t)row * D + 16 * dt + col] = T::from_float(dv[b][dt][i]);
        }
      }
    }
}

// ---------------------------------------------------------------------------
// dK / dV, fp32
// ---------------------------------------------------------------------------
template <int D>
struct DkdvSmem32 {
  float q[64 * (D + 4)];
  float dout[64 * (D + 4)];
  float lse[64];
  float dlt[64];
};

// One wave per SIMD from head_dim 64 up: the compensated accumulators, the
// register-staged next tile and the four MFMA chains then fit in VGPRs + AGPRs
// (at two waves per SIMD, head_dim 64 spilled 400 bytes per lane: the c1
// backward took 0.284 against 0.213 ms, a B1 H16 N8192 fp32 backward 2.65
// against 2.0 ms).
template <int D>
__global__ __launch_bounds__(256, D >= 64 ? 1 : 2) void dkdv_kernel_32(
    Geom g, const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, float* __restrict__ dK, float* __restrict__ dV,
    const float* __restrict__ LSE, const float* __restrict__ Delta,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ col_idx, KvWork w) {
  // LSE: the forward's natural LSE; Delta: rowsum(O dO) from delta_kernel
  constexpr int KS = D / 4;
  constexpr int DT = D / 16;
  constexpr int LD = D + 4;
  // the four key subtiles unrolled below head_dim 128; at 128 a rolled loop
  // keeps the kernel in VGPRs + AGPRs (unrolled it spilled 868 bytes per lane)
  constexpr int kSubtileUnroll = D >= 128 ? 1 : 4;
  __shared__ __align__(16) DkdvSmem32<D> sm;
  Stage32<D> sq, sdo;

  // one workgroup per (b, kv head, work item), as in the 16-bit kernel
  const int BH = g.B * g.H_kv;
  int bh;
  const KvItem item = kv_item_of(blockIdx.x, BH, w, bh);
  // an empty column (no kept q tile) only writes zeros: its K / V rows are not read
  const bool has_work = item.it1 > item.it0;
  const int kt = item.kt;
  const size_t kb = (size_t)bh * g.n_kv * D;
  const int bhq0 = (bh / g.H_kv) * g.H + (bh % g.H_kv) * g.group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int k_w = kt * kTileN + wave * 16;
  const int my_kv = k_w + col;

  float kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const bool ok = has_work && my_kv < g.n_kv;
    kf[ks] = ok ? K[kb + (size_t)my_kv * D + 4 * ks + grp] : 0.f;
    vf[ks] = ok ? V[kb + (size_t)my_kv * D + 4 * ks + grp] : 0.f;
  }
  floatx4 dk[DT], dv[DT], ck[DT], cv[DT];   // running sums and their compensation
#pragma unroll
  for (int i = 0; i < DT; ++i) dk[i] = dv[i] = ck[i] = cv[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int e_beg = col_ptr[kt], e_end = col_ptr[kt + 1];
  float lreg = 0.f, dreg = 0.f;
  auto load_tile = [&](int q0, int bhq) {
    const size_t qb = (size_t)bhq * g.n_q * D;
    sq.load(Q + qb, q0, g.n_q, tid);
    sdo.load(dO + qb, q0, g.n_q, tid);
    if (tid < 64) {
      const int r = q0 + tid;
      lreg = r < g.n_q ? LSE[(size_t)bhq * g.n_q + r] : 0.f;
      dreg = r < g.n_q ? Delta[(size_t)bhq * g.n_q + r] : 0.f;
    }
  };
  const int L = e_end - e_beg;
  const int n_it = item.it1 - item.it0;
  const int h0 = L > 0 ? item.it0 / L : 0;
  int e_nx = e_beg + (item.it0 - h0 * L), q_nx = bhq0 + h0;
  if (n_it > 0) load_tile((col_idx[e_nx] & kIdxMask) * kTileM, q_nx);

  const int kv_hi_wave = min(k_w + 15, g.n_kv - 1);
  for (int it = 0; it < n_it; ++it) {
    const int ent = col_idx[e_nx];
    if (++e_nx == e_end) {
      e_nx = e_beg;
      ++q_nx;
    }
    const int q0 = (ent & kIdxMask) * kTileM;
    const bool partial = (ent >> kPartialBit) & 1;
    __syncthreads();
    sq.store(sm.q, tid);
    sdo.store(sm.dout, tid);
    if (tid < 64) {
      sm.lse[tid] = lreg;
      sm.dlt[tid] = dreg;
    }
    __syncthreads();
    if (it + 1 < n_it) load_tile((col_idx[e_nx] & kIdxMask) * kTileM, q_nx);

    const bool need_mask = partial || (q0 + kTileM > g.n_q) || (k_w + 15 >= g.n_kv) ||
                           !tile_all_visible(g, q0, min(q0 + kTileM - 1, g.n_q - 1), k_w, kv_hi_wave);
#pragma unroll kSubtileUnroll
    for (int t = 0; t < 4; ++t) {
      floatx4 fk[DT], fv[DT];          // this subtile's 16 rows, folded in compensated
#pragma unroll
      for (int i = 0; i < DT; ++i) fk[i] = fv[i] = floatx4{0.f, 0.f, 0.f, 0.f};
      const int r = rho(t, col);
      const floatx4 s = mfma_f32_dot<KS>([&](int ks) { return sm.q[r * LD + 4 * ks + grp]; },
                                         [&](int ks) { return kf[ks]; });
      const floatx4 dp = mfma_f32_dot<KS>([&](int ks) { return sm.dout[r * LD + 4 * ks + grp]; },
                                          [&](int ks) { return vf[ks]; });
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qr = rho(t, 4 * grp + i);
        float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], g.scale, -sm.lse[qr]) * kLog2e);
        if (need_mask && !elem_valid(g, q0 + qr, my_kv, partial)) pv = 0.f;
        const float dsv = pv * (dp[i] - sm.dlt[qr]) * g.scale;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          fv[dt] = mfma_f32(pv, sm.dout[qr * LD + 16 * dt + col], fv[dt]);
          fk[dt] = mfma_f32(dsv, sm.q[qr * LD + 16 * dt + col], fk[dt]);
        }
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        two_sum_fold(dk[dt], ck[dt], fk[dt]);
        two_sum_fold(dv[dt], cv[dt], fv[dt]);
      }
    }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dk[dt] += ck[dt];
    dv[dt] += cv[dt];
  }
  if (item.pslot >= 0) {             // a split column: partials for the reduce
    float* pk = w.partials + ((size_t)bh * w.n_pslots + item.pslot) * 2 * (kTileN * D);
    float* pv = pk + kTileN * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wave * 16 + 4 * grp + i;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        pk[r * D + 16 * dt + col] = dk[dt][i];
        pv[r * D + 16 * dt + col] = dv[dt][i];
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = k_w + 4 * grp + i;
    if (row < g.n_kv) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dK[kb + (size_t)row * D + 16 * dt + col] = dk[dt][i];
        dV[kb + (size_t)row * D + 16 * dt + col] = dv[dt][i];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dQ, 16-bit. K and V tiles row-major in LDS (double-buffered, staged by
// LDS-DMA); the
// dQ^T += K^T dS^T operand K^T comes from lds_tr8.
// ---------------------------------------------------------------------------
template <typename T, int D, bool PRE>
__global__ __launch_bounds__(256, 2) void dq_kernel_16(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ O, const uint16_t* __restrict__ dO,
    uint16_t* __restrict__ dQ, const float* __restrict__ LSE, float* __restrict__ Delta,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ row_idx, int n_qt,
    const int32_t* __restrict__ dq_order) {
  constexpr int KS = (D + 31) / 32;
  constexpr int DT = D / 16;
  using Tile = RowTile<D>;
  __shared__ __align__(16) uint16_t sk[2][64 * D];
  __shared__ __align__(16) uint16_t sv[2][64 * D];

  const int n_wg = n_qt * g.B * g.H;
  const int wg = work_of(blockIdx.x, n_wg, dq_order);
  if (wg < 0) return;
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bh) * g.n_kv * D;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int q0 = qt * kTileM + wave * 16;
  const int my_q = q0 + col;

  uint4 qf[KS], df[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = 32 * ks + 8 * grp;
    const bool ok = my_q < g.n_q && d0 < D;
    qf[ks] = ok ? *(const uint4*)(Q + qb + (size_t)my_q * D + d0) : make_uint4(0, 0, 0, 0);
    df[ks] = ok ? *(const uint4*)(dO + qb + (size_t)my_q * D + d0) : make_uint4(0, 0, 0, 0);
  }
  // the stored natural LSE in base 2 (one rounding, once per row)
  const float lse2 = my_q < g.n_q ? lse_base2(LSE[(size_t)bh * g.n_q + my_q]) : 0.f;
  // Delta = rowsum(O * dO) in fp32 over the stored O (the preprocessing pass,
  // sparse_triton_kernel.py:354-392, fused here): the lane already holds its
  // row's dO chunks, the four lane groups of a row are summed across. Every q
  // row has exactly one dQ workgroup, which writes it (and the base-2 LSE)
  // for the dK/dV kernel that runs next.
  float part = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = 32 * ks + 8 * grp;
    if (my_q < g.n_q && d0 < D) {
      const uint4 o4 = *(const uint4*)(O + qb + (size_t)my_q * D + d0);
      const uint16_t* ho = (const uint16_t*)&o4;
      const uint16_t* hd = (const uint16_t*)&df[ks];
#pragma unroll
      for (int i = 0; i < 8; ++i) part += T::to_float(ho[i]) * T::to_float(hd[i]);
    }
  }
  // Stored negated: both kernels start their dP accumulators at -Delta, so
  // they end as dP - Delta. With PRE the dO operand and -Delta carry the
  // (power-of-two) scale, so the accumulators end as (dP - Delta) * scale.
  const float ndlt = PRE ? -wave_sum16x4(part) * g.scale : -wave_sum16x4(part);
  if constexpr (PRE) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) df[ks] = scale8<T>(df[ks], g.scale);
  }
  if (my_q < g.n_q && grp == 0) {
    Delta[(size_t)bh * g.n_q + my_q] = ndlt;
    Delta[(size_t)g.B * g.H * g.n_q + (size_t)bh * g.n_q + my_q] = lse2;
  }

  floatx4 dq[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dq[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  DmaTile<D> dma;
  dma.init(tid);
  // K / V tiles: full tiles by LDS-DMA, the ragged last one through registers
  // (rows past n_kv zero).
  auto stage = [&](int k0, int buf) {
    if (k0 + kTileN <= g.n_kv) {
      dma.load(K + kb, k0, sk[buf]);
      dma.load(V + kb, k0, sv[buf]);
    } else {
      Tile t;
      t.load(K + kb, k0, g.n_kv, tid);
      t.store(sk[buf], tid);
      t.load(V + kb, k0, g.n_kv, tid);
      t.store(sv[buf], tid);
      dma_wait();   // nothing of this branch pending where it rejoins the DMA path
    }
  };
  if (e_beg < e_end) stage((row_idx[e_beg] & kIdxMask) * kTileN, 0);
  dma_wait();
  __syncthreads();
  const int q_hi_wave = min(q0 + 15, g.n_q - 1);
  for (int e = e_beg; e < e_end; ++e) {
    const int buf = (e - e_beg) & 1;
    const int ent = row_idx[e];
    const int k0 = (ent & kIdxMask) * kTileN;
    const bool partial = (ent >> kPartialBit) & 1;
    const bool has_next = e + 1 < e_end;
    if (has_next) stage((row_idx[e + 1] & kIdxMask) * kTileN, buf ^ 1);
    const uint16_t* ck = sk[buf];
    const uint16_t* cv = sv[buf];
    const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                           !tile_all_visible(g, q0, q_hi_wave, k0, k0 + kTileN - 1);
    floatx4 ds[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 dp = floatx4{ndlt, ndlt, ndlt, ndlt};
      const int r = rho(t, col);
      mfma_priority_hi<(D <= 64)>();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        const uint4 ak = (d0 < D) ? lds_row8<D>(ck, r, d0) : make_uint4(0, 0, 0, 0);
        const uint4 av = (d0 < D) ? lds_row8<D>(cv, r, d0) : make_uint4(0, 0, 0, 0);
        s = T::mfma(ak, qf[ks], s);
        dp = T::mfma(av, df[ks], dp);
      }
      mfma_priority_lo<(D <= 64)>();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], g.scale_log2, -lse2));
        ds[t][i] = PRE ? pv * dp[i] : pv * (dp[i] * g.scale);
      }
    }
    if (need_mask) {     // masked elements: dS = 0 (bit select, as in the dK/dV kernel)
      const LaneBits vis(row_valid_bits(g, my_q, k0, partial), grp);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) ds[t][i] = vis.pick(t, i, ds[t][i], 0.f);
    }
    mfma_priority_hi<(D <= 64)>();
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint4 b = pack8<T>(ds[2 * st], ds[2 * st + 1]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dq[dt] = T::mfma(lds_tr8<D>(ck, 32 * st, 16 * dt, lane), b, dq[dt]);
    }
    mfma_priority_lo<(D <= 64)>();
    dma_wait();        // the next tile's LDS-DMA has landed before the barrier
    __syncthreads();
  }
  if (my_q < g.n_q) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint2 w;
      w.x = pack2<T>(dq[dt][0], dq[dt][1]);
      w.y = pack2<T>(dq[dt][2], dq[dt][3]);
      *(uint2*)(dQ + qb + (size_t)my_q * D + 16 * dt + 4 * grp) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// dQ, 16-bit, head_dim 64, in quadrants: wave w owns q rows 32 (w >> 1) ..
// +31 of the 64-row q tile (two 16-row blocks, the MFMAs' B-operand columns)
// against kv rows 32 (w & 1) .. +31 of each kv tile (rho subtiles 2 kh,
// 2 kh + 1). Every K / V row read and every K^T transposed read from LDS then
// feeds the MFMAs of both q blocks: 16 LDS reads per 24 MFMAs per wave and
// tile instead of 32. The two kv halves' fp32 dQ sums meet once, through LDS,
// at the end (the kh = 0 wave adds the kh = 1 wave's, a fixed order).
// ---------------------------------------------------------------------------
template <typename T, bool PRE>
__global__ __launch_bounds__(256, 4) void dq_kernel_q64(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ O, const uint16_t* __restrict__ dO,
    uint16_t* __restrict__ dQ, const float* __restrict__ LSE, float* __restrict__ Delta,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ row_idx, int n_qt,
    const int32_t* __restrict__ dq_order) {
  constexpr int D = 64, KS = 2, DT = 4;
  using Tile = RowTile<D>;
  __shared__ __align__(16) uint16_t sk[2][64 * D];
  __shared__ __align__(16) uint16_t sv[2][64 * D];

  const int n_wg = n_qt * g.B * g.H;
  const int wg = work_of(blockIdx.x, n_wg, dq_order);
  if (wg < 0) return;
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bh) * g.n_kv * D;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int qh = __builtin_amdgcn_readfirstlane(wave >> 1), kh = __builtin_amdgcn_readfirstlane(wave & 1);
  const int q0w = qt * kTileM + 32 * qh;       // the wave's first q row

  uint4 qf[2][KS], df[2][KS];
  float lse2[2], ndlt[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int my_q = q0w + 16 * b + col;
    const bool ok = my_q < g.n_q;
    float part = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 32 * ks + 8 * grp;
      qf[b][ks] = ok ? *(const uint4*)(Q + qb + (size_t)my_q * D + d0) : make_uint4(0, 0, 0, 0);
      df[b][ks] = ok ? *(const uint4*)(dO + qb + (size_t)my_q * D + d0) : make_uint4(0, 0, 0, 0);
      // Delta = rowsum(O * dO) over the stored O (sparse_triton_kernel.py:354-392)
      if (ok) {
        const uint4 o4 = *(const uint4*)(O + qb + (size_t)my_q * D + d0);
        const uint16_t* ho = (const uint16_t*)&o4;
        const uint16_t* hd = (const uint16_t*)&df[b][ks];
#pragma unroll
        for (int i = 0; i < 8; ++i) part += T::to_float(ho[i]) * T::to_float(hd[i]);
      }
    }
    lse2[b] = ok ? lse_base2(LSE[(size_t)bh * g.n_q + my_q]) : 0.f;
    // stored negated (and scaled with PRE), as in dq_kernel_16
    ndlt[b] = PRE ? -wave_sum16x4(part) * g.scale : -wave_sum16x4(part);
    if constexpr (PRE) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) df[b][ks] = scale8<T>(df[b][ks], g.scale);
    }
    if (ok && grp == 0 && kh == 0) {     // the two kv-half waves hold the same rows
      Delta[(size_t)bh * g.n_q + my_q] = ndlt[b];
      Delta[(size_t)g.B * g.H * g.n_q + (size_t)bh * g.n_q + my_q] = lse2[b];
    }
  }

  floatx4 dq[2][DT];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < DT; ++i) dq[b][i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  DmaTile<D> dma;
  dma.init(tid);
  auto stage = [&](int k0, int buf) {
    if (k0 + kTileN <= g.n_kv) {
      dma.load(K + kb, k0, sk[buf]);
      dma.load(V + kb, k0, sv[buf]);
    } else {
      Tile t;
      t.load(K + kb, k0, g.n_kv, tid);
      t.store(sk[buf], tid);
      t.load(V + kb, k0, g.n_kv, tid);
      t.store(sv[buf], tid);
      dma_wait();   // nothing of this branch pending where it rejoins the DMA path
    }
  };
  if (e_beg < e_end) stage((row_idx[e_beg] & kIdxMask) * kTileN, 0);
  dma_wait();
  __syncthreads();
  const int q_hi_wave = min(q0w + 31, g.n_q - 1);
  for (int e = e_beg; e < e_end; ++e) {
    const int buf = (e - e_beg) & 1;
    const int ent = row_idx[e];
    const int k0 = (ent & kIdxMask) * kTileN;
    const bool partial = (ent >> kPartialBit) & 1;
    if (e + 1 < e_end) stage((row_idx[e + 1] & kIdxMask) * kTileN, buf ^ 1);
    const uint16_t* ck = sk[buf];
    const uint16_t* cv = sv[buf];
    const int kw0 = k0 + 32 * kh;              // the wave's first kv row
    const bool need_mask = partial || (q0w + 31 >= g.n_q) || (kw0 + 32 > g.n_kv) ||
                           !tile_all_visible(g, q0w, q_hi_wave, kw0, kw0 + 31);
    floatx4 ds[2][2];                          // [subtile 2 kh + u][q block]
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r = rho(2 * kh + u, col);
      floatx4 sc[2], dp[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        sc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
        dp[b] = floatx4{ndlt[b], ndlt[b], ndlt[b], ndlt[b]};
      }
      mfma_priority_hi<true>();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        const uint4 ak = lds_row8<D>(ck, r, d0);
        const uint4 av = lds_row8<D>(cv, r, d0);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          sc[b] = T::mfma(ak, qf[b][ks], sc[b]);
          dp[b] = T::mfma(av, df[b][ks], dp[b]);
        }
      }
      mfma_priority_lo<true>();
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[b][i], g.scale_log2, -lse2[b]));
          ds[u][b][i] = PRE ? pv * dp[b][i] : pv * (dp[b][i] * g.scale);
        }
    }
    if (need_mask) {     // masked elements: dS = 0 (bit select)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const LaneBits vis(row_valid_bits(g, q0w + 16 * b + col, k0, partial), grp);
        // the word of subtiles 2 kh, 2 kh + 1, chosen by a uniform select (an
        // index by kh would put the pair in scratch)
        const uint32_t wk = kh ? vis.w[1] : vis.w[0];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = __builtin_amdgcn_sbfe((int)wk, 4 * u + i, 1);   // 0 or -1
            ds[u][b][i] = __int_as_float(__float_as_int(ds[u][b][i]) & m);
          }
      }
    }
    uint4 pb[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) pb[b] = pack8<T>(ds[0][b], ds[1][b]);
    mfma_priority_hi<true>();
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint4 a = lds_tr8<D>(ck, 32 * kh, 16 * dt, lane);
#pragma unroll
      for (int b = 0; b < 2; ++b) dq[b][dt] = T::mfma(a, pb[b], dq[b][dt]);
    }
    mfma_priority_lo<true>();
    dma_wait();        // the next tile's LDS-DMA has landed before the barrier
    __syncthreads();
  }
  // the kv-half sums meet in LDS (the K buffers are free: every wave passed the
  // loop's last barrier): kh = 1 waves store, kh = 0 waves add theirs first.
  // Row offsets from the lane index afresh (mbcnt: not provably the one
  // above), not the prologue's held (spilled) across the loop.
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int grp_e = lane_e >> 4, col_e = lane_e & 15;
  floatx4* red = (floatx4*)&sk[0][0] + qh * (2 * DT * 64);
  if (kh == 1) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) red[(b * DT + dt) * 64 + lane_e] = dq[b][dt];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int my_q = q0w + 16 * b + col_e;
    if (my_q >= g.n_q) continue;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const floatx4 o = red[(b * DT + dt) * 64 + lane_e];
      uint2 w;
      w.x = pack2<T>(dq[b][dt][0] + o[0], dq[b][dt][1] + o[1]);
      w.y = pack2<T>(dq[b][dt][2] + o[2], dq[b][dt][3] + o[3]);
      *(uint2*)(dQ + qb + (size_t)my_q * D + 16 * dt + 4 * grp_e) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// dQ, fp32
// ---------------------------------------------------------------------------
template <int D>
struct DqSmem32 {
  float k[64 * (D + 4)];
  float v[64 * (D + 4)];
};

// One wave per SIMD at head_dim 128 (two spilled 764 bytes per lane). At 64
// two waves win on full grids (B1 H16 N8192 fp32 backward 2.33 -> 1.99 ms
// against one wave; equal on c1).
template <int D>
__global__ __launch_bounds__(256, D >= 128 ? 1 : 2) void dq_kernel_32(
    Geom g, const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, float* __restrict__ dQ, const float* __restrict__ LSE,
    const float* __restrict__ Delta, const int32_t* __restrict__ row_ptr,
    const int32_t* __restrict__ row_idx, int n_qt, const int32_t* __restrict__ dq_order) {
  constexpr int KS = D / 4;
  constexpr int DT = D / 16;
  constexpr int LD = D + 4;
  // the four key subtiles in a rolled loop at head_dim 64: two waves per SIMD
  // then fit without scratch (209 VGPRs; unrolled, 36 bytes spilled per lane)
  constexpr int kSubtileUnroll = D == 64 ? 1 : 4;
  __shared__ __align__(16) DqSmem32<D> sm;
  Stage32<D> sk, sv;

  const int n_wg = n_qt * g.B * g.H;
  const int wg = work_of(blockIdx.x, n_wg, dq_order);
  if (wg < 0) return;
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bh) * g.n_kv * D;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int q0 = qt * kTileM + wave * 16;
  const int my_q = q0 + col;

  float qf[KS], df[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const bool ok = my_q < g.n_q;
    qf[ks] = ok ? Q[qb + (size_t)my_q * D + 4 * ks + grp] : 0.f;
    df[ks] = ok ? dO[qb + (size_t)my_q * D + 4 * ks + grp] : 0.f;
  }
  const float lse = my_q < g.n_q ? LSE[(size_t)bh * g.n_q + my_q] : 0.f;   // natural
  const float dlt = my_q < g.n_q ? Delta[(size_t)bh * g.n_q + my_q] : 0.f;
  floatx4 dq[DT], cq[DT];              // running sum and its compensation (two_sum_fold)
#pragma unroll
  for (int i = 0; i < DT; ++i) dq[i] = cq[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  if (e_beg < e_end) {
    const int k0 = (row_idx[e_beg] & kIdxMask) * kTileN;
    sk.load(K + kb, k0, g.n_kv, tid);
    sv.load(V + kb, k0, g.n_kv, tid);
  }
  const int q_hi_wave = min(q0 + 15, g.n_q - 1);
  for (int e = e_beg; e < e_end; ++e) {
    const int ent = row_idx[e];
    const int k0 = (ent & kIdxMask) * kTileN;
    const bool partial = (ent >> kPartialBit) & 1;
    __syncthreads();
    sk.store(sm.k, tid);
    sv.store(sm.v, tid);
    __syncthreads();
    if (e + 1 < e_end) {
      const int k1 = (row_idx[e + 1] & kIdxMask) * kTileN;
      sk.load(K + kb, k1, g.n_kv, tid);
      sv.load(V + kb, k1, g.n_kv, tid);
    }
    const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                           !tile_all_visible(g, q0, q_hi_wave, k0, k0 + kTileN - 1);
#pragma unroll kSubtileUnroll
    for (int t = 0; t < 4; ++t) {
      floatx4 fq[DT];                  // this subtile's 16 keys, folded in compensated
#pragma unroll
      for (int i = 0; i < DT; ++i) fq[i] = floatx4{0.f, 0.f, 0.f, 0.f};
      const int r = rho(t, col);
      const floatx4 s = mfma_f32_dot<KS>([&](int ks) { return sm.k[r * LD + 4 * ks + grp]; },
                                         [&](int ks) { return qf[ks]; });
      const floatx4 dp = mfma_f32_dot<KS>([&](int ks) { return sm.v[r * LD + 4 * ks + grp]; },
                                          [&](int ks) { return df[ks]; });
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kr = rho(t, 4 * grp + i);
        float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], g.scale, -lse) * kLog2e);
        if (need_mask && !elem_valid(g, my_q, k0 + kr, partial)) pv = 0.f;
        const float dsv = pv * (dp[i] - dlt) * g.scale;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) fq[dt] = mfma_f32(sm.k[kr * LD + 16 * dt + col], dsv, fq[dt]);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) two_sum_fold(dq[dt], cq[dt], fq[dt]);
    }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dq[dt] += cq[dt];
  if (my_q < g.n_q) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      float4 w = make_float4(dq[dt][0], dq[dt][1], dq[dt][2], dq[dt][3]);
      *(float4*)(dQ + qb + (size_t)my_q * D + 16 * dt + 4 * grp) = w;
    }
  }
}

template <typename T, int D>
void launch_delta(const void* o, const void* dout, float* delta, int64_t rows, hipStream_t stream) {
  constexpr int VEC = T::is_f32 ? 4 : 8;
  constexpr int RPB = 256 / (D / VEC);
  const int64_t grid = (rows + RPB - 1) / RPB;
  hipLaunchKernelGGL((delta_kernel<T, D>), dim3((unsigned)grid), dim3(256), 0, stream,
                     (const typename T::storage*)o, (const typename T::storage*)dout, delta, rows);
}

// dQ first: it also produces -Delta and the base-2 LSE rows, which dK/dV reads
// from the two halves of the row-term workspace
template <typename T, int D, bool PRE>
void launch_bwd16_as(const Geom& g, const void* q, const void* k, const void* v, const void* o,
                     const void* dout, const float* lse, void* dq, void* dk, void* dv, float* delta,
                     const int32_t* row_ptr, const int32_t* row_idx, int n_qt, const int32_t* dq_order,
                     const int32_t* col_ptr, const int32_t* col_idx, const KvWork& w, hipStream_t stream) {
  const int BH = g.B * g.H, BHkv = g.B * g.H_kv;
  const float* lse2 = delta + (size_t)BH * g.n_q;
  if constexpr (D == 64)
    hipLaunchKernelGGL((dq_kernel_q64<T, PRE>), dim3(n_qt * BH), dim3(256), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)o,
                       (const uint16_t*)dout, (uint16_t*)dq, lse, delta, row_ptr, row_idx, n_qt, dq_order);
  else
    hipLaunchKernelGGL((dq_kernel_16<T, D, PRE>), dim3(n_qt * BH), dim3(256), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)o,
                       (const uint16_t*)dout, (uint16_t*)dq, lse, delta, row_ptr, row_idx, n_qt, dq_order);
  if constexpr (D == 64)
    hipLaunchKernelGGL((dkdv_kernel_q64<T, PRE>), dim3(w.n_items * BHkv), dim3(256), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)dout,
                       (uint16_t*)dk, (uint16_t*)dv, lse2, delta, col_ptr, col_idx, w);
  else
    hipLaunchKernelGGL((dkdv_kernel_16<T, D, PRE>), dim3(w.n_items * BHkv), dim3(256), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)dout,
                       (uint16_t*)dk, (uint16_t*)dv, lse2, delta, col_ptr, col_idx, w);
}

template <typename T, int D>
void launch_bwd16(const Geom& g, const void* q, const void* k, const void* v, const void* o,
                  const void* dout, const float* lse, void* dq, void* dk, void* dv, float* delta,
                  const int32_t* row_ptr, const int32_t* row_idx, int n_qt, const int32_t* dq_order,
                  const int32_t* col_ptr, const int32_t* col_idx, const KvWork& w, hipStream_t stream) {
  if (g.prescale)
    launch_bwd16_as<T, D, true>(g, q, k, v, o, dout, lse, dq, dk, dv, delta, row_ptr, row_idx, n_qt,
                                dq_order, col_ptr, col_idx, w, stream);
  else
    launch_bwd16_as<T, D, false>(g, q, k, v, o, dout, lse, dq, dk, dv, delta, row_ptr, row_idx, n_qt,
                                 dq_order, col_ptr, col_idx, w, stream);
}

template <int D>
int launch_bwd(int dtype, const Geom& g, const void* q, const void* k, const void* v, const void* o,
               const void* dout, const float* lse, void* dq, void* dk, void* dv, float* delta,
               const int32_t* row_ptr, const int32_t* row_idx, int n_qt, const int32_t* dq_order,
               const int32_t* col_ptr, const int32_t* col_idx, const KvWork& w, hipStream_t stream) {
  const int BH = g.B * g.H, BHkv = g.B * g.H_kv;
  const int64_t rows = (int64_t)BH * g.n_q;
  const dim3 kv_grid(w.n_items * BHkv), red_grid(w.n_split * BHkv * kReduceWgPerTile<D>);
  if (dtype == kF32) {
    launch_delta<F32, D>(o, dout, delta, rows, stream);
    hipLaunchKernelGGL(dkdv_kernel_32<D>, kv_grid, dim3(256), 0, stream, g, (const float*)q,
                       (const float*)k, (const float*)v, (const float*)dout, (float*)dk, (float*)dv,
                       lse, delta, col_ptr, col_idx, w);
    if (w.n_split > 0)
      hipLaunchKernelGGL((dkdv_reduce_kernel<F32, D>), red_grid, dim3(256), 0, stream, g, w,
                         (float*)dk, (float*)dv);
    hipLaunchKernelGGL(dq_kernel_32<D>, dim3(n_qt * BH), dim3(256), 0, stream, g, (const float*)q,
                       (const float*)k, (const float*)v, (const float*)dout, (float*)dq, lse, delta,
                       row_ptr, row_idx, n_qt, dq_order);
  } else if (dtype == kF16) {
    launch_bwd16<F16, D>(g, q, k, v, o, dout, lse, dq, dk, dv, delta, row_ptr, row_idx, n_qt,
                         dq_order, col_ptr, col_idx, w, stream);
    if (w.n_split > 0)
      hipLaunchKernelGGL((dkdv_reduce_kernel<F16, D>), red_grid, dim3(256), 0, stream, g, w,
                         (uint16_t*)dk, (uint16_t*)dv);
  } else {
    launch_bwd16<BF16, D>(g, q, k, v, o, dout, lse, dq, dk, dv, delta, row_ptr, row_idx, n_qt,
                          dq_order, col_ptr, col_idx, w, stream);
    if (w.n_split > 0)
      hipLaunchKernelGGL((dkdv_reduce_kernel<BF16, D>), red_grid, dim3(256), 0, stream, g, w,
                         (uint16_t*)dk, (uint16_t*)dv);
  }
  return check_launch("gki_bsa_bwd");
}

}  // namespace

int bwd_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                 const void* o, const void* dout, const float* lse, void* dq, void* dk, void* dv,
                 float* delta, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
                 const int32_t* dq_order, const int32_t* col_ptr, const int32_t* col_idx, const KvWork& w,
                 hipStream_t stream) {
#define GKI_BWD_CASE(DD)                                                                          \
  case DD:                                                                                        \
    return launch_bwd<DD>(dtype, g, q, k, v, o, dout, lse, dq, dk, dv, delta, row_ptr, row_idx,   \
                          n_qt, dq_order, col_ptr, col_idx, w, stream);
  switch (head_dim) {
    GKI_BWD_CASE(16)
    GKI_BWD_CASE(32)
    GKI_BWD_CASE(64)
    GKI_BWD_CASE(128)
    default: return fail(2, "unsupported head_dim " + std::to_string(head_dim));
  }
#undef GKI_BWD_CASE
}

}  // namespace gki
