// Block-sparse StreamingLLM attention: prefill forward kernel for gfx950.
//
// Replaces the reference's Triton `_fwd_kernel` (sparse_triton_kernel.py:231-352)
// and its launch (sparse_triton_kernel.py:662-682). Semantics follow the
// reference: S = (Q K^T) * scale in fp32, token mask (causal & (sink | window))
// inside visited tiles, online softmax, P cast to V's dtype before P V,
// O = acc / l, LSE = m + log(l) with the (O = 0, LSE = 0) sentinel for rows that
// saw no key (sparse_triton_kernel.py:341-352). The running max m and sum l
// are kept in base 2 (scores times log2 e, for v_exp_f32); the stored LSE is
// the natural m + ln(l) of the reference, converted once per row.
//
// 16-bit design (one workgroup = 4 waves = one 128-row q tile; wave w owns rows
// 32w .. 32w+31 as two 16-row blocks h = 0, 1):
//  * S^T = K Q^T on v_mfma_f32_16x16x32_{bf16,f16}. In the accumulator layout
//    lane (g, c) holds q row c of its block, so the running max / sum are
//    per-lane scalars; row reductions need two cross-group shuffles.
//  * Every K / V^T operand read from LDS feeds the MFMAs of both row blocks:
//    LDS traffic per flop is half that of 16 rows per wave.
//  * K tile rows are fetched through the rho() permutation, which makes the S^T
//    accumulators of subtiles (2s, 2s+1) the B operand of O^T += V^T P^T as-is;
//    V^T operands come from the gfx950 LDS transpose read (ds_read_b64_tr_b16).
//  * K and V tiles are staged row-major (XOR-swizzled chunks, conflict-free for
//    both read patterns) with coalesced 16-byte loads, double-buffered: one
//    barrier per tile, the next tile's global loads in flight during the MFMAs.
//  * Only kept tiles are visited (GPU-resident CSR list); the O^T rescale is
//    skipped, exactly, when no row max of a block moved.
//  * The running max is kept on unscaled scores, so Q is read through the
//    Geom::q_and / q_xor transform that makes the effective scale positive.
// The fp32 path uses v_mfma_f32_16x16x4f32 on 64-row tiles (16 rows per wave).
#include "gki_common.cuh"

namespace gki {
namespace {

// Online-softmax reference max moves only when a tile's row max exceeds it by
// more than this many log2 units, so p = exp2(s - m) stays below 2^8 and the O
// rescale is almost never needed. O = acc / l and LSE = m + ln(l) are exact for
// any reference max.
constexpr float kRescaleSlack = 8.f;
// Reference max of a row before it has seen a visible key: the most negative
// finite float, so exp2(s * c - m) needs no guard (a masked score gives
// exp2(-inf) = 0) and any visible score, whose scaled value is finite and
// larger, replaces it at the first rescale test.
constexpr float kNoMax = -3.40282347e38f;

// Rows per wave: kFwdRB 16-row blocks, every K / V^T operand read feeding
// kFwdRB MFMAs; 8 / kFwdRB waves per 128-row workgroup. One block per wave
// (eight waves, twice the waves per SIMD at head_dim 128) was 10% slower: the
// doubled LDS reads per MFMA cost more than the occupancy gained.
constexpr int kFwdRB = 2;
constexpr int kFwdThreads = 64 * (8 / kFwdRB);
// Workgroups per CU the compiler must fit in registers: 4 (up to 128 VGPRs) for
// head_dim <= 64, whose 32 KB of K / V buffers allow four workgroups per CU (the
// extra waves hide more latency: 4-7% faster than three at head_dim 64); 2 for
// head_dim 128 (64 KB of buffers).
template <typename T, int D>
__global__ __launch_bounds__(kFwdThreads, D <= 64 ? 4 : 2) void fwd_kernel_16(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ LSE,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ row_idx, int n_qt,
    const int32_t* __restrict__ wg_order) {
  constexpr int KS = (D + 31) / 32;   // k-steps of the QK^T contraction
  constexpr int DT = D / 16;          // 16-row tiles of O^T
  constexpr int RB = kFwdRB;
  constexpr int NW = 8 / RB;          // waves per workgroup
  constexpr int NT = 64 * NW;
  __shared__ __align__(16) uint16_t sk[2][kTileN * D];
  __shared__ __align__(16) uint16_t sv[2][kTileN * D];

  const int n_wg = n_qt * g.B * g.H;
  const int wg = work_of(blockIdx.x, n_wg, wg_order);
  if (wg < 0) return;
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bh) * g.n_kv * D;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int qw = qt * kTileMF + wave * 16 * RB;   // first row of this wave

  uint4 qf[RB][KS];
#pragma unroll
  for (int h = 0; h < RB; ++h) {
    const int q = qw + 16 * h + col;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 32 * ks + 8 * grp;
      qf[h][ks] = (q < g.n_q && d0 < D) ? q_words(g, *(const uint4*)(Q + qb + (size_t)q * D + d0))
                                        : make_uint4(0, 0, 0, 0);
    }
  }

  floatx4 o[RB][DT];
  // Row sums run on the MFMA pipe (ones x P^T): lane (g, c) holds the sum of
  // row c in every component; it sums the same 16-bit P that multiplies V.
  floatx4 lsum[RB];
  // m: the row's reference max (scaled, log2 units); thr: the unscaled score
  // above which it must move, (m + slack) / c, so the per-tile test is one
  // compare (qk_scale_log2 = c > 0)
  float m[RB], thr[RB];
  const float inv_c = __builtin_amdgcn_rcpf(g.qk_scale_log2);   // a trigger: approximate is fine
#pragma unroll
  for (int h = 0; h < RB; ++h) {
#pragma unroll
    for (int i = 0; i < DT; ++i) o[h][i] = floatx4{0.f, 0.f, 0.f, 0.f};
    lsum[h] = floatx4{0.f, 0.f, 0.f, 0.f};
    m[h] = kNoMax;
    thr[h] = (kNoMax + kRescaleSlack) * inv_c;
  }
  const uint4 ones = T::ones8();

  DmaTile<D, NW> dma;
  dma.init(tid);
  // Full tiles go LDS-DMA; the ragged last kv tile goes through registers so
  // that its out-of-range rows are zero (P = 0 must not meet stale V).
  auto stage = [&](int k0, int b) {
    if (k0 + kTileN <= g.n_kv) {
      dma.load(K + kb, k0, sk[b]);
      dma.load(V + kb, k0, sv[b]);
    } else {
      RowTile<D, NT> t;
      t.load(K + kb, k0, g.n_kv, tid);
      t.store(sk[b], tid);
      t.load(V + kb, k0, g.n_kv, tid);
      t.store(sv[b], tid);
      // Unconditional, so that no register load of this branch is pending
      // where it rejoins the DMA path: otherwise the compiler waits for all
      // vector memory there, the just-issued DMA of the next tile included.
      dma_wait();
    }
  };

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  if (e_beg < e_end) stage((row_idx[e_beg] & kIdxMask) * kTileN, 0);
  dma_wait();
  __syncthreads();

  for (int e = e_beg; e < e_end; ++e) {
    const int buf = (e - e_beg) & 1;
    const int ent = row_idx[e];
    const int k0 = (ent & kIdxMask) * kTileN;
    const bool partial = (ent >> kPartialBit) & 1;
    if (e + 1 < e_end) stage((row_idx[e + 1] & kIdxMask) * kTileN, buf ^ 1);
    const uint16_t* ck = sk[buf];
    const uint16_t* cv = sv[buf];

    floatx4 s[RB][4];
    mfma_priority_hi<(D <= 64)>();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int h = 0; h < RB; ++h) s[h][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      const int r = rho(t, col);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        const uint4 a = (d0 < D) ? lds_row8<D>(ck, r, d0) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int h = 0; h < RB; ++h) s[h][t] = T::mfma(a, qf[h][ks], s[h][t]);
      }
    }

    mfma_priority_lo<(D <= 64)>();
#pragma unroll
    for (int h = 0; h < RB; ++h) {
      const int q0 = qw + 16 * h;
      const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                             !tile_all_visible(g, q0, min(q0 + 15, g.n_q - 1), k0, k0 + kTileN - 1);
      if (need_mask) {
        const LaneBits vis(row_valid_bits(g, q0 + col, k0, partial), grp);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) s[h][t][i] = vis.pick(t, i, s[h][t][i], kNegInf);
      }
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[h][t][i]);
      // A row's max exceeds the reference by the slack only if one of its
      // lanes' maxima does (qk_scale_log2 > 0, so scaling after the max is
      // exact): the cross-lane reduction runs only then. The threshold is a
      // trigger only: whether m moves is decided exactly inside.
      if (__any(mx > thr[h])) {
        mx = wave_max16x4(mx) * g.qk_scale_log2;
        const bool grow = mx > m[h] + kRescaleSlack;
        const float alpha = grow ? __builtin_amdgcn_exp2f(m[h] - mx) : 1.f;
        m[h] = grow ? mx : m[h];
        thr[h] = (m[h] + kRescaleSlack) * inv_c;
        lsum[h][0] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[h][dt] *= alpha;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[h][t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[h][t][i], g.qk_scale_log2, -m[h]));
    }

    mfma_priority_hi<(D <= 64)>();
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      uint4 b[RB];
#pragma unroll
      for (int h = 0; h < RB; ++h) b[h] = pack8<T>(s[h][2 * st], s[h][2 * st + 1]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint4 a = lds_tr8<D>(cv, 32 * st, 16 * dt, lane);
#pragma unroll
        for (int h = 0; h < RB; ++h) o[h][dt] = T::mfma(a, b[h], o[h][dt]);
      }
#pragma unroll
      for (int h = 0; h < RB; ++h) lsum[h] = T::mfma(ones, b[h], lsum[h]);
    }
    mfma_priority_lo<(D <= 64)>();
    dma_wait();        // the next tile's LDS-DMA has landed before the barrier
    __syncthreads();
  }

#pragma unroll
  for (int h = 0; h < RB; ++h) {
    const int my_q = qw + 16 * h + col;
    const float l_tot = lsum[h][0];
    const bool valid = l_tot > 0.f;
    const float inv = valid ? 1.f / l_tot : 1.f;
    if (my_q < g.n_q) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 w;
        w.x = pack2<T>(o[h][dt][0] * inv, o[h][dt][1] * inv);
        w.y = pack2<T>(o[h][dt][2] * inv, o[h][dt][3] * inv);
        *(uint2*)(O + qb + (size_t)my_q * D + 16 * dt + 4 * grp) = w;
      }
      if (grp == 0) LSE[(size_t)bh * g.n_q + my_q] = valid ? lse_natural(m[h], l_tot) : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 path (v_mfma_f32_16x16x4f32, 64-row tiles): K and V stay row-major in LDS.
// The softmax runs in natural units: the running max m is that of the scaled
// scores S * scale and each exponent is exp2(fma(S, scale, -m) * log2 e), so
// the scale is applied exactly and only the (small) difference is rounded;
// the backward forms P = exp(S * scale - LSE) the same way from the stored
// LSE = m + ln(l), which therefore matches these scores to within its own
// rounding.
// ---------------------------------------------------------------------------
template <int D>
struct FwdSmem32 {
  static constexpr int LD = D + 4;
  float k[kTileN * LD];
  float v[kTileN * LD];
};

template <int D>
__global__ __launch_bounds__(256, 2) void fwd_kernel_32(
    Geom g, const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ LSE, const int32_t* __restrict__ row_ptr,
    const int32_t* __restrict__ row_idx, int n_qt, const int32_t* __restrict__ wg_order) {
  constexpr int KS = D / 4;
  constexpr int DT = D / 16;
  constexpr int CPR = D / 4;           // 16-byte chunks per row
  constexpr int CH = kTileN * CPR;
  constexpr int P = (CH + 255) / 256;
  using Smem = FwdSmem32<D>;
  __shared__ __align__(16) Smem sm;

  const int n_wg = n_qt * g.B * g.H;
  const int wg = work_of(blockIdx.x, n_wg, wg_order);
  if (wg < 0) return;
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)kv_bh(g, bh) * g.n_kv * D;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int q0 = qt * kTileM + wave * 16;
  const int my_q = q0 + col;

  float qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = (my_q < g.n_q) ? Q[qb + (size_t)my_q * D + 4 * ks + grp] : 0.f;

  floatx4 o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  float4 kreg[P], vreg[P];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = tid + 256 * p;
      const int r = c / CPR, ch = c - r * CPR;
      const bool ok = c < CH && k0 + r < g.n_kv;
      kreg[p] = ok ? *(const float4*)(K + kb + (size_t)(k0 + r) * D + ch * 4) : make_float4(0, 0, 0, 0);
      vreg[p] = ok ? *(const float4*)(V + kb + (size_t)(k0 + r) * D + ch * 4) : make_float4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = tid + 256 * p;
      if (c < CH) {
        const int r = c / CPR, ch = c - r * CPR;
        *(float4*)(&sm.k[r * Smem::LD + ch * 4]) = kreg[p];
        *(float4*)(&sm.v[r * Smem::LD + ch * 4]) = vreg[p];
      }
    }
  };

  if (e_beg < e_end) load_tile((row_idx[e_beg] & kIdxMask) * kTileN);
  const int q_hi_wave = min(q0 + 15, g.n_q - 1);
  for (int e = e_beg; e < e_end; ++e) {
    const int ent = row_idx[e];
    const int k0 = (ent & kIdxMask) * kTileN;
    const bool partial = (ent >> kPartialBit) & 1;
    __syncthreads();
    store_tile();
    __syncthreads();
    if (e + 1 < e_end) load_tile((row_idx[e + 1] & kIdxMask) * kTileN);

    floatx4 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = rho(t, col);
      s[t] = mfma_f32_dot<KS>([&](int ks) { return sm.k[r * Smem::LD + 4 * ks + grp]; },
                              [&](int ks) { return qf[ks]; });
    }
    const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                           !tile_all_visible(g, q0, q_hi_wave, k0, k0 + kTileN - 1);
    float mx = kNegInf;
    uint32_t vis = 0xFFFFu;            // bit 4 t + i: element visible
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = !need_mask || elem_valid(g, my_q, k0 + rho(t, 4 * grp + i), partial);
        if (!ok) vis &= ~(1u << (4 * t + i));
        mx = fmaxf(mx, ok ? s[t][i] * g.scale : kNegInf);
      }
    }
    mx = wave_max16x4(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m - m_use) * kLog2e);
    float rs = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][i], g.scale, -m_use) * kLog2e);
        const float p = (vis >> (4 * t + i)) & 1u ? e : 0.f;
        s[t][i] = p;
        rs += p;
      }
    }
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rho(t, 4 * grp + i);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = mfma_f32(sm.v[r * Smem::LD + 16 * dt + col], s[t][i], o[dt]);
      }
    }
  }

  const float l_tot = wave_sum16x4(l);
  const bool valid = l_tot > 0.f;
  if (my_q < g.n_q) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      float4 w;
      w.x = valid ? o[dt][0] / l_tot : o[dt][0];
      w.y = valid ? o[dt][1] / l_tot : o[dt][1];
      w.z = valid ? o[dt][2] / l_tot : o[dt][2];
      w.w = valid ? o[dt][3] / l_tot : o[dt][3];
      *(float4*)(O + qb + (size_t)my_q * D + 16 * dt + 4 * grp) = w;
    }
    if (grp == 0) LSE[(size_t)bh * g.n_q + my_q] = valid ? (float)((double)m + log((double)l_tot)) : 0.f;
  }
}

template <int D>
int launch_fwd(int dtype, const Geom& g, const void* q, const void* k, const void* v, void* o,
               float* lse, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
               const int32_t* wg_order, hipStream_t stream) {
  const int grid = n_qt * g.B * g.H;
  if (dtype == kF32) {
    hipLaunchKernelGGL(fwd_kernel_32<D>, dim3(grid), dim3(256), 0, stream, g, (const float*)q,
                       (const float*)k, (const float*)v, (float*)o, lse, row_ptr, row_idx, n_qt,
                       wg_order);
  } else if (dtype == kF16) {
    hipLaunchKernelGGL((fwd_kernel_16<F16, D>), dim3(grid), dim3(kFwdThreads), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse,
                       row_ptr, row_idx, n_qt, wg_order);
  } else {
    hipLaunchKernelGGL((fwd_kernel_16<BF16, D>), dim3(grid), dim3(kFwdThreads), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse,
                       row_ptr, row_idx, n_qt, wg_order);
  }
  return check_launch("gki_bsa_fwd");
}

}  // namespace

int fwd_tile_m(int dtype) { return dtype == kF32 ? kTileM : kTileMF; }

int fwd_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                 void* o, float* lse, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
                 const int32_t* wg_order, hipStream_t stream) {
  switch (head_dim) {
    case 16: return launch_fwd<16>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, wg_order, stream);
    case 32: return launch_fwd<32>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, wg_order, stream);
    case 64: return launch_fwd<64>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, wg_order, stream);
    case 128: return launch_fwd<128>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, wg_order, stream);
    default: return fail(2, "unsupported head_dim " + std::to_string(head_dim));
  }
}

}  // namespace gki
