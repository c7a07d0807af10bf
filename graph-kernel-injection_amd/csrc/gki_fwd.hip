// Block-sparse StreamingLLM attention: prefill forward kernel for gfx950.
//
// Replaces the reference's Triton `_fwd_kernel` (sparse_triton_kernel.py:231-352)
// and its launch (sparse_triton_kernel.py:662-682). Semantics follow the
// reference: S = (Q K^T) * scale in fp32, token mask (causal & (sink | window))
// inside visited tiles, online softmax, P cast to V's dtype before P V,
// O = acc / l, LSE = m + ln(l) with the (O = 0, LSE = 0) sentinel for rows that
// saw no key (sparse_triton_kernel.py:341-352).
//
// Design (one workgroup = 4 waves = one 64-row q tile, wave w owns rows 16w..16w+15):
//  * S^T = K Q^T on v_mfma_f32_16x16x32_{bf16,f16} (v_mfma_f32_16x16x4f32 for
//    fp32). In the accumulator layout lane (g, c) holds q row c, so the running
//    max / sum are per-lane scalars; row reductions need two cross-group shuffles.
//  * K tile rows are fetched through the rho() permutation, which makes the S^T
//    accumulators of subtiles (2s, 2s+1) the B operand of O^T += V^T P^T as-is.
//  * K (row-major) and V^T (XOR-swizzled) tiles are staged in LDS; the next
//    tile's global loads are issued before the current tile's MFMAs.
//  * Only kept tiles are visited: the workgroup walks a GPU-resident CSR list.
#include "gki_common.cuh"

namespace gki {
namespace {

template <typename T, int D>
struct FwdCfg;

// 16-bit element types: K row-major (padded), V transposed.
template <int D, typename T>
struct FwdSmem16 {
  static constexpr int KLD = D + 8;
  uint16_t k[kTileN * KLD];
  uint16_t vt[D * kTileN];
};

template <int D>
struct FwdSmem32 {
  static constexpr int LD = D + 4;
  float k[kTileN * LD];
  float v[kTileN * LD];
};

// ---------------------------------------------------------------------------
// 16-bit path
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256, 2) void fwd_kernel_16(
    Geom g, const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ LSE,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ row_idx, int n_qt) {
  constexpr int KS = (D + 31) / 32;   // k-steps of the QK^T contraction
  constexpr int DT = D / 16;          // 16-row tiles of O^T
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int KCH = kTileN * CPR;   // chunks in a K tile
  constexpr int KP = (KCH + 255) / 256;
  constexpr int VTASK = 16 * CPR;     // (4-row group, chunk) tasks for V^T staging
  constexpr int VP = (VTASK + 255) / 256;
  using Smem = FwdSmem16<D, T>;
  __shared__ Smem sm;

  const int n_wg = n_qt * g.B * g.H;
  const int wg = xcd_remap(blockIdx.x, n_wg);
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)bh * g.n_kv * D;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 4, col = lane & 15;
  const int q0 = qt * kTileM + wave * 16;
  const int my_q = q0 + col;

  uint4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = 32 * ks + 8 * grp;
    qf[ks] = (my_q < g.n_q && d0 < D) ? *(const uint4*)(Q + qb + (size_t)my_q * D + d0)
                                      : make_uint4(0, 0, 0, 0);
  }

  floatx4 o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  uint4 kreg[KP];
  uint4 vreg[VP][4];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int p = 0; p < KP; ++p) {
      const int c = tid + 256 * p;
      const int r = c / CPR, ch = c - r * CPR;
      kreg[p] = (c < KCH && k0 + r < g.n_kv)
                    ? *(const uint4*)(K + kb + (size_t)(k0 + r) * D + ch * 8)
                    : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < VP; ++p) {
      const int task = tid + 256 * p;
      const int rg = task & 15, ch = task >> 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = k0 + 4 * rg + r;
        vreg[p][r] = (task < VTASK && row < g.n_kv)
                         ? *(const uint4*)(V + kb + (size_t)row * D + ch * 8)
                         : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int p = 0; p < KP; ++p) {
      const int c = tid + 256 * p;
      if (c < KCH) {
        const int r = c / CPR, ch = c - r * CPR;
        *(uint4*)(&sm.k[r * Smem::KLD + ch * 8]) = kreg[p];
      }
    }
#pragma unroll
    for (int p = 0; p < VP; ++p) {
      const int task = tid + 256 * p;
      if (task < VTASK) {
        const int rg = task & 15, ch = task >> 4;
        const uint16_t* e0 = (const uint16_t*)&vreg[p][0];
        const uint16_t* e1 = (const uint16_t*)&vreg[p][1];
        const uint16_t* e2 = (const uint16_t*)&vreg[p][2];
        const uint16_t* e3 = (const uint16_t*)&vreg[p][3];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int d = ch * 8 + j;
          const int phys = (((rg >> 1) ^ (d & 7)) << 3) + ((rg & 1) << 2);
          uint2 w;
          w.x = (uint32_t)e0[j] | ((uint32_t)e1[j] << 16);
          w.y = (uint32_t)e2[j] | ((uint32_t)e3[j] << 16);
          *(uint2*)(&sm.vt[d * kTileN + phys]) = w;
        }
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
      s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      const int r = rho(t, col);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        const uint4 a = (d0 < D) ? *(const uint4*)(&sm.k[r * Smem::KLD + d0]) : make_uint4(0, 0, 0, 0);
        s[t] = T::mfma(a, qf[ks], s[t]);
      }
    }

    const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                           !tile_all_visible(g, q0, q_hi_wave, k0, k0 + kTileN - 1);
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = s[t][i] * g.scale_log2;
        if (need_mask && !elem_valid(g, my_q, k0 + rho(t, 4 * grp + i), partial)) x = kNegInf;
        s[t][i] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = wave_max16x4(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    float rs = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[t][i] - m_use);
        s[t][i] = p;
        rs += p;
      }
    }
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;

#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float pv[8] = {s[2 * st][0], s[2 * st][1], s[2 * st][2], s[2 * st][3],
                     s[2 * st + 1][0], s[2 * st + 1][1], s[2 * st + 1][2], s[2 * st + 1][3]};
      const uint4 b = pack8<T>(pv);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 16 * dt + col;
        const int phys = ((4 * st + grp) ^ (d & 7)) << 3;
        const uint4 a = *(const uint4*)(&sm.vt[d * kTileN + phys]);
        o[dt] = T::mfma(a, b, o[dt]);
      }
    }
  }

  const float l_tot = wave_sum16x4(l);
  const bool valid = l_tot > 0.f;
  const float inv = valid ? 1.f / l_tot : 1.f;
  if (my_q < g.n_q) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint2 w;
      w.x = (uint32_t)T::from_float(o[dt][0] * inv) | ((uint32_t)T::from_float(o[dt][1] * inv) << 16);
      w.y = (uint32_t)T::from_float(o[dt][2] * inv) | ((uint32_t)T::from_float(o[dt][3] * inv) << 16);
      *(uint2*)(O + qb + (size_t)my_q * D + 16 * dt + 4 * grp) = w;
    }
    if (grp == 0) LSE[(size_t)bh * g.n_q + my_q] = valid ? m * kLn2 + __logf(l_tot) : 0.f;
  }
}

// ---------------------------------------------------------------------------
// fp32 path (v_mfma_f32_16x16x4f32): K and V stay row-major in LDS.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256, 2) void fwd_kernel_32(
    Geom g, const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ LSE, const int32_t* __restrict__ row_ptr,
    const int32_t* __restrict__ row_idx, int n_qt) {
  constexpr int KS = D / 4;
  constexpr int DT = D / 16;
  constexpr int CPR = D / 4;           // 16-byte chunks per row
  constexpr int CH = kTileN * CPR;
  constexpr int P = (CH + 255) / 256;
  using Smem = FwdSmem32<D>;
  __shared__ Smem sm;

  const int n_wg = n_qt * g.B * g.H;
  const int wg = xcd_remap(blockIdx.x, n_wg);
  const int bh = wg / n_qt, qt = wg - bh * n_qt;
  const size_t qb = (size_t)bh * g.n_q * D;
  const size_t kb = (size_t)bh * g.n_kv * D;
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
      s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      const int r = rho(t, col);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s[t] = mfma_f32(sm.k[r * Smem::LD + 4 * ks + grp], qf[ks], s[t]);
    }
    const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                           !tile_all_visible(g, q0, q_hi_wave, k0, k0 + kTileN - 1);
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = s[t][i] * g.scale_log2;
        if (need_mask && !elem_valid(g, my_q, k0 + rho(t, 4 * grp + i), partial)) x = kNegInf;
        s[t][i] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = wave_max16x4(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    float rs = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[t][i] - m_use);
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
    if (grp == 0) LSE[(size_t)bh * g.n_q + my_q] = valid ? m * kLn2 + __logf(l_tot) : 0.f;
  }
}

template <int D>
int launch_fwd(int dtype, const Geom& g, const void* q, const void* k, const void* v, void* o,
               float* lse, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
               hipStream_t stream) {
  const int grid = n_qt * g.B * g.H;
  if (dtype == kF32) {
    hipLaunchKernelGGL(fwd_kernel_32<D>, dim3(grid), dim3(256), 0, stream, g, (const float*)q,
                       (const float*)k, (const float*)v, (float*)o, lse, row_ptr, row_idx, n_qt);
  } else if (dtype == kF16) {
    hipLaunchKernelGGL((fwd_kernel_16<F16, D>), dim3(grid), dim3(256), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse,
                       row_ptr, row_idx, n_qt);
  } else {
    hipLaunchKernelGGL((fwd_kernel_16<BF16, D>), dim3(grid), dim3(256), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse,
                       row_ptr, row_idx, n_qt);
  }
  return check_launch("gki_bsa_fwd");
}

}  // namespace

int fwd_dispatch(int dtype, int head_dim, const Geom& g, const void* q, const void* k, const void* v,
                 void* o, float* lse, const int32_t* row_ptr, const int32_t* row_idx, int n_qt,
                 hipStream_t stream) {
  switch (head_dim) {
    case 16: return launch_fwd<16>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, stream);
    case 32: return launch_fwd<32>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, stream);
    case 64: return launch_fwd<64>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, stream);
    case 128: return launch_fwd<128>(dtype, g, q, k, v, o, lse, row_ptr, row_idx, n_qt, stream);
    default: return fail(2, "unsupported head_dim " + std::to_string(head_dim));
  }
}

}  // namespace gki
