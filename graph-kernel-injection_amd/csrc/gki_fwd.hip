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
//  * head_dim 128 runs the loop skewed by one kv tile (fwd_kernel_16's PIPE),
//    so that one wave's MFMAs of the next tile overlap its own softmax.
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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Issue order of the skewed (PIPE) loop, imposed with sched_group_barrier
// (masks: 0x008 MFMA, 0x100 LDS read, 0x002 VALU). S_{j+1}: kPipeAheadS K
// reads first, then per MFMA pair one more read and kPipeValu1 + kPipeValu2
// VALU ops of the exp work between the two MFMAs and after them. O += V P:
// kPipeAheadO V^T reads first, then two reads and one VALU op (the maxima of
// S_{j+1}) per MFMA pair. Measured on the c2 forward: 2 + 1 VALU beat 3 + 2
// by 1.5%; reads 4 / 8 ahead beat 2 / 4 by 1.6%; without the imposed order
// the compiler issues every MFMA first and the loop is 5% slower than this.
constexpr int kPipeAheadS = 4, kPipeAheadO = 8, kPipeValu1 = 2, kPipeValu2 = 1;
constexpr int kFwdThreads = 64 * (8 / kFwdRB);
// Waves per SIMD the compiler must fit in registers (HIP's second launch
// bound): 4 (up to 128 VGPRs) for head_dim <= 64, whose 32 KB of K / V buffers
// allow four workgroups per CU (the extra waves hide more latency: 4-7% faster
// than three at head_dim 64); 2 for head_dim 128 (64 KB of buffers, two
// workgroups per CU). Eight-wave workgroups over 256-row q tiles (half the K /
// V staging per flop) ran 6-13% slower at both head dims.
//
// PIPE selects the tile schedule. Without it every kv tile runs S = K Q^T,
// then mask / max / exp, then O += V P in turn, and the matrix cores idle
// through the softmax unless the SIMD's other wave has MFMAs to issue. With
// it the loop is skewed by one tile: iteration j runs S_{j+1} = K_{j+1} Q^T
// while it exponentiates S_j (MFMA and VALU of one wave in one straight-line
// block, interleaved in the order kPipe* describes), then O += V_j P_j while
// it takes the row maxima of S_{j+1}. K is therefore read one tile ahead of V:
// at iteration j the LDS holds K_{j+1} and V_j while K_{j+2} and V_{j+1} land
// in the other halves of the two double buffers (the same 2 x 2 tiles of LDS).
// The loop is unrolled by two so that the two score tiles swap roles without
// register copies, and P_j is pinned (an empty asm that takes it) inside the
// S_{j+1} block: otherwise the compiler sinks the exp work past the mask
// branch into the O += V P block and no MFMA of S_{j+1} overlaps it.
template <typename T, int D, bool PIPE>
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
  const int tid = threadIdx.x, wave = tid >> 6;
  const int lane = tid & 63, grp = lane >> 4, col = lane & 15;
  const int qw = qt * kTileMF + wave * 16 * RB;   // first row of this wave

  uint4 qf[RB][KS];
#pragma unroll
  for (int h = 0; h < RB; ++h) {
    const int q = qw + 16 * h + col;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 32 * ks + 8 * grp;
      const uint4 v = q_words(g, row16_or_zero<D>(Q + qb, q, g.n_q, d0));
      qf[h][ks] = (q < g.n_q && d0 < D) ? v : make_uint4(0, 0, 0, 0);
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
  auto stage1 = [&](const uint16_t* src, int k0, uint16_t* dst) {
    if (k0 + kTileN <= g.n_kv) {
      dma.load(src + kb, k0, dst);
    } else {
      RowTile<D, NT> t;
      t.load(src + kb, k0, g.n_kv, tid);
      t.store(dst, tid);
      // Unconditional, so that no register load of this branch is pending
      // where it rejoins the DMA path: otherwise the compiler waits for all
      // vector memory there, the just-issued DMA of the next tile included.
      dma_wait();
    }
  };
  auto tile_k0 = [&](int ent) { return (ent & kIdxMask) * kTileN; };

  // S^T of one kv tile for both row blocks.
  auto scores = [&](const uint16_t* ck, floatx4 (&s)[RB][4]) {
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
  };
  // Token mask of row block h of a tile (only where some element of it can
  // be hidden).
  auto apply_mask = [&](int ent, int h, floatx4 (&s)[4]) {
    const int k0 = tile_k0(ent);
    const bool partial = (ent >> kPartialBit) & 1;
    const int q0 = qw + 16 * h;
    const bool need_mask = partial || (q0 + 15 >= g.n_q) || (k0 + kTileN > g.n_kv) ||
                           !tile_all_visible(g, q0, min(q0 + 15, g.n_q - 1), k0, k0 + kTileN - 1);
    if (need_mask) {
      const LaneBits vis(row_valid_bits(g, q0 + col, k0, partial), grp);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t][i] = vis.pick(t, i, s[t][i], kNegInf);
    }
  };
  auto lane_max = [&](const floatx4 (&s)[4]) {
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[t][i]);
    return mx;
  };
  // A row's max exceeds the reference by the slack only if one of its lanes'
  // maxima does (qk_scale_log2 > 0, so scaling after the max is exact): the
  // cross-lane reduction runs only then. The threshold is a trigger only:
  // whether m moves is decided exactly inside. Rescales O and the row sums of
  // block h, so it runs after every product of the tiles before.
  auto move_max = [&](int h, float mx) {
    if (__any(mx > thr[h])) {
      const float mr = wave_max16x4(mx) * g.qk_scale_log2;
      const bool grow = mr > m[h] + kRescaleSlack;
      const float alpha = grow ? __builtin_amdgcn_exp2f(m[h] - mr) : 1.f;
      m[h] = grow ? mr : m[h];
      thr[h] = (m[h] + kRescaleSlack) * inv_c;
      lsum[h][0] *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[h][dt] *= alpha;
    }
  };
  // P = exp2(S c - m) of row block h, in place.
  auto exp_h = [&](int h, floatx4 (&s)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        s[t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][i], g.qk_scale_log2, -m[h]));
  };
  // P of both row blocks packed to 16-bit MFMA operands (subtiles 2st, 2st+1).
  auto probs = [&](floatx4 (&s)[RB][4], uint4 (&p)[2][RB]) {
#pragma unroll
    for (int h = 0; h < RB; ++h) {
      exp_h(h, s[h]);
#pragma unroll
      for (int st = 0; st < 2; ++st) p[st][h] = pack8<T>(s[h][2 * st], s[h][2 * st + 1]);
    }
  };
  // O^T += V^T P^T and the row sums; operand(st, h) gives P of subtiles
  // (2st, 2st+1) of row block h.
  auto accumulate = [&](const uint16_t* cv, auto&& operand) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      uint4 b[RB];
#pragma unroll
      for (int h = 0; h < RB; ++h) b[h] = operand(st, h);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint4 a = lds_tr8<D>(cv, 32 * st, 16 * dt, lane);
#pragma unroll
        for (int h = 0; h < RB; ++h) o[h][dt] = T::mfma(a, b[h], o[h][dt]);
      }
#pragma unroll
      for (int h = 0; h < RB; ++h) lsum[h] = T::mfma(ones, b[h], lsum[h]);
    }
  };
  // K and V of one tile into buffer b (the ragged tile with one wait).
  auto stage2 = [&](int k0, int b) {
    if (k0 + kTileN <= g.n_kv) {
      dma.load(K + kb, k0, sk[b]);
      dma.load(V + kb, k0, sv[b]);
    } else {
      RowTile<D, NT> t;
      t.load(K + kb, k0, g.n_kv, tid);
      t.store(sk[b], tid);
      t.load(V + kb, k0, g.n_kv, tid);
      t.store(sv[b], tid);
      dma_wait();
    }
  };

  const int e_beg = row_ptr[qt], e_end = row_ptr[qt + 1];
  if constexpr (!PIPE) {
    if (e_beg < e_end) stage2(tile_k0(row_idx[e_beg]), 0);
    dma_wait();
    __syncthreads();

    for (int e = e_beg; e < e_end; ++e) {
      const int buf = (e - e_beg) & 1;
      const int ent = row_idx[e];
      const int k0 = tile_k0(ent);
      const bool partial = (ent >> kPartialBit) & 1;
      if (e + 1 < e_end) stage2(tile_k0(row_idx[e + 1]), buf ^ 1);
      const uint16_t* ck = sk[buf];
      const uint16_t* cv = sv[buf];

      floatx4 s[RB][4];
      mfma_priority_hi<(D <= 64)>();
      scores(ck, s);
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
  } else {
    const int n = e_end - e_beg;
    floatx4 sa[RB][4], sb[RB][4];
    // Prologue: K_0, V_0 and K_1 in LDS, S_0 with its maxima.
    if (n > 0) {
      const int k0 = tile_k0(row_idx[e_beg]);
      stage1(K, k0, sk[0]);
      stage1(V, k0, sv[0]);
      if (n > 1) stage1(K, tile_k0(row_idx[e_beg + 1]), sk[1]);
    }
    dma_wait();
    __syncthreads();
    if (n > 0) {
      const int ent = row_idx[e_beg];
      scores(sk[0], sa);
#pragma unroll
      for (int h = 0; h < RB; ++h) {
        apply_mask(ent, h, sa[h]);
        move_max(h, lane_max(sa[h]));
      }
    }
    __syncthreads();   // every wave is done with K_0 before iteration 0 refills its buffer

    // Iteration j (j + 1 < n): S_{j+1} from K_{j+1} into sn while s = S_j
    // becomes P_j; O += V_j P_j while sn's maxima are taken.
    auto step = [&](int j, floatx4 (&s)[RB][4], floatx4 (&sn)[RB][4]) {
      const int e = e_beg + j;
      const int ent1 = row_idx[e + 1];
      // LDS: K_{j+1} in sk[(j+1)&1], V_j in sv[j&1]; refill the other halves
      if (j + 2 < n) stage1(K, tile_k0(row_idx[e + 2]), sk[j & 1]);
      stage1(V, tile_k0(ent1), sv[(j + 1) & 1]);

      uint4 p[2][RB];
      scores(sk[(j + 1) & 1], sn);   // MFMA ...
      probs(s, p);                   // ... under VALU
      // P is formed here, not sunk past the mask branch into the next block
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int h = 0; h < RB; ++h) {
          u32x4 w = __builtin_bit_cast(u32x4, p[st][h]);
          asm volatile("" : "+v"(w));
          p[st][h] = __builtin_bit_cast(uint4, w);
        }
      // issue order: the MFMAs of S_{j+1} (4 KS RB, in pairs) between the exp work
      __builtin_amdgcn_sched_group_barrier(0x100, kPipeAheadS, 0);
#pragma unroll
      for (int i = 0; i < 2 * KS * RB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i + kPipeAheadS < 4 * KS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kPipeValu1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kPipeValu2, 0);
      }
#pragma unroll
      for (int h = 0; h < RB; ++h) apply_mask(ent1, h, sn[h]);
      accumulate(sv[j & 1], [&](int st, int h) { return p[st][h]; });   // MFMA ...
      float mx[RB];
#pragma unroll
      for (int h = 0; h < RB; ++h) mx[h] = lane_max(sn[h]);   // ... under VALU
      // issue order: the 2 DT MFMA pairs of O += V P (two V^T reads each) with
      // the maxima of S_{j+1} between them
      __builtin_amdgcn_sched_group_barrier(0x100, kPipeAheadO, 1);
#pragma unroll
      for (int i = 0; i < 2 * DT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        if (2 * i + kPipeAheadO < 4 * DT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        if (2 * i + 1 + kPipeAheadO < 4 * DT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
      }
#pragma unroll
      for (int h = 0; h < RB; ++h) move_max(h, mx[h]);
      dma_wait();
      __syncthreads();
    };
    auto last = [&](floatx4 (&s)[RB][4]) {
      uint4 p[2][RB];
      probs(s, p);
      accumulate(sv[(n - 1) & 1], [&](int st, int h) { return p[st][h]; });
    };
    // Unrolled by two so that the score buffers swap roles without copies.
    int j = 0;
    for (; j + 2 < n; j += 2) {
      step(j, sa, sb);
      step(j + 1, sb, sa);
    }
    if (j + 1 < n) {
      step(j, sa, sb);
      last(sb);
    } else if (n > 0) {
      last(sa);
    }
  }

  // The epilogue's row offsets from the lane index afresh (mbcnt: not provably
  // the one above), not the prologue's Q offsets held across the loop.
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int grp_e = lane_e >> 4, col_e = lane_e & 15;
#pragma unroll
  for (int h = 0; h < RB; ++h) {
    const int my_q = qw + 16 * h + col_e;
    const float l_tot = lsum[h][0];
    const bool valid = l_tot > 0.f;
    const float inv = valid ? 1.f / l_tot : 1.f;
    if (my_q < g.n_q) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 w;
        w.x = pack2<T>(o[h][dt][0] * inv, o[h][dt][1] * inv);
        w.y = pack2<T>(o[h][dt][2] * inv, o[h][dt][3] * inv);
        *(uint2*)(O + qb + (size_t)my_q * D + 16 * dt + 4 * grp_e) = w;
      }
      if (grp_e == 0) LSE[(size_t)bh * g.n_q + my_q] = valid ? lse_natural(m[h], l_tot) : 0.f;
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

// One wave per SIMD at head_dim 128: VGPRs + AGPRs hold it without scratch
// (two waves spilled 284 bytes per lane: B1 H16 N8192 fp32 forward 1.39
// against 1.12 ms, B1 H4 N1024 0.072 against 0.055 ms).
template <int D>
__global__ __launch_bounds__(256, D >= 128 ? 1 : 2) void fwd_kernel_32(
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

// The skewed schedule holds two score tiles (32 more VGPRs): head_dim 128
// has them within its 256; at head_dim 64 it would cost the fourth workgroup
// per CU (168 VGPRs), and three skewed workgroups ran 2-7% slower than four
// plain ones (c3 / c5 forward).
template <int D>
constexpr bool kFwdPipe = D >= 128;

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
    hipLaunchKernelGGL((fwd_kernel_16<F16, D, kFwdPipe<D>>), dim3(grid), dim3(kFwdThreads), 0, stream, g,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse,
                       row_ptr, row_idx, n_qt, wg_order);
  } else {
    hipLaunchKernelGGL((fwd_kernel_16<BF16, D, kFwdPipe<D>>), dim3(grid), dim3(kFwdThreads), 0, stream, g,
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
