// Shared device/host helpers for the gfx950 block-sparse attention kernels.
//
// Everything here is CDNA4-specific: wave64, v_mfma_f32_16x16x32_{bf16,f16}
// and v_mfma_f32_16x16x4f32 fragments, LDS staging helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace gki {

// ---------------------------------------------------------------------------
// Element types. Storage is always the raw 16/32-bit pattern; conversions go
// through __bf16 / _Float16 so the compiler emits v_cvt_pk_bf16_f32 (RNE) and
// v_cvt_f16_f32 (RNE), matching torch's .to(dtype) rounding.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

struct F32 {
  using storage = float;
  static constexpr bool is_f32 = true;
  __device__ static inline float to_float(float x) { return x; }
  __device__ static inline float from_float(float x) { return x; }
};
struct F16 {
  using storage = uint16_t;
  using vec8 = f16x8;
  static constexpr bool is_f32 = false;
  __device__ static inline float to_float(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  __device__ static inline uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  __device__ static inline floatx4 mfma(const uint4& a, const uint4& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // eight 1.0 elements: an all-ones MFMA operand (row sums on the matrix pipe)
  __device__ static inline uint4 ones8() { return make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u); }
  // a.lo * b.lo + a.hi * b.hi + c in fp32 on packed pairs (v_dot2_f32_f16)
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
};
struct BF16 {
  using storage = uint16_t;
  using vec8 = bf16x8;
  static constexpr bool is_f32 = false;
  __device__ static inline float to_float(uint16_t x) {
    return __builtin_bit_cast(float, ((uint32_t)x) << 16);
  }
  __device__ static inline uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  __device__ static inline floatx4 mfma(const uint4& a, const uint4& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint4 ones8() { return make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u); }
  // a.lo * b.lo + a.hi * b.hi + c in fp32 on packed pairs (v_dot2_f32_bf16)
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a), __builtin_bit_cast(b2, b), c, false);
  }
};

__device__ inline floatx4 mfma_f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// fp32 dot products over the head dimension on v_mfma_f32_16x16x4f32, KS
// k-steps of 4: the steps go round-robin into NC independent accumulators,
// summed pairwise at the end, so a long contraction (D = 64: 16 steps, 2 per
// accumulator; D = 128: 32 steps, 4 per accumulator) rounds like a short one.
// With 4 accumulators at D = 64 the scores' and dP's rounding was the largest
// error of the fp32 gradients at large logits (2x the eager path's on some
// inputs); 8 halve it. a(ks) / b(ks) give step ks's operands.
template <int KS, typename FA, typename FB>
__device__ inline floatx4 mfma_f32_dot(FA a, FB b) {
  constexpr int NC = KS >= 16 ? 8 : (KS >= 8 ? 4 : (KS >= 4 ? 2 : 1));
  floatx4 c[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) c[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) c[ks % NC] = mfma_f32(a(ks), b(ks), c[ks % NC]);
  if constexpr (NC == 8) return ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
  else if constexpr (NC == 4) return (c[0] + c[1]) + (c[2] + c[3]);
  else if constexpr (NC == 2) return c[0] + c[1];
  else return c[0];
}

// 16-byte streaming (non-temporal) global load.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld_nt16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Two fp32 -> two 16-bit elements in one v_cvt_pk_{bf16,f16}_f32 (RNE).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ inline uint32_t pack2(float a, float b);
template <>
__device__ inline uint32_t pack2<BF16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <>
__device__ inline uint32_t pack2<F16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// Eight 16-bit elements times a power-of-two scale, rounded back (exact
// unless a result falls below the format's smallest normal).
template <typename T>
__device__ inline uint4 scale8(const uint4& v, float s) {
  const uint16_t* h = (const uint16_t*)&v;
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = T::to_float(h[i]) * s;
  return make_uint4(pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3]), pack2<T>(f[4], f[5]),
                    pack2<T>(f[6], f[7]));
}

// Pack 8 fp32 values into 8 16-bit elements (one 16x16x32 MFMA operand).
template <typename T>
__device__ inline uint4 pack8(const float* v) {
  return make_uint4(pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]),
                    pack2<T>(v[6], v[7]));
}
// Same, from the accumulators of two 16x16 subtiles (rows 0-3 then 4-7).
template <typename T>
__device__ inline uint4 pack8(const floatx4& lo, const floatx4& hi) {
  return make_uint4(pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3]), pack2<T>(hi[0], hi[1]),
                    pack2<T>(hi[2], hi[3]));
}

// LDS tile layout for 16-bit [64][D] tiles: row-major, no padding, 16-byte
// chunks XOR-swizzled per row. gfx950 LDS has 64 banks of 4 bytes (one
// 256-byte "bank row" per clock), so a read is conflict-free when the 16-byte
// chunks that one clock serves land on 16 distinct positions of a bank row.
// With a = row & 3, b = (row >> 3) & 3 the swizzle is a bijection of the
// (a, b) pairs the two read patterns touch at once:
//  * 16-byte reads of rows {b..b+3, b+8..b+11, b+16.., b+24..} at one chunk
//    (the rho() row order; 16 lanes per clock),
//  * ds_read_b64_tr_b16 over rows {r..r+3, r+8..r+11} x 2 adjacent chunks
//    (32 lanes per clock),
// and the tile fill (consecutive lanes, consecutive chunks of one bank row).
// Tiles narrower than 256 bytes share a bank row between 256/(2D) rows; the
// row bits that select the slice take the place of a. D = 16 keeps a 2-way
// conflict (only 2 chunks per row).
template <int D>
__device__ inline int lds_swz(int row) {
  const int b = (row >> 3) & 3;
  const int bb = 2 * (b & 1) + (b >> 1);
  if constexpr (D >= 128) return (4 * (row & 3) + bb) & (D / 8 - 1);
  else if constexpr (D == 64) return 4 * ((row >> 1) & 1) + bb;
  else if constexpr (D == 32) return bb;
  else return 0;
}
template <int D>
__device__ inline int lds_off(int row, int col) {
  return row * D + ((((col >> 3) ^ lds_swz<D>(row))) << 3) + (col & 7);
}

// Transposed MFMA operand from a swizzled 16-bit LDS tile via
// ds_read_b64_tr_b16: within each 16-lane group, lane l points at row
// k0 + l/4, columns n0 + 4*(l%4) .. +3, and the instruction hands lane i column
// n0 + i of those four rows. Two reads give lane (g, c) = (lane/16, lane%16)
// the 8 elements tile[k0 + 8g + e][n0 + c], e = 0..7: the K-operand layout of
// v_mfma_f32_16x16x32_{bf16,f16} for a matrix stored K-major. (k0 is a
// multiple of 32, so rows r and r+4 share a swizzle.)
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
template <int D>
__device__ inline uint4 lds_tr8(const uint16_t* tile, int k0, int n0, int lane) {
  const int g = lane >> 4, l = lane & 15;
  const uint16_t* p = tile + lds_off<D>(k0 + 8 * g + (l >> 2), n0 + 4 * (l & 3));
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p);
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 4 * D));
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return make_uint4(a.x, a.y, b.x, b.y);
}
// 16-byte row read (8 elements starting at a multiple-of-8 column).
template <int D>
__device__ inline uint4 lds_row8(const uint16_t* tile, int row, int col) {
  return *(const uint4*)(tile + lds_off<D>(row, col));
}

// Stage a 64-row tile of a row-major [n, D] 16-bit matrix: each thread moves
// P 16-byte chunks, consecutive threads covering consecutive bytes of a row.
// The loads go through a buffer resource over the rows that exist, so rows at
// or past n_rows read as zero without a per-element predicate, and the lane
// offsets are 32-bit (chunk c of the tile sits at byte 16 c).
template <int D, int NT = 256>
struct RowTile {
  static constexpr int CPR = D / 8;          // 16-byte chunks per row
  static constexpr int CH = 64 * CPR;
  static constexpr int P = (CH + NT - 1) / NT;
  uint4 reg[P];
  // base and r0 are uniform at every call site (kernel arguments and a tile
  // index from the schedule); reading them through readfirstlane lets the
  // compiler keep the resource in scalar registers (no per-lane loop).
  __device__ inline void load(const uint16_t* base, int r0, int n_rows, int tid) {
    const int rows = max(0, min(64, n_rows - r0));
    const uint64_t a = (uint64_t)(uintptr_t)(base + (size_t)r0 * D);
    const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(uintptr_t)u, (short)0, __builtin_amdgcn_readfirstlane(rows * D * 2), 0x00020000);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = tid + NT * p;
      reg[p] = make_uint4(0, 0, 0, 0);
      if (CH % NT == 0 || c < CH)
        reg[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16 * c, 0, 0));
    }
  }
  __device__ inline void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int c = tid + NT * p;
      if (c < CH) *(uint4*)(lds + lds_off<D>(c / CPR, (c % CPR) * 8)) = reg[p];
    }
  }
};

// 16 bytes at (row, d0) of a row-major [n_rows, D] 16-bit matrix, zero when
// row >= n_rows or d0 >= D (n_rows >= 1). The load is unconditional, from a
// clamped in-bounds address, and the zero a select: as a predicated load each
// would sit in its own branch with its own wait, so that a kernel prologue's
// row loads would land one after another instead of together.
template <int D>
__device__ inline uint4 row16_or_zero(const uint16_t* base, int row, int n_rows, int d0) {
  const bool ok = row < n_rows && d0 < D;
  const uint4 v = *(const uint4*)(base + (size_t)min(row, n_rows - 1) * D + (d0 < D ? d0 : 0));
  return ok ? v : make_uint4(0, 0, 0, 0);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// One gfx950 LDS-DMA load: every lane fetches 16 bytes from its global address
// `src` and the wave writes them to LDS bytes [lds, lds + 1024), lane i at
// lds + 16 i. Issued as inline asm so that the compiler does not guard every
// later LDS read with a wait on it (it cannot tell which buffer the DMA
// targets); callers wait explicitly with dma_wait() before the barrier that
// publishes the buffer. Only M0 and memory are touched.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void dma_load16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
// Buffer-resource variant: lane i fetches 16 bytes at the resource base +
// voff[i] (same LDS placement), so the per-tile address arithmetic is scalar
// (the base) and the lane offsets stay in registers unchanged; offsets at or
// past `bytes` read zero instead of faulting. Measured faster than the global
// form for the forward's K / V tiles.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ inline i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));   // stride 0
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);                   // num_records
  r.w = 0x00020000;                                                   // DATA_FORMAT 32
  return r;
}
__device__ inline void dma_buf16(i32x4 rsrc, int voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc),
               "s"(lds)
               : "memory", "m0");
}
// 4-byte variant: lane i writes lds + 4 i.
__device__ inline void dma_load4(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// Wait until this wave's vector-memory operations (LDS-DMA included) are done:
// s_waitcnt vmcnt(0) (gfx9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15). Issued via
// the builtin so the compiler's own wait tracking also sees every earlier load
// as complete and inserts no further vmcnt waits for them.
__device__ inline void dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Stage a full 64-row tile of a row-major [n, D] 16-bit matrix straight into
// the swizzled LDS layout with LDS-DMA loads: no VGPR staging and no ds_write.
// One wave instruction fills 1 KB of LDS, lane i writing bytes 16i..16i+15,
// so the swizzle is applied on the global side: lane i fetches the chunk that
// belongs at its LDS position. The workgroup's NW waves cover the tile's D/8
// blocks of 1 KB (block NW p + wave for p = 0, 1, ...); `off` is the lane's
// element offset inside the tile for each block it moves (computed once).
// Only for tiles whose 64 rows are all in bounds.
template <int D, int NW = 4>
struct DmaTile {
  static constexpr int NB = D / 8;                     // 1 KB blocks per tile
  static constexpr int NP = (NB + NW - 1) / NW;        // blocks per wave
  int off[NP];
  int wave;
  __device__ inline void init(int tid) {
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int e = (NW * p + wave) * 512 + 8 * lane;  // LDS element offset
      const int row = e / D, pch = (e % D) >> 3;
      off[p] = row * D + ((pch ^ lds_swz<D>(row)) << 3);
    }
  }
  // Rows r0 .. r0+63 of `base` through a buffer resource over those rows: the
  // tile base is uniform, so a tile costs no per-lane address arithmetic.
  __device__ inline void load(const uint16_t* base, int r0, const uint16_t* lds) const {
    const i32x4 rsrc = buffer_rsrc(base + (size_t)r0 * D, 64 * D * 2);
    const uint32_t l0 = lds_addr(lds);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int blk = NW * p + wave;
      if (NB % NW == 0 || blk < NB) dma_buf16(rsrc, 2 * off[p], l0 + blk * 1024);
    }
  }
};

// ---------------------------------------------------------------------------
// Kernel tiling. The forward uses 128x64 (q x kv) tiles, four waves per
// workgroup, each wave owning 32 query rows; the backward kernels use 64x64
// tiles, each wave owning 16 rows of the tile's outer axis. The decode kernel
// (n_q <= kDecodeMaxQ) uses a single 16-row q tile.
// ---------------------------------------------------------------------------
constexpr int kTileM = 64;       // q rows of the dQ / dK-dV tiles
constexpr int kTileN = 64;       // kv rows of every tile
constexpr int kTileMF = 128;     // q rows of the forward tile (4 waves x 32 rows)
constexpr int kDecodeTileM = 16;
constexpr int kDecodeMaxQ = 4;
// dK/dV work items: at least kDkdvMinChunk iterations each, and about
// kDkdvTargetItems items over the whole grid when the column walks are long.
constexpr int kDkdvMinChunk = 32;
constexpr int kDkdvTargetItems = 8192;

// q heads one decode workgroup serves: a whole group of grouped-query heads
// when its group * n_q rows fit the kernel's row limit (K / V read once per
// group), else one head.
inline int decode_heads_per_workgroup(int group, int n_q) {
  return group > 1 && group * n_q <= kDecodeMaxQ ? group : 1;
}

constexpr int kPartialBit = 30;       // schedule entry flag: needs per-element mask lookup
constexpr int kIdxMask = (1 << kPartialBit) - 1;

// Row permutation rho(t, j) of a 64-row tile into four 16-row MFMA subtiles.
// Subtile t = 2s+h, lane-row j = 4a+i holds tile row 32s + 8a + 4h + i. With
// this order the fp32 accumulator of subtiles (2s, 2s+1) held by lane group a
// covers rows 32s+8a .. 32s+8a+7 contiguously, i.e. it already IS the 8-element
// K-operand of a 16x16x32 MFMA over those rows: no register transpose needed.
__device__ inline int rho(int t, int j) {
  return ((t >> 1) << 5) + ((j >> 2) << 3) + ((t & 1) << 2) + (j & 3);
}

// Geometry + masking parameters shared by all attention kernels.
struct Geom {
  int B, H;
  int H_kv, group;    // K/V heads and q heads per K/V head (grouped-query attention; 1 = MHA)
  int n_q, n_kv, q_off;
  float scale;        // natural-log softmax scale (any finite value)
  float scale_log2;   // scale * log2(e)
  // The 16-bit prefill and matrix-core decode kernels track the running max
  // on unscaled scores, which needs a positive scale. They read each 32-bit
  // word w of Q as (w & q_and) ^ q_xor and scale by qk_scale_log2 instead:
  // scale < 0 flips the sign of Q (exact: (-Q) K^T * |scale| equals
  // Q K^T * scale bit for bit), scale == 0 zeroes Q (every score 0, as
  // Q K^T * 0) with qk_scale_log2 = log2(e); scale > 0 leaves Q as it is.
  float qk_scale_log2;
  uint32_t q_and, q_xor;
  // 16-bit backward: dS = P (dP - Delta) scale, cast to 16 bits before the
  // dK / dQ products. For a power-of-two scale in [2^-4, 1] (1/8 at
  // head_dim 64) the kernels multiply the V (dK/dV) or dO (dQ) operand and
  // -Delta by it once: every product and partial sum of the dP accumulator
  // is then the same value times the scale (exact in fp32), so it ends as
  // (dP - Delta) scale and dS costs one multiply (prescale = 1). Only a 16-bit
  // operand that the scale takes below the smallest normal rounds (by at most
  // half its subnormal spacing, 2^-25 for fp16). Otherwise prescale = 0.
  int prescale;
  int causal, sink, window;
  // original block mask (used only for tiles flagged partial)
  const int32_t* mask;
  int n_qb, n_kb, bm, bn;
};

// Work list of the dK / dV grid (built on the host by gki_dkdv_items). A kv
// tile's walk -- group x (its kept q tiles) iterations, iteration i visiting
// list entry i % L of q head i / L -- is cut into items of at most a chunk of
// iterations, so no workgroup carries a long column (the sink column, the
// columns of a large grouped-query group) alone. A column with one item stores
// dK / dV itself; the items of a split column store fp32 partials, which a
// reduce pass sums in item order (deterministic).
struct KvWork {
  const int32_t* items;   // [n_items][4]: kv tile, first iteration, end iteration, partial slot (-1: none)
  int n_items;
  const int32_t* split;   // [n_split][3]: kv tile, its first partial slot, number of slots
  int n_split;
  int n_pslots;           // partial slots per (b, kv head)
  float* partials;        // [B * H_kv][n_pslots][2 (dK, dV)][64][D] fp32
};

// A 16-byte Q fragment as the unscaled-max kernels read it (see Geom::q_and).
__device__ inline uint4 q_words(const Geom& g, uint4 w) {
  return make_uint4((w.x & g.q_and) ^ g.q_xor, (w.y & g.q_and) ^ g.q_xor, (w.z & g.q_and) ^ g.q_xor,
                    (w.w & g.q_and) ^ g.q_xor);
}

// (b, q head) -> (b, kv head) row index of K / V (and dK / dV).
__device__ inline int kv_bh(const Geom& g, int bh) {
  return g.group == 1 ? bh : (bh / g.H) * g.H_kv + (bh % g.H) / g.group;
}

// Bounds + token predicate for (q row, kv column), branch-free.
__host__ __device__ inline bool elem_tok(const Geom& g, int q_row, int kv) {
  const int qa = q_row + g.q_off;
  const bool in = (q_row < g.n_q) & (kv < g.n_kv);
  const bool vis = (kv <= qa) & ((kv < g.sink) | (kv >= qa - g.window + 1));
  return in & ((g.causal == 0) | vis);
}

// Full element predicate for (q row, kv column) of a tile flagged "needs mask":
// tiles flagged partial also consult the lifted block mask.
__host__ __device__ inline bool elem_valid(const Geom& g, int q_row, int kv, bool partial) {
  bool ok = elem_tok(g, q_row, kv);
  if (partial && ok) ok = g.mask[(size_t)(q_row / g.bm) * g.n_kb + kv / g.bn] != 0;
  return ok;
}

// ---------------------------------------------------------------------------
// The same predicate for 64 elements at once: one query row against the 64
// keys of a tile (or one key against the 64 query rows of a tile) as a 64-bit
// word, bit j = element j. The token rule is an interval condition along
// either axis, so the word costs a few shifts per lane and tile instead of a
// compare chain per element.
// ---------------------------------------------------------------------------

// Bits lo .. hi of a 64-bit word (clamped to 0 .. 63; empty when hi < lo).
__host__ __device__ inline uint64_t bit_range(int lo, int hi) {
  lo = lo < 0 ? 0 : lo;
  hi = hi > 63 ? 63 : hi;
  return hi < lo ? 0 : (~0ull >> (63 - hi)) & (~0ull << lo);
}

// Window length for the visibility words: any window of at least n_kv keys
// reaches key 0 from every row, so clamping there is exact and keeps the
// window-edge arithmetic inside int for n_q, n_kv < 2^30.
__host__ __device__ inline int word_window(const Geom& g) {
  return g.window < g.n_kv ? g.window : g.n_kv;
}

// elem_valid(g, q_row, k0 + j, partial) for j = 0 .. 63, as bits.
__host__ __device__ inline uint64_t row_valid_bits(const Geom& g, int q_row, int k0, bool partial) {
  if (q_row >= g.n_q) return 0;
  uint64_t b = bit_range(0, g.n_kv - 1 - k0);
  if (g.causal) {
    const int qa = q_row + g.q_off - k0;           // key j visible iff j <= qa and
    b &= bit_range(0, qa) &                        // (j >= qa - W + 1 or k0 + j < S)
         (bit_range(qa - word_window(g) + 1, 63) | bit_range(0, g.sink - 1 - k0));
  }
  if (partial) {                                 // kept blocks of the row's block row
    const int mrow = (q_row / g.bm) * g.n_kb;     // 32-bit: the mask has < 2^31 blocks
    uint64_t kept = 0;
    for (int kb = k0 / g.bn; kb < g.n_kb && kb * g.bn < k0 + 64; ++kb)
      if (g.mask[mrow + kb]) kept |= bit_range(kb * g.bn - k0, (kb + 1) * g.bn - 1 - k0);
    b &= kept;
  }
  return b;
}

// elem_valid(g, q0 + j, kv, partial) for j = 0 .. 63, as bits.
__host__ __device__ inline uint64_t col_valid_bits(const Geom& g, int kv, int q0, bool partial) {
  if (kv >= g.n_kv) return 0;
  uint64_t b = bit_range(0, g.n_q - 1 - q0);
  if (g.causal) {
    const int a = kv - g.q_off - q0;               // row j visible iff j >= a and
    b &= bit_range(a, 63) &                        // (kv < S or j <= a + W - 1)
         (kv < g.sink ? ~0ull : bit_range(0, a + word_window(g) - 1));
  }
  if (partial) {                                 // kept blocks of the key's block column
    const int kb = kv / g.bn;
    uint64_t kept = 0;
    for (int qb = q0 / g.bm; qb < g.n_qb && qb * g.bm < q0 + 64; ++qb)
      if (g.mask[qb * g.n_kb + kb]) kept |= bit_range(qb * g.bm - q0, (qb + 1) * g.bm - 1 - q0);
    b &= kept;
  }
  return b;
}

// The 16 elements that lane group `grp` holds in the rho() layout: element
// (t, i) is tile row / key rho(t, 4 grp + i) = 32 (t >> 1) + 8 grp + 4 (t & 1) + i,
// i.e. bit 4 (t & 1) + i of byte `grp` of word half t >> 1. Returned as two
// words whose low 8 bits are those bytes.
struct LaneBits {
  uint32_t w[2];
  __device__ inline LaneBits(uint64_t bits, int grp) {
    w[0] = (uint32_t)bits >> (8 * grp);
    w[1] = (uint32_t)(bits >> 32) >> (8 * grp);
  }
  // x where element (t, i) is set, `other` where it is not (bit-select, no compare)
  __device__ inline float pick(int t, int i, float x, float other) const {
    const int m = __builtin_amdgcn_sbfe((int)w[t >> 1], 4 * (t & 1) + i, 1);   // 0 or -1
    return __int_as_float((__float_as_int(x) & m) | (__float_as_int(other) & ~m));
  }
};

// Is some (q, k) with q in [q_lo, q_hi], k in [k_lo, k_hi] (inclusive, absolute
// positions, non-empty) visible under the token rule (k <= q) & (k < S | k >= q-W+1)?
__device__ inline bool any_visible(long q_lo, long q_hi, long k_lo, long k_hi, long sink, long window) {
  const bool sink_part = k_lo < sink && k_lo <= q_hi;
  // window: some q with max(k_lo, q-W+1) <= min(k_hi, q)
  const long qa = q_lo > k_lo ? q_lo : k_lo;
  const long qb = q_hi < k_hi + window - 1 ? q_hi : k_hi + window - 1;
  const bool window_part = window >= 1 && qa <= qb;
  return sink_part || window_part;
}

// True when every (q, kv) with q in [q_lo, q_hi], kv in [k_lo, k_hi] (inclusive,
// already in bounds) is visible under the StreamingLLM token rule.
__device__ inline bool tile_all_visible(const Geom& g, int q_lo, int q_hi, int k_lo, int k_hi) {
  if (!g.causal) return true;
  const int qa = q_lo + g.q_off, qb = q_hi + g.q_off;
  if (k_hi > qa) return false;
  return (k_hi < g.sink) || (k_lo >= qb - g.window + 1);
}

// XCD-aware remap: hardware dispatches workgroup b to XCD b % 8. Give each XCD
// one contiguous range of logical ids so neighbouring q tiles of one head (which
// share most K/V tiles) run on the same XCD and hit in its L2.
constexpr int kXcd = 8;
// First logical id of XCD x's range (of n); the range holds n / 8 ids, one more
// for the first n % 8 XCDs (as many as the hardware hands that XCD).
__host__ __device__ inline int xcd_start(int x, int n) {
  const int per = n / kXcd, rem = n % kXcd;
  return x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
}
__host__ __device__ inline int xcd_remap(int b, int n) { return xcd_start(b % kXcd, n) + b / kXcd; }

// Wave issue priority around a cluster of MFMAs (ON: the D <= 64 kernels).
// While a wave issues its products it wins the SIMD's issue arbitration over
// the waves in their softmax / dS VALU phase, so the matrix pipe is fed more
// evenly: at D = 64 (four waves per SIMD) the forward ran 2% and the
// backward 0.5-1.3% faster on long StreamingLLM sequences; at D = 128 (two
// waves per SIMD) it made the forward 3% slower, so it is off there.
template <bool ON>
__device__ inline void mfma_priority_hi() {
  if constexpr (ON) __builtin_amdgcn_s_setprio(1);
}
template <bool ON>
__device__ inline void mfma_priority_lo() {
  if constexpr (ON) __builtin_amdgcn_s_setprio(0);
}

// Work unit of workgroup b in a launch over n units: its XCD-remapped logical
// id, or, with an order table (gki_fwd_order), the unit that table lists at
// that id (each XCD's range sorted heaviest first, so the units dispatched last
// are the short ones and the launch ends with less idle tail). -1 (the
// workgroup exits) for a table entry outside 0 .. n-1.
__device__ inline int work_of(int b, int n, const int32_t* order) {
  const int l = xcd_remap(b, n);
  if (order == nullptr) return l;
  const int w = __builtin_amdgcn_readfirstlane(order[l]);
  return (unsigned)w < (unsigned)n ? w : -1;
}

// Reductions across the 4 lane groups (lanes l, l^16, l^32, l^48) with the
// gfx950 VALU row swaps, no LDS trip. v_permlane32_swap a, b exchanges the
// upper 32 lanes of a with the lower 32 lanes of b; with a = b = x, lane l then
// holds {x[l], x[l^32]} in (a, b). v_permlane16_swap does the same for odd /
// even 16-lane rows ({x[l], x[l^16]}). Inline asm because the compiler's
// builtin returns the first register for both results (checked on gfx950);
// the s_nop pairs keep the VALU -> permlane -> VALU wait states.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void swap32(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ inline void swap16(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
#pragma clang diagnostic pop
// DPP row permute of a float (VALU rate, no LDS): CTRL is a gfx9 dpp_ctrl
// code; all rows / banks enabled, every source lane lies in the same 16-lane row.
template <int CTRL>
__device__ inline float dpp_perm(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i of each 8 reads lane 7-i
constexpr int kDppMirror = 0x140;     // lane i of each 16 reads lane 15-i

// Sum over aligned groups of N lanes (N a power of two, 1..64); every lane gets
// its group's sum. Once the lanes of each quad (8, 16-lane half) hold equal
// values, the mirrors pair each with the other quad (half): no LDS traffic.
template <int N>
__device__ inline float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_perm<kDppXor1>(x);
  if constexpr (N >= 4) x += dpp_perm<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp_perm<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_perm<kDppMirror>(x);
  if constexpr (N >= 32) {
    float a = x, b = x;
    swap16(a, b);
    x = a + b;
  }
  if constexpr (N >= 64) {
    float a = x, b = x;
    swap32(a, b);
    x = a + b;
  }
  return x;
}

// Max across the 64/N aligned groups of N lanes, for values that are uniform
// within each group (so any pairing of whole groups is a valid exchange).
template <int N>
__device__ inline float cross_group_max(float x) {
  if constexpr (N <= 1) x = fmaxf(x, dpp_perm<kDppXor1>(x));
  if constexpr (N <= 2) x = fmaxf(x, dpp_perm<kDppXor2>(x));
  if constexpr (N <= 4) x = fmaxf(x, dpp_perm<kDppHalfMirror>(x));
  if constexpr (N <= 8) x = fmaxf(x, dpp_perm<kDppMirror>(x));
  if constexpr (N <= 16) {
    float a = x, b = x;
    swap16(a, b);
    x = fmaxf(a, b);
  }
  if constexpr (N <= 32) {
    float a = x, b = x;
    swap32(a, b);
    x = fmaxf(a, b);
  }
  return x;
}

// Swaps and maxes in one asm block: through fmaxf the compiler canonicalises
// both asm outputs (v_max x, x, x) before every max.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline float wave_max16x4(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1\n\tv_max_f32 %0, %0, %1\n\t"
      "v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1\n\t"
      "v_max_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
}
#pragma clang diagnostic pop
__device__ inline float wave_sum16x4(float x) {
  float a = x, b = x;
  swap32(a, b);
  x = a + b;
  a = x;
  b = x;
  swap16(a, b);
  return a + b;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// The kernels keep each row's running max m2 and sum l in base 2 (scores
// times log2 e); the stored LSE is the natural log-sum-exp m + ln(l)
// (sparse_triton_kernel.py:351). Both conversions run once per row in double,
// so each is a single fp32 rounding of the exact value.
__device__ inline float lse_natural(float m2, float l) {
  return (float)(((double)m2 + (double)log2f(l)) * 0.6931471805599453);
}
__device__ inline float lse_base2(float lse) { return (float)((double)lse * 1.4426950408889634); }

}  // namespace gki

// ---------------------------------------------------------------------------
// Host-side error plumbing for the C ABI.
// ---------------------------------------------------------------------------
namespace gki {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
}  // namespace gki

#define GKI_REQUIRE(cond, code, msg)          \
  do {                                        \
    if (!(cond)) return ::gki::fail(code, msg); \
  } while (0)
