/*
 * gki_bsa.h -- C ABI of the MI355X (gfx950) block-sparse StreamingLLM
 * FlashAttention library `libgki_bsa.so`.
 *
 * Conventions
 *  - Tensors are device pointers to contiguous [B, H, N, D] arrays (BHND,
 *    row-major), as produced by `.contiguous()` in the reference
 *    (sparse_triton_kernel.py:834). LSE is contiguous fp32 [B, H, N_Q].
 *  - LSE is the reference's: the natural log of each row's sum of exp of its
 *    scaled scores, m + ln(l) (sparse_triton_kernel.py:351), 0 for rows that
 *    see no key (its sentinel, :341-352). The kernels keep the running max in
 *    base 2 and convert once per row (in double, one fp32 rounding); the
 *    backward converts the stored value back once per row.
 *  - Grouped-query attention: Q / O / dQ have H heads, K / V / dK / dV have
 *    H_kv heads, H_kv dividing H; q head h reads kv head h / (H / H_kv).
 *    H_kv == H is the reference's multi-head case (the reference rejects any
 *    other head count, sparse_triton_kernel.py:640-641). dK / dV of a kv head
 *    sum the contributions of its H / H_kv q heads in fp32 before the single
 *    store (no atomics). The decode kernels serve a group's q heads from one
 *    K / V stream when (H / H_kv) * n_q <= decode_max_q, and, for 16-bit
 *    inputs (head_dim 64 / 128), when the computed-stream decode
 *    (gki_rolling_decode) has 2 .. 2 * decode_tile_m query rows per K / V
 *    stream.
 *  - dtype codes: 0 = fp32, 1 = fp16, 2 = bf16. head_dim in {16, 32, 64, 128}.
 *  - The block mask is an int32 [n_qb, n_kb] device array with
 *    n_qb = ceil(N_Q / block_m), n_kb = ceil(N_KV / block_n), shared across B, H.
 *  - Kernel schedules are int32 CSR / CSC lists over the kernels' fixed tiles
 *    (see gki_tile_sizes); entries are `tile_index | partial << 30`, where
 *    `partial` marks a tile only partly covered by kept mask blocks.
 *  - `stream` is a hipStream_t. Every call is asynchronous on it, never
 *    allocates or frees device memory, and keeps no pointer after returning.
 *  - Return value: 0 on success; otherwise non-zero (1 = bad argument,
 *    2 = unsupported configuration, 3 = HIP launch error), with the message in
 *    gki_last_error() (thread-local).
 */
#ifndef GKI_BSA_H_
#define GKI_BSA_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version (currently 8: grouped-query attention, H_kv after H; dK/dV work
 * items from gki_dkdv_items, whose chunk can be capped by max_chunk; the
 * optional workgroup orders of the forward and dQ grids from gki_fwd_order;
 * natural-log LSE in every output; gki_bsa_bwd's row-term workspace holds
 * 2 * B * H * N_Q floats; the gki_read_probe measurement helper). */
int gki_abi_version(void);

/* Message of the last failing call on this thread. */
const char* gki_last_error(void);

/* Kernel tile geometry the schedules must be built for: q rows of the forward
 * tile for 16-bit and fp32 inputs, q rows of the backward tile, kv rows of
 * every tile, q rows of the decode tile, and max query rows handled by the
 * decode kernel. Any pointer may be NULL. */
int gki_tile_sizes(int32_t* fwd_tile_m_16, int32_t* fwd_tile_m_32, int32_t* bwd_tile_m,
                   int32_t* tile_n, int32_t* decode_tile_m, int32_t* decode_max_q);

/* Block-level StreamingLLM mask, bit-exact with `make_streaming_mask`
 * (sparse_triton_kernel.py:104-181): keep (i, j) iff q_hi > k_lo and
 * (k_lo < sink or k_hi - 1 >= q_lo - window + 1), q_lo = i*block_m + n_kv - n_q.
 * `mask` holds ceil(n_q/block_m) * ceil(n_kv/block_n) int32. */
int gki_streaming_mask(int32_t* mask, int64_t n_q, int64_t n_kv, int64_t sink,
                       int64_t window, int64_t block_m, int64_t block_n, void* stream);

/* Dense / dense-causal block mask, `make_dense_mask`
 * (sparse_triton_kernel.py:184-210); requires block sizes dividing n_q, n_kv. */
int gki_dense_mask(int32_t* mask, int64_t n_q, int64_t n_kv, int64_t block_m,
                   int64_t block_n, int32_t causal, void* stream);

/* Classify the kernels' tile_m x tile_n tiles against a block mask of any
 * granularity, honouring the StreamingLLM token rule when is_causal:
 * 0 = no in-bounds element is both kept by the lifted mask and allowed by the
 * token rule, 1 = the lifted mask keeps every element the token rule allows,
 * 2 = partly kept (kernels then consult the mask per element). No reference
 * counterpart: the reference gates its Triton tiles directly on the mask
 * (sparse_triton_kernel.py:283-285) and masks tokens inside (:312-322). */
int gki_tile_mask(const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m,
                  int32_t block_n, int32_t n_q, int32_t n_kv, int32_t tile_m,
                  int32_t tile_n, int32_t is_causal, int32_t sink_size,
                  int32_t window_size, int32_t* tile_mask, void* stream);

/* Kept-block list, step 1: per-row / per-column kept counts of an int32
 * [n_rows, n_cols] matrix and their exclusive prefix sums (row_ptr[n_rows+1],
 * col_ptr[n_cols+1]). Replaces the reference's per-iteration int32 gate loads
 * (sparse_triton_kernel.py:283-285, 448-450, 563-565) with a CSR/CSC list. */
int gki_block_list_counts(const int32_t* m, int32_t n_rows, int32_t n_cols,
                          int32_t* row_cnt, int32_t* col_cnt, int32_t* row_ptr,
                          int32_t* col_ptr, void* stream);

/* Kept-block list, step 2: fill CSR (row -> ascending columns) and/or CSC
 * (column -> ascending rows) indices; either output may be NULL. For a 0/1
 * mask the CSR order equals `mask.nonzero()`. */
int gki_block_list_fill(const int32_t* m, int32_t n_rows, int32_t n_cols,
                        const int32_t* row_ptr, const int32_t* col_ptr,
                        int32_t* row_idx, int32_t* col_idx, void* stream);

/* Work list of the dK/dV grid (host arrays; no reference counterpart -- the
 * reference runs one program per kv tile, sparse_triton_kernel.py:719-777).
 * col_ptr: the CSC column pointers (n_kt + 1, host copy) of the backward tiles;
 * group: q heads per K/V head; bh_kv: B * H_kv. A kv tile's walk of
 * group x (its list length) iterations becomes one item, or -- when longer than
 * the chunk max(32, ceil(total iterations / 8192)) -- several near-equal items
 * whose fp32 partials gki_bsa_bwd sums in item order (deterministic; fp32
 * partials with a compensated sum). max_chunk > 0 caps the chunk (more,
 * shorter items: a caller may cut columns of any length, as the tests do to
 * run the split path on short sequences); 0 keeps the rule above. The Python
 * op passes max(2, ceil(total iterations / 512)) for fp32 inputs whose
 * B * H_kv * n_kt columns number under 512: the fp32 dK/dV kernel runs one
 * workgroup per CU, and short grids would leave CUs idle. Writes
 * items [n_items][4] = (kv tile, first iteration, end iteration, partial slot or
 * -1) and split [n_split][3] = (kv tile, first slot, slot count), and the counts;
 * pass items = split = NULL to size them first. n_pslots partial slots per
 * (b, kv head) need 2 * 64 * head_dim floats each. */
int gki_dkdv_items(const int32_t* col_ptr, int32_t n_kt, int32_t group, int32_t bh_kv,
                   int32_t max_chunk, int32_t* items, int32_t* n_items, int32_t* split,
                   int32_t* n_split, int32_t* n_pslots);

/* Order of the forward (or dQ) grid's workgroups (host arrays; no reference
 * counterpart -- the reference's grids run their programs in index order,
 * sparse_triton_kernel.py:662-682, 756-777). row_ptr: the forward (or
 * backward) CSR row pointers (n_qt + 1, host copy); bh: B * H. Writes order[n_qt * bh], a permutation of
 * the work units (b * H + h) * n_qt + qt: the units each XCD receives (one
 * contiguous range per XCD, as the kernels map workgroups) sorted by
 * descending kept-tile count, ties in index order, so that each XCD ends its
 * share with the short units. Results do not depend on the order. */
int gki_fwd_order(const int32_t* row_ptr, int32_t n_qt, int32_t bh, int32_t* order);

/* Prefill forward: replaces the `_fwd_kernel` launch in
 * `_BlockSparseFlashAttention.forward` (sparse_triton_kernel.py:662-682).
 * O = softmax(mask(Q K^T * scale)) V, LSE = m + ln(l) (natural), 0 for empty rows.
 * row_ptr/row_idx: CSR over ceil(n_q/fwd_tile_m) q tiles (fwd_tile_m_16 or
 * fwd_tile_m_32 by dtype) of kept kv tiles. wg_order: NULL (index order) or a
 * device copy of gki_fwd_order's table for this CSR and B * H (a workgroup
 * whose entry is out of range does nothing). */
int gki_bsa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                int32_t dtype, int32_t B, int32_t H, int32_t H_kv, int32_t n_q, int32_t n_kv,
                int32_t head_dim, const int32_t* row_ptr, const int32_t* row_idx,
                int32_t n_qt, const int32_t* wg_order, const int32_t* mask, int32_t n_qb,
                int32_t n_kb, int32_t block_m, int32_t block_n, float softmax_scale,
                int32_t is_causal, int32_t sink_size, int32_t window_size, void* stream);

/* Backward: replaces the three launches in `_BlockSparseFlashAttention.backward`
 * (sparse_triton_kernel.py:719-777): the row terms Delta = rowsum(O * dO), dK/dV
 * over the CSC list (device copies of gki_dkdv_items' lists: kv_items 16-byte
 * aligned; kv_partials a 16-byte aligned fp32 workspace
 * [B * H_kv][n_pslots][2][64][head_dim], needed when n_split > 0) and dQ over
 * the CSR list, both over bwd_tile_m x tile_n tiles. `lse` is the forward's
 * (natural) LSE. `delta` is a caller-owned fp32 [2, B, H, N_Q] workspace for
 * the row terms (its contents on return are internal: Delta -- negated and
 * scaled for fp16 / bf16 -- then each row's LSE in base 2). dq, dk, dv are
 * fully written (no zero-fill needed). dq_order: NULL (index order) or a
 * device copy of gki_fwd_order's table for the backward CSR and B * H (the
 * dQ grid runs each XCD's q tiles longest list first). */
int gki_bsa_bwd(const void* q, const void* k, const void* v, const void* o,
                const void* dout, const float* lse, void* dq, void* dk, void* dv,
                float* delta, int32_t dtype, int32_t B, int32_t H, int32_t H_kv,
                int32_t n_q, int32_t n_kv, int32_t head_dim, const int32_t* row_ptr,
                const int32_t* row_idx, int32_t n_qt, const int32_t* col_ptr,
                const int32_t* col_idx, int32_t n_kt, const int32_t* kv_items,
                int32_t n_items, const int32_t* kv_split, int32_t n_split,
                int32_t n_pslots, float* kv_partials, const int32_t* dq_order,
                const int32_t* mask, int32_t n_qb, int32_t n_kb,
                int32_t block_m, int32_t block_n, float softmax_scale, int32_t is_causal,
                int32_t sink_size, int32_t window_size, void* stream);

/* Floats of workspace gki_bsa_decode needs for a given split count (none is
 * read when n_splits == 1). */
int64_t gki_bsa_decode_workspace_floats(int32_t B, int32_t H, int32_t n_q,
                                        int32_t head_dim, int32_t n_splits);

/* Decode token stream (once per mask): expands the kept kv tiles of the single
 * decode q tile (`tile_list`, n_tiles entries of the decode_tile_m x tile_n
 * schedule) into exactly the positions some query row can see (per tile its
 * sink run and its window run under the token rule; every in-bounds position
 * when not causal), ascending, entry = position | partial << 30. `tokens` holds n_tiles * tile_n int32; the count
 * is written to the device scalar `n_tokens`. No reference counterpart: the
 * reference visits whole tiles (sparse_triton_kernel.py:283-299). */
int gki_decode_tokens(const int32_t* tile_list, int32_t n_tiles, int32_t n_q, int32_t n_kv,
                      const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m,
                      int32_t block_n, int32_t is_causal, int32_t sink_size,
                      int32_t window_size, int32_t* tokens, int32_t* n_tokens, void* stream);

/* Decode step (n_q <= decode_max_q, head_dim 64 or 128): replaces the
 * reference's BLOCK_M = 1 use of `_fwd_kernel` for decode
 * (benchmark.py:500-511, 802-804). n_splits workgroups per (b, h) each stream
 * an equal slice of the token list (from gki_decode_tokens); with
 * n_splits == 1 they write O / LSE directly, otherwise they write partials to
 * `workspace` and a second launch merges them. Same outputs as gki_bsa_fwd. */
int gki_bsa_decode(const void* q, const void* k, const void* v, void* o, float* lse,
                   int32_t dtype, int32_t B, int32_t H, int32_t H_kv, int32_t n_q, int32_t n_kv,
                   int32_t head_dim, const int32_t* tokens, int32_t n_tokens,
                   const int32_t* mask, int32_t n_qb, int32_t n_kb, int32_t block_m,
                   int32_t block_n, float softmax_scale, int32_t is_causal,
                   int32_t sink_size, int32_t window_size, float* workspace,
                   int32_t n_splits, void* stream);

/* ---- Rolling StreamingLLM KV cache -------------------------------------------
 * No reference counterpart: the reference decodes from a full [B, H, N_KV, D]
 * cache (sparse_triton_kernel.py:636-641) although only S + W tokens are ever
 * visible (README.md:41-67). A rolling cache holds, per (b, h), `sink_size`
 * sink slots followed by a ring of `ring_size` slots: position p < sink_size
 * lives in slot p, position p >= sink_size in slot
 * sink_size + (p - sink_size) mod ring_size. Cache tensors are
 * [B, H, sink_size + ring_size, head_dim], contiguous, in the input dtype. For
 * decode rows n_q the ring must hold window_size + n_q - 1 positions. */

/* Host-only: the visible-token stream of the n_q decode rows (the last n_q of
 * `length` positions): sinks [0, n_sink), then positions window_lo ..
 * length - 1; n_tokens = n_sink + max(0, length - window_lo). This is the same
 * ascending stream gki_decode_tokens yields for a full cache with the
 * StreamingLLM mask. Any output pointer may be NULL. */
int gki_rolling_stream(int64_t length, int32_t n_q, int32_t sink_size, int32_t window_size,
                       int32_t ring_size, int32_t* n_sink, int32_t* window_lo,
                       int32_t* n_tokens);

/* Append n_new tokens (k_new / v_new: [B, H, n_new, head_dim]) at positions
 * start_pos .. start_pos + n_new - 1. Positions that a later position of the
 * same call overwrites are skipped, so each slot is written at most once. */
int gki_rolling_append(void* k_cache, void* v_cache, const void* k_new, const void* v_new,
                       int32_t dtype, int32_t B, int32_t H, int32_t head_dim,
                       int32_t sink_size, int32_t ring_size, int64_t start_pos,
                       int32_t n_new, void* stream);

/* Decode step over a rolling cache holding positions 0 .. length - 1: the n_q
 * query rows (q: [B, H, n_q, head_dim]) sit at positions length - n_q ..
 * length - 1 and see (k <= q) & (k < sink_size | k >= q - window_size + 1).
 * Same kernel, stream order and split rule as gki_bsa_decode over a full cache
 * of `length` tokens (bit-identical O and LSE for the same n_splits); the
 * workspace is sized by gki_bsa_decode_workspace_floats. */
int gki_rolling_decode(const void* q, const void* k_cache, const void* v_cache, void* o,
                       float* lse, int32_t dtype, int32_t B, int32_t H, int32_t H_kv, int32_t n_q,
                       int32_t head_dim, int32_t sink_size, int32_t window_size,
                       int32_t ring_size, int64_t length, float softmax_scale,
                       float* workspace, int32_t n_splits, void* stream);

/* gki_rolling_decode without a workspace argument: the split partials
 * (gki_bsa_decode_workspace_floats(B, H, n_q, head_dim, n_splits) floats when
 * n_splits > 1) live in a library-owned device array of 4194304 floats
 * (16 MiB), one per GPU, held until the process ends; larger requests return
 * 1 with a message and launch nothing. The call allocates nothing (no hipMalloc,
 * no allocating library routine). Same kernels, stream order and results as
 * gki_rolling_decode with the same n_splits. Calls that overlap on one GPU
 * (other streams, other threads) share the array and race; serialise them.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). The array used is that of the device `stream` launches on (the
 * current device for the null stream), looked up once per device. */
int gki_rolling_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, void* o,
                               float* lse, int32_t dtype, int32_t B, int32_t H, int32_t H_kv,
                               int32_t n_q, int32_t head_dim, int32_t sink_size,
                               int32_t window_size, int32_t ring_size, int64_t length,
                               float softmax_scale, int32_t n_splits, void* stream);

/* Measurement helper, no counterpart in the reference: reads exactly the K and V
 * bytes a single-position StreamingLLM decode step reads from a full cache --
 * per (b, kv head) slice of bh slices of n_kv rows of row_bytes (a multiple of
 * 16) the sink rows 0 .. min(sink_size, n_kv) - 1 and the window rows
 * max(that, n_kv - window_size) .. n_kv - 1 -- with 16-byte non-temporal loads
 * and nothing else, XOR-folding them into `out` (gki_read_probe_words(bh)
 * words; the XOR of all of them is the XOR of every 32-bit word read). For
 * timing the decode step against the read ceiling of its own access pattern
 * (bench.py). Asynchronous on `stream`; allocates nothing. */
int64_t gki_read_probe_words(int32_t bh);
int gki_read_probe(const void* k, const void* v, int32_t bh, int64_t n_kv, int32_t row_bytes,
                   int32_t sink_size, int32_t window_size, uint32_t* out, int64_t out_words,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GKI_BSA_H_ */
