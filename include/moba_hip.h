/*
 * moba_hip.h -- C ABI of libmoba_hip.so, the gfx950 MoBA sparse block
 * attention kernels.
 *
 * Conventions shared by every entry point:
 *   - All pointers are DEVICE pointers unless stated otherwise; the library
 *     never allocates, frees or synchronises.  Workspaces are passed in.
 *   - `stream` is a hipStream_t (void* here to keep the header HIP-free); all
 *     work is enqueued on it, so every call is capturable into a hipGraph.
 *   - `dtype`: 0 = bf16, 1 = fp16 (16-bit element storage).
 *   - Tensors are dense row-major with the shapes given; [T,H,D] means
 *     element (t,h,d) at ((t*H)+h)*D+d.
 *   - Return 0 on success; otherwise a MOBA_ERR_* code and
 *     moba_hip_last_error() describes the failure (thread-local).
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the Xiaotangyuan-xty/moba-merge-cuda repository).
 */
#ifndef MOBA_HIP_H
#define MOBA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOBA_HIP_ABI_VERSION 1
#define MOBA_OK 0
#define MOBA_ERR_ARG 1
#define MOBA_ERR_LAUNCH 2
#define MOBA_ERR_CAPACITY 3
#define MOBA_ERR_STALE 4    /* a plan made before the pool's last change */

/* Message of the last failed call on this thread. */
const char* moba_hip_last_error(void);
int moba_hip_version(void);

/* ---------------------------------------------------------------- prefill */

/* Chunk-mean key pooling of the F routing candidates.
 * Replaces `keys.mean(1)` / `keys.float().mean(1)` of
 * src/moba_opt/grouped_attention.py:48-52 (diagnostic.py:391-399).
 * k [T,Hkv,D]; chunk_start[F] first token of each candidate chunk;
 * precision 0 = "upstream" (mean rounded to dtype), 1 = "fp32".
 * means [F,Hkv,D] fp32.  Canonical order: lane j of a wave sums tokens j,
 * j+64, ...; the 64 partials are added by the fixed tree part[j] += part[j+off],
 * off = 32..1; then / chunk (the CPU oracle implements the same order). */
int moba_hip_chunk_means(const void* k, int dtype, int T, int Hkv, int D,
                         const int* chunk_start, int F, int chunk, int precision,
                         float* means, void* stream);

/* Gate scores + mask + stable top-R of every (token, q head).
 * Replaces the einsum/mask/topk of src/moba_opt/grouped_attention.py:55-71
 * (diagnostic.py:401-426).  q [T,Hq,D]; means [F,Hkv,D];
 * cu_chunk[nchunk+1], chunk_batch[nchunk], first_chunk[nchunk] (first chunk of
 * the chunk's sequence); R = min(topk-1, F) in [1,8].
 * sel [T,Hq,R] int32: selected global chunk ids ascending, -1 padded.
 * gate (nullable) [F,Hq,T] fp32 masked scores (-inf where illegal). */
int moba_hip_route_prefill(const void* q, int dtype, int T, int Hq, int Hkv, int D,
                           const float* means, const int* cu_chunk, int nchunk,
                           const int* chunk_batch, const int* first_chunk, int R, int F,
                           int* sel, float* gate, void* stream);

/* Expert-major row lists (expert e = f*Hkv + kvhead, rows ordered
 * (group head, token) like grouped_attention.py:78-86).
 * counts[E], row_off[E+1], tile_off[E+1] (tiles of block_rows rows), rows[sum
 * counts] = ((s*Hq + h) << 3) | j where j is the chunk's rank in sel[s,h,:]
 * (R <= 8, T*Hq < 2^28); the partial slot of that row is (s*Hq + h)*R + j.
 * work is an 8-byte aligned int32 workspace of moba_hip_pack_experts_work(T,
 * Hq, Hkv, F) entries (64-bit selection masks of every (token, head), then
 * per-block candidate counts of each expert).
 * Replaces the nonzero/index_select packing of grouped_attention.py:78-94. */
int moba_hip_pack_experts(const int* sel, int T, int Hq, int Hkv, int R,
                          const int* cu_chunk, const int* chunk_batch, const int* cu_seqlens,
                          const int* filtered, int F, int block_rows, int* counts,
                          int* row_off, int* tile_off, int* rows, int* work, void* stream);

/* Size in int32 entries of the work buffer of moba_hip_pack_experts (-1 for a
 * bad shape).  Helper of the entry above; no counterpart in the reference. */
int64_t moba_hip_pack_experts_work(int T, int Hq, int Hkv, int F);

/* Query rows per prefill tile for head dim D (-1 for an unsupported D): the
 * block_rows of moba_hip_pack_experts and the row step of the self tiles
 * passed to moba_hip_prefill_fwd / _bwd.  Helper of those entries; no
 * counterpart in the reference. */
int moba_hip_prefill_rows(int D);

/* Sparse block attention forward + global-softmax merge.
 * Replaces OptMixedAttention.forward (src/moba_opt/mixed_attention.py:42-139):
 * both _flash_attn_varlen_forward calls and merge_forward_cuda
 * (src/moba_opt/ops/merge.cu:187-288).
 * q [T,Hq,D], k/v [T,Hkv,D]; self_tiles[n_self_tiles][3] = (chunk, first row,
 * kv head) tiles of moba_hip_prefill_rows(D) rows, chunk -1 for an empty entry;
 * the G workgroups of entries [x*n/8, (x+1)*n/8) run on XCD x when n is a
 * multiple of 8 (any list is correct; this layout keeps a run in one L2); sel/R, filtered[F] and the pack_experts outputs (with
 * block_rows = moba_hip_prefill_rows(D)) describe
 * the remote rows (R = 0: self branch only, e.g. the full-causal fallback with
 * one chunk per sequence).  max_remote_tiles bounds tile_off[E].
 * part_o [T*Hq*R, D] (dtype) and part_ml [T*Hq*R, 2] fp32 (per-slot softmax
 * max and sum in the log2 domain) are workspaces.
 * out [T,Hq,D] (dtype), lse [T,Hq] fp32 natural-log global LSE. */
int moba_hip_prefill_fwd(const void* q, const void* k, const void* v, int dtype, int T, int Hq,
                         int Hkv, int D, float scale, const int* cu_chunk, const int* self_tiles,
                         int n_self_tiles, const int* sel, int R, const int* filtered, int E,
                         const int* tile_off, const int* row_off, const int* counts,
                         const int* rows, int max_remote_tiles, void* part_o, float* part_ml,
                         void* out, float* lse, void* stream);

/* Backward of moba_hip_prefill_fwd with the GLOBAL O and LSE.
 * Replaces OptMixedAttention.backward (src/moba_opt/mixed_attention.py:141-225):
 * both _flash_attn_varlen_backward calls plus the autograd scatter of the
 * packed remote grads (grouped_attention.py:81-89).  out/dout [T,Hq,D],
 * lse [T,Hq] from the forward; kv_tiles[n_kv_tiles][4] = (chunk, first key,
 * filtered index or -1, kv head): one workgroup per entry, tiles of 128
 * keys; chunk -1 marks an empty entry.  delta [2*T*Hq] and
 * part_dq [T*Hq*R, D] (dtype) are workspaces.  pack is a workspace of
 * T*Hq*R*(4*D + 8) bytes, required when R > 0 and D <= 128 (the expert rows
 * of q, dO, lse / scale and delta copied contiguously by the parts-1 launches and read
 * by the key-major kernel: pass the same buffer to both calls), else may be
 * NULL.  dq [T,Hq,D], dk/dv [T,Hkv,D] (dtype) are fully written (every key
 * belongs to exactly one kv tile).
 * parts selects the launches: 1 = Delta, expert-row packing and dq
 * (query-major kernels), 2 = dk/dv (key-major kernel, needs the Delta and
 * packing of a parts-1 call), 3 = both in order.
 * kv_splits in [1,16]: when > 1 the launch runs n_kv_tiles*kv_splits
 * workgroups and a device-built schedule cuts each key tile's query-row
 * tiles into segments of near-equal length, so heavy tiles (early chunks that
 * many rows select) get more workgroups than light ones; part_dkv is then a
 * workspace of moba_hip_prefill_bwd_work(n_kv_tiles, kv_splits, D) bytes and
 * n_kv_tiles must be <= 4096.
 * Deterministic: no atomics, fixed reduction order (the schedule is a fixed
 * function of the expert row counts). */
int moba_hip_prefill_bwd(const void* q, const void* k, const void* v, const void* out,
                         const void* dout, const float* lse, int dtype, int T, int Hq, int Hkv,
                         int D, float scale, const int* cu_chunk, const int* self_tiles,
                         int n_self_tiles, const int* kv_tiles, int n_kv_tiles, const int* sel,
                         int R, const int* filtered, int E, const int* tile_off,
                         const int* row_off, const int* counts, const int* rows,
                         int max_remote_tiles, float* delta, void* part_dq, void* dq, void* dk,
                         void* dv, int parts, int kv_splits, float* part_dkv, void* pack,
                         void* stream);

/* Bytes of the row-split workspace moba_hip_prefill_bwd needs for kv_splits
 * > 1 (0 for kv_splits < 2 or bad arguments).  No counterpart in the
 * reference, whose backward is two flash-attention calls; a shape query like
 * moba_hip_pack_experts_work. */
int64_t moba_hip_prefill_bwd_work(int n_kv_tiles, int kv_splits, int D);

/* Standalone global-softmax merge of caller-owned partials.
 * Replaces merge_forward(self_out, self_lse, remote_out, remote_lse, mapping,
 * kmax, check_capacity, deterministic) (src/moba_opt/ops/bindings.cpp:6-22,
 * src/moba_opt/ops/merge.cu:187-288).  self_out [T,H,D] and remote_out [M,D]
 * in dtype (0 bf16, 1 fp16, 2 fp32), self_lse [T,H] and remote_lse [M] fp32
 * natural log, mapping [M] int64 (row p = t*H + h of each remote partial).
 * out [T,H,D] (dtype) and lse [T,H] fp32: m = max of the row's LSEs,
 * O = (w_self o_self + sum w_j o_j) / z, z = sum w_j + w_self, L = m + log z.
 * Always deterministic and atomic-free: remote partials are taken in
 * ascending j (a stable radix sort by row), merged one wave64 per row.
 * D a multiple of 8 in [8,256], kmax in [1,8].  work: moba_hip_merge_work(T*H,
 * M) bytes.  status [2] int32 (device), written on the stream: status[0] = 1
 * if a mapping entry lies outside [0,T*H) (ignored), status[1] = 1 if a row
 * has more than kmax remote partials (the first kmax are used); the
 * reference's check_capacity is the caller reading them after the call. */
int moba_hip_merge(const void* self_out, const float* self_lse, const void* remote_out,
                   const float* remote_lse, const int64_t* mapping, int dtype, int64_t T, int H,
                   int D, int64_t M, int kmax, void* work, int* status, void* out, float* lse,
                   void* stream);

/* Bytes of the work buffer of moba_hip_merge for P = T*H rows and M remote
 * partials (-1 for bad sizes).  Shape query; no reference counterpart. */
int64_t moba_hip_merge_work(int64_t P, int64_t M);

/* ----------------------------------------------------------------- decode */

/* Number of work-list entries decode_route emits per (query, kv head, block
 * of 16 q heads): (Hq / Hkv) * nslot.  Each entry is 16 bytes (int4: chunk,
 * head mask, 4-bit slot indices of heads 0-7, of heads 8-15). */
int moba_hip_decode_work_items(int Hq, int Hkv, int nslot);

/* Scatter N new tokens k/v [N,Hkv,D] into the page pool
 * k_cache/v_cache [num_pages, page_size, Hkv, D] at (token_seq[n], token_pos[n])
 * through table [B, table_width] (physical page per logical page).
 * Replaces _append_kernel (src/moba_opt/ops/paged_decode.py:10-23). */
int moba_hip_paged_append(const void* k, const void* v, int dtype, int N, int Hkv, int D,
                          void* k_cache, void* v_cache, int page_size, const int* table,
                          int table_width, const int* token_seq, const int* token_pos,
                          void* stream);

/* Key means of closed chunks into means [B, max_chunks, Hkv, D] (cache dtype):
 * canonical fp32 sum (64 strided partial sums, then a fixed pairwise tree),
 * / chunk, for chunk in [1, 1024].  mode 0: item i = (item_seq[i], chunk
 * item_chunk_or_pos[i]); mode 1: item i = query row at position p, closing
 * chunk p / chunk only when (p + 1) % chunk == 0.
 * Replaces _closed_means_kernel (paged_decode.py:26-44) and _step_means
 * (src/moba_opt/ops/prepared_decode.py:23-41). */
int moba_hip_block_means(const void* k_cache, int dtype, int Hkv, int D, int page_size,
                         const int* table, int table_width, const int* item_seq,
                         const int* item_chunk_or_pos, int n_items, int mode, int chunk,
                         void* means, int max_chunks, void* stream);

/* Route of decode queries q [Nq,Hq,D]: fp32 fma-chain scores against the means
 * of the closed chunks c with (c+1)*chunk <= pos, stable top-R (descending,
 * ties -> lowest chunk).  selected [Nq,Hq,1+R]: slot 0 = pos / chunk, then the
 * chosen chunks, -1 padded.  scores [Nq,Hq,width] (required when R > 0; -inf
 * for illegal chunks; width <= 8192).  work_items (nullable)
 * [Nq*Hkv*ceil(G/16), moba_hip_decode_work_items(Hq,Hkv,R+1)] int4 and
 * work_counts [Nq*Hkv*ceil(G/16)]: per 16-head block the union of the chosen
 * chunks for paged_attention.  At most 64 q heads per kv head.
 * Replaces _route_kernel + torch.topk / _stable_topk + _selected
 * (paged_decode.py:47-64, src/moba_opt/kv_cache.py:208-223,
 * prepared_decode.py:44-88). */
int moba_hip_decode_route(const void* q, int dtype, int Nq, int Hq, int Hkv, int D,
                          const void* means, int max_chunks, const int* q_seq, const int* q_pos,
                          int chunk, int width, int R, float* scores, int* selected,
                          void* work_items, int* work_counts, void* stream);

/* Paged attention of q [Nq,Hq,D] over the selected chunks (selected
 * [Nq,Hq,nslot] + the route work list) or, with dense != 0, over every token
 * <= pos; tokens are read through the page table, each selected page once per
 * 16-head block of a KV-head group.  max_chunks_bound (dense) bounds
 * pos / chunk + 1.  part_o [Nq*Hq*S, D] and part_ml [Nq*Hq*S, 2] fp32
 * (S = nslot, or max_chunks_bound when dense) are workspaces.
 * out [Nq,Hq,D] (dtype), lse [Nq,Hq] fp32 natural log.
 * Replaces _attention_kernel (paged_decode.py:67-112). */
int moba_hip_paged_attention(const void* q, int dtype, int Nq, int Hq, int Hkv, int D,
                             const void* k_cache, const void* v_cache, int page_size,
                             const int* table, int table_width, const int* lengths,
                             const int* q_seq, const int* q_pos, const int* selected, int nslot,
                             const void* work_items, const int* work_counts, int dense,
                             int chunk, int max_chunks_bound, float* part_o, float* part_ml,
                             void* out, float* lse, void* stream);

/* Prepared-decode metadata step for B fixed rows: apply the page-table delta
 * [2,B] (logical, physical; -1 = none), write positions = lengths (append) or
 * lengths - 1, and advance lengths when append != 0.
 * Replaces _metadata (prepared_decode.py:6-20). */
int moba_hip_decode_metadata(int* table, int table_width, int* lengths, const int* ids,
                             int* positions, const int* delta, int B, int append, void* stream);

/* Prepared-decode step prologue in ONE launch for B fixed rows: apply the
 * page-table delta, positions = lengths, lengths += 1, scatter the new token
 * k/v [B,Hkv,D] into the pool, and, for a row whose token closes its chunk,
 * write that chunk's mean (same canonical order as moba_hip_block_means); chunk in [1, 1024].
 * Replaces _metadata + _append_kernel + _step_means
 * (prepared_decode.py:6-41, paged_decode.py:10-23). */
int moba_hip_decode_step(int* table, int table_width, int* lengths, const int* ids,
                         int* positions, const int* delta, int B, const void* k, const void* v,
                         int dtype, void* k_cache, void* v_cache, int page_size, int Hkv, int D,
                         int chunk, void* means, int max_chunks, void* stream);

/* Virtual kv heads per kv head of moba_hip_decode_fused: the fewest Vg that
 * cut the Hq/Hkv q heads of a kv head into equal groups of at most 16 (1 up
 * to 16 q heads per kv head, 2 up to 32, ...); 0 when Hq is not a multiple
 * of Hkv.  The reference's kernel takes any group size in one program per
 * (query, q head) (paged_decode.py:67-112); here a group of at most 16 q
 * heads shares one pass over the K/V the group selected. */
int moba_hip_decode_fused_groups(int Hq, int Hkv);

/* 1 when moba_hip_decode_fused handles this shape: Hq a multiple of Hkv, D a
 * multiple of 8 in [8,256], and a route width and page-table width
 * (table_width entries per row, staged in LDS) whose scratch fits the
 * launch's 64 KiB of dynamic LDS. */
int moba_hip_decode_fused_supported(int Hq, int Hkv, int D, int width, int table_width);

/* Whole decode for Nq query rows (one query per row), two launches on the
 * stream: routing (scores over the closed chunks c < min(pos / chunk, width),
 * stable top-R per q head, selected [Nq,Hq,R+1] with slot 0 = pos / chunk, -1
 * pad; not written when dense) and the paged attention over the union of the
 * heads' chunks into S split partials, then their merge into out [Nq,Hq,D]
 * and lse [Nq,Hq] fp32 natural log.
 * pos_mode 0: positions [Nq] are given (read only; no table, length or pool
 *             change).
 * ids [Nq] maps rows to cache slots (pos_mode 1 and 2); null means row i is
 *             slot i, which saves the kernel a dependent load before the
 *             position is known.
 * pos_mode 1: position = lengths[ids[row]] - 1 (prepared attend); the
 *             page-table delta [2,Nq] (logical, physical; -1 = none; may be
 *             null) is applied; positions written.
 * pos_mode 2: position = lengths[ids[row]] (prepared step): as mode 1, plus the
 *             new token k/v [Nq,Hkv,D] is scattered into the pool, the mean of
 *             the chunk it closes is written to means (canonical order, as
 *             moba_hip_block_means), and lengths advance by one.
 * The workgroups of a row are laid out per virtual kv head: Hv = Hkv * Vg
 * (Vg = moba_hip_decode_fused_groups(Hq, Hkv)), virtual head u serving q
 * heads u*G .. u*G+G-1 (G = Hq/Hv) against physical kv head u / Vg.
 * splits S in [1,64] workgroups per (row, virtual kv head), or, with a
 * schedule sched (may be null), at most S: sched holds n_sched workgroup
 * entries (row * Hv + virtual head, split, splits of that row), every split of
 * every (row, virtual head) exactly once, followed by the Nq*Hv split counts.
 * Workspaces part_o [Nq*Hq*S, D] and part_ml [Nq*Hq*S, 2] fp32.  width must
 * be >= max(position) / chunk.  Outputs are deterministic for a fixed
 * schedule.
 * Replaces _metadata + _append_kernel + _step_means + _route_kernel + top-k +
 * _selected + _attention_kernel (prepared_decode.py:6-94, paged_decode.py:10-112). */
int moba_hip_decode_fused(const void* q, const void* k, const void* v, int dtype, int Nq, int Hq,
                          int Hkv, int D, void* k_cache, void* v_cache, int page_size, int* table,
                          int table_width, int* lengths, const int* ids, int* positions,
                          const int* delta, void* means, int max_chunks, int chunk, int width,
                          int R, int dense, int pos_mode, int splits, const int* sched,
                          int n_sched, int* selected, float* part_o, float* part_ml, void* out,
                          float* lse, void* stream);

/* Decode attention for callers that cannot allocate (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same as moba_hip_decode_fused with
 * pos_mode 0 (positions given; nothing in the cache changes) and the uniform
 * split count S = clamp(ceil(256 / (Nq*Hv)), 1, 64), but the split partials
 * live in a static per-device scratch array of 8 MiB instead of caller
 * workspaces: calls needing more than Nq*Hq*S*(D+2)*4 (+256) bytes fail
 * with MOBA_ERR_CAPACITY before launching anything.  It calls no allocating
 * routine.  Every call on a device shares that device's scratch: calls that
 * overlap on one device (different streams, or different host threads)
 * race; calls serialised on one stream do not. */
int moba_hip_decode_attend_noalloc(const void* q, int dtype, int Nq, int Hq, int Hkv, int D,
                                   const void* k_cache, const void* v_cache, int page_size,
                                   const int* table, int table_width, const int* lengths,
                                   const int* ids, const int* positions, const void* means,
                                   int max_chunks, int chunk, int width, int R, int dense,
                                   int* selected, void* out, float* lse, void* stream);

/* ------------------------------------------------ host page pool (CPU only)
 *
 * The page allocator of the paged KV cache as a host object (no device
 * calls; usable without a GPU).  Replaces PageAllocator / IncrementalLayout
 * (src/moba_opt/cache_layout.py:23-148) with the same observable behaviour:
 * a LIFO free-page stack whose initial order hands out page 0 first, reset
 * pushing a slot's pages back in logical order, transactional plans (a
 * failed plan changes nothing; commit refuses a plan older than the pool with
 * MOBA_ERR_STALE), and O(rows) decode steps.  Messages of MOBA_ERR_ARG are
 * the reference's ValueError messages.  A pool is not thread-safe: callers
 * serialise access (the Python cache holds its lock). */

/* New pool of `batch` slots, table width ceil(max_seq_len / page_size). */
int moba_pool_create(int batch, int max_seq_len, int page_size, int num_pages, int chunk,
                     void** pool);
void moba_pool_destroy(void* pool);
/* Independent copy (the prepared-decode lease, cache_layout.py:108-114). */
int moba_pool_clone(const void* pool, void** out);
/* dst takes src's state (same shapes); views of dst stay valid
 * (the lease's publish, cache_layout.py:143-148). */
int moba_pool_assign(void* dst, const void* src);
/* info[8] = batch, max_seq_len, page_size, num_pages, chunk, table width,
 * version, free page count. */
int moba_pool_info(const void* pool, int64_t* info);
/* Views of the pool's storage (valid for the pool's lifetime):
 * table [batch][width] (-1 = unmapped), lengths [batch], free stack
 * [free count] (bottom first; the last entry is handed out next). */
const int32_t* moba_pool_table(const void* pool);
const int32_t* moba_pool_lengths(const void* pool);
const int32_t* moba_pool_free(const void* pool);
/* Reorders the free stack (a permutation of the current free pages), e.g.
 * the seeded fragmented pool of benchmarks/benchmark_prepared.py:79-81. */
int moba_pool_set_free(void* pool, const int32_t* pages, int n);
/* 0 when ids[n] are valid slot ids (nonempty; unique if `unique`). */
int moba_pool_check_ids(const void* pool, const int32_t* ids, int n, int unique);
/* Plans appending counts[i] tokens to slot ids[i] without changing the pool
 * (PageAllocator.plan_append, cache_layout.py:54-87): token_seq/token_pos
 * [sum counts] (nullable), closed (slot, chunk) pairs [2*closed_cap] of the
 * chunks the append completes, grants (slot, logical page, physical page)
 * [3*grants_cap] taken from the top of the free stack in order, and the new
 * length of every slot.  *version identifies the pool state planned on. */
int moba_pool_plan_append(const void* pool, const int32_t* ids, const int32_t* counts, int n,
                          int32_t* token_seq, int32_t* token_pos, int32_t* closed,
                          int closed_cap, int* n_closed, int32_t* grants, int grants_cap,
                          int* n_grants, int32_t* new_lengths, int64_t* version);
/* Installs a plan of moba_pool_plan_append (PageAllocator.commit,
 * cache_layout.py:89-93); MOBA_ERR_STALE unless the pool is unchanged since. */
int moba_pool_commit_append(void* pool, const int32_t* ids, int n, const int32_t* new_lengths,
                            const int32_t* grants, int n_grants, int64_t version);
/* Frees the pages of slots ids[n] and empties them (PageAllocator.reset,
 * cache_layout.py:95-103); nothing changes on an error. */
int moba_pool_reset(void* pool, const int32_t* ids, int n);
/* Plans one token for each slot ids[n] (IncrementalLayout.plan,
 * cache_layout.py:116-127): positions[n] (nullable) = current lengths, and
 * delta [2][n] = (logical page, physical page) for a row whose position
 * starts a page, else (-1, -1); *n_grants rows take a page. */
int moba_pool_plan_step(const void* pool, const int32_t* ids, int n, int32_t* positions,
                        int32_t* delta, int* n_grants, int64_t* version);
/* Installs a step plan (IncrementalLayout.commit, cache_layout.py:129-137). */
int moba_pool_commit_step(void* pool, const int32_t* ids, int n, const int32_t* delta,
                          int64_t version);

/* ------------------------------------------------- prepared-decode driver
 *
 * The host side of PreparedDecode.step / .attend / .capture
 * (src/moba_opt/prepared_decode.py:99-187) in native code: per call it plans
 * one token per leased slot on a page-pool lease (moba_pool_clone of the
 * cache's pool), stages the page-table delta of rows that start a page
 * through pinned memory onto the device (no host synchronisation), refreshes
 * the fused kernel's split schedule when rows moved by more than 1/8, launches
 * the step (moba_hip_decode_fused, the multi-kernel sequence, or one
 * hipGraphLaunch of the captured launches) and commits the plan.  All device
 * buffers belong to the caller and must outlive the handle; the driver owns
 * only pinned staging memory, events and graphs. */
typedef struct MobaPrepDesc {
  int dtype, rows, hq, hkv, head_dim, page_size, table_width, max_chunks, chunk, width, remote;
  int dense;    /* 1: attend every token <= pos */
  int fused;    /* 1: moba_hip_decode_fused; 0: step/metadata + route + paged_attention */
  int splits;   /* fused: split cap (<= 64) */
  int n_sched;  /* fused: workgroups of the schedule (moba_prep_sched_workgroups) */
  void* lease;  /* page pool the driver plans on (caller-owned) */
  const void *q, *k, *v;          /* [rows,Hq,D], [rows,Hkv,D] inputs */
  void *k_cache, *v_cache;        /* [num_pages,page,Hkv,D] */
  int *table, *lengths;           /* [B,table_width], [B] */
  const int* ids_dev;             /* [rows] slot ids */
  int *positions, *delta;         /* [rows], [2,rows] */
  void* means;                    /* [B,max_chunks,Hkv,D] */
  int* selected;                  /* [rows,Hq,remote+1] (null when dense) */
  float* scores;                  /* multi-kernel route scores [rows,Hq,width] */
  void* items; int* item_counts;  /* multi-kernel route work list */
  float *part_o, *part_ml;        /* split (fused) or slot partials */
  void* out; float* lse;          /* [rows,Hq,D], [rows,Hq] */
  int* sched;                     /* fused schedule [3*n_sched + rows*Hkv] (nullable) */
} MobaPrepDesc;

/* Driver for slots ids[desc->rows]. */
int moba_prep_create(const MobaPrepDesc* desc, const int32_t* ids, void** handle);
void moba_prep_destroy(void* handle);
/* One step (append != 0: a token per slot, k/v of the descriptor) or attend
 * on `stream`; positions[rows] receives each row's position.  use_graph
 * replays the graph of moba_prep_capture.  Input errors change nothing. */
int moba_prep_run(void* handle, int append, int use_graph, void* stream, int32_t* positions);
/* The three parts of moba_prep_run, for callers that put the launches of
 * several layers into one stream sequence or one captured graph (a model
 * decode step):  plan stages this call's page-table delta and schedule on
 * `stream` and fills positions (host work; never inside a capture);
 * launch enqueues the device work (capturable when use_graph is 0); commit
 * installs the planned token in the lease (after the launches). */
int moba_prep_plan(void* handle, int append, void* stream, int32_t* positions);
int moba_prep_launch(void* handle, int append, int use_graph, void* stream);
int moba_prep_commit(void* handle);
/* Captures the launches of a step / attend into a hipGraph (nothing runs;
 * no state changes). */
int moba_prep_capture(void* handle, int append, void* stream);
/* Steps whose page-table delta was uploaded. */
int64_t moba_prep_delta_uploads(const void* handle);
/* Workgroups of a fused schedule: max(rows*hkv, min(workgroups, rows*hkv*max_splits)). */
int moba_prep_sched_workgroups(int rows, int hkv, int workgroups, int max_splits);
/* Split counts per (row, kv head) by the expected attended
 * tokens plus the route each workgroup recomputes (each extra workgroup to
 * the row with the most route + expected tokens per split, each count in
 * [1, max_splits]) over
 * moba_prep_sched_workgroups workgroups: entries [3*n + rows*hkv] =
 * (row*hkv + kv head, split, splits) interleaved across rows, then the
 * counts; splits[rows*hkv] (nullable) the counts.  No counterpart in the
 * reference (its decode kernel has one program per (query, q head)). */
int moba_prep_schedule(const int32_t* positions, int rows, int hkv, int group, int remote,
                       int chunk, int dense, int workgroups, int max_splits, int32_t* entries,
                       int32_t* splits);

#ifdef __cplusplus
}
#endif
#endif /* MOBA_HIP_H */
