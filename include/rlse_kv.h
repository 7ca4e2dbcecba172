/*
 * rlse_kv.h -- C ABI of the MI355X (gfx950) paged KV-cache hot path of the
 * rlse serving engine (crate `rlse` 0.2.0).
 *
 * Conventions (carried over from the reference's FFI precedent,
 * docs/colab_cuda_kernels/mini_serve_kernels.cu:247-296):
 *   - every entry point returns an int status: 0 on success, a hipError_t
 *     value (1 = hipErrorInvalidValue for rejected arguments) or an
 *     RLSE_ERR_* code >= 10000; nothing ever exits or aborts the process;
 *   - device buffers are owned by the caller unless a *_create call says
 *     otherwise; all device work is asynchronous on the given stream
 *     (NULL = the default stream) and nothing synchronises;
 *   - arguments are validated before any device work is queued (fail closed);
 *   - handles are not internally locked: the caller serialises, as the
 *     reference's backend mutex does (src/backends/candle.rs:385).
 *
 * Physical KV pool layout, per layer, for both K and V (the reference
 * prototype's index formula, mini_serve_kernels.cu:68-70, 93):
 *     pool[num_blocks][num_kv_heads][16][head_dim]
 *     elem(block, head, slot, dim) = ((block*Hkv + head)*16 + slot)*head_dim + dim
 * A sequence's token t lives in block block_table[t / 16], slot t % 16.
 * Block tables are int32 [batch][max_blocks_per_seq], row-major.
 */
#ifndef RLSE_KV_H
#define RLSE_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* rlse_stream_t; /* a hipStream_t */

enum rlse_dtype { RLSE_DTYPE_F32 = 0, RLSE_DTYPE_BF16 = 1, RLSE_DTYPE_F16 = 2 };

#define RLSE_OK 0
#define RLSE_ERR_INVALID_VALUE 1 /* == hipErrorInvalidValue */
#define RLSE_ERR_CACHE_PRESSURE 10001
#define RLSE_ERR_UNKNOWN_REQUEST 10002
#define RLSE_ERR_BUFFER_TOO_SMALL 10003
#define RLSE_ERR_TOKEN_LIMIT 10004 /* EngineError::TokenLimitExceeded */
#define RLSE_ERR_DEVICE_TIMEOUT 10005 /* a merge on the device gave up waiting */
#define RLSE_BLOCK_SIZE 16 /* src/core/constants.rs:1 DEFAULT_BLOCK_SIZE */

/* Message of the last failing call on this thread ("" if none). */
const char* rlse_last_error(void);
/* Library ABI version (major*10000 + minor*100 + patch). */
int rlse_version(void);

/* ------------------------------------------------------------------ */
/* Device-side failures. Kernels that hand partial results between     */
/* workgroups (decode, the K-split projections) raise sticky flags in  */
/* word 0 of their workspace instead of failing silently:              */
/*   RLSE_WS_ERR_MERGE_TIMEOUT: a merge gave up waiting for a partial  */
/*     (the affected output rows are NaN);                              */
/*   RLSE_WS_ERR_LENGTH: a sequence length exceeded its block table    */
/*     (max_blocks_per_seq*16); its output row is zeros and nothing was */
/*     appended for it.                                                 */
/*   RLSE_WS_ERR_PREFIX: a cascade step's batch broke its contract (a   */
/*     sequence's first prefix_pages table entries differ from sequence */
/*     0's, or its new token lies inside them); the step's outputs are  */
/*     not its attention.                                               */
/* The reference turns a failed step into BackendError and quarantines */
/* the backend (src/backends/candle.rs:689-696); a caller maps a       */
/* nonzero rlse_workspace_check to the same.                           */
/* ------------------------------------------------------------------ */
#define RLSE_WS_ERR_MERGE_TIMEOUT 1u
#define RLSE_WS_ERR_LENGTH 2u
#define RLSE_WS_ERR_PREFIX 4u
/* Synchronises stream, then reads and clears the flags of a decode or
 * projection workspace (NULL: the library's own decode workspaces of the
 * current device -- the one used by calls without a workspace and the
 * static one of rlse_decode_step_noalloc). *flags (may be NULL) receives
 * them. Returns
 * RLSE_ERR_DEVICE_TIMEOUT if a merge timed out, else RLSE_ERR_TOKEN_LIMIT
 * if a length exceeded its table, else RLSE_ERR_INVALID_VALUE if a cascade
 * step's batch broke its contract, else 0 (or a hip error). No counterpart
 * in the reference: its CPU/Candle ops return errors synchronously. */
int rlse_workspace_check(void* workspace, rlse_stream_t stream, unsigned* flags);
/* Bound on a merge's wait for an earlier workgroup's partial, in
 * nanoseconds, for launches queued after the call (default 100 ms; 0 =
 * give up at the first miss). Process-wide. Meant for tests of the failure
 * path: every kernel still ends normally. */
int rlse_set_merge_wait_ns(unsigned long long ns);

/* ------------------------------------------------------------------ */
/* Physical paged KV pool (device memory owned by the handle).         */
/* Replaces the per-request contiguous candle_nn KvCache buffers that  */
/* Attention::append_kv creates (src/backends/qwen2.rs:349-361) and    */
/* sizes in ModelForCausalLM::set_kv_capacity (qwen2.rs:603-618).      */
/* One block id spans all layers, as a KVCache id does                 */
/* (src/cache/kv_cache.rs:15-35). The pool is zero-filled at creation. */
/* ------------------------------------------------------------------ */
typedef struct rlse_kv_pool rlse_kv_pool;

int rlse_pool_create(int num_layers, int num_blocks, int num_kv_heads, int head_dim,
                     int dtype, int block_size, rlse_kv_pool** out_pool);
int rlse_pool_destroy(rlse_kv_pool* pool);
/* Device pointers of one layer's K and V pools. */
int rlse_pool_layer(const rlse_kv_pool* pool, int layer, void** k_pool, void** v_pool);
/* Elements between consecutive layers' K (and V) pools. */
int rlse_pool_info(const rlse_kv_pool* pool, int* num_layers, int* num_blocks,
                   int* num_kv_heads, int* head_dim, int* dtype,
                   long long* layer_stride_elems);

/* ------------------------------------------------------------------ */
/* KV data movement (bit-exact).                                       */
/* ------------------------------------------------------------------ */

/* Append num_tokens new K/V rows ([num_tokens][Hkv][head_dim] each) at
 * the given positions. Token i belongs to sequence seq_index[i]
 * (seq_index == NULL: token i belongs to sequence i) and is written to
 * block block_tables[seq][pos/16], slot pos%16. block_tables has num_seqs
 * rows; tokens whose sequence is outside [0, num_seqs) are skipped.
 * Replaces Attention::append_kv -> KvCache::append (src/backends/qwen2.rs:349-361),
 * i.e. slice_set into the contiguous buffer at cur_len. Tokens whose block
 * id is outside [0, num_blocks) or whose position is outside
 * [0, max_blocks_per_seq*16) are skipped. */
int rlse_kv_append(const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                   const int32_t* block_tables, int num_seqs, const int32_t* seq_index,
                   const int32_t* positions, int num_tokens, int num_kv_heads,
                   int head_dim, int max_blocks_per_seq, int num_blocks, int dtype,
                   rlse_stream_t stream);

/* Checksums of the pool's rows: for every (sequence, KV head) row of the
 * block tables, the sum mod 2^32 over its attended positions t < seq_lens[b]
 * and the 32-bit words j of a position's head_dim elements of
 *     (w ^ (t * 0x9E3779B1 + j * 0x85EBCA77)) * 0xC2B2AE3D,
 * K then V: ADDED into out [batch][num_kv_heads][2] (zero-fill it first; a
 * caller may accumulate several layers). Pages whose id lies outside
 * [0, num_blocks) contribute nothing; a length beyond the table's capacity
 * counts as 0. No counterpart in the reference, whose tests compare snapshot
 * buffers byte for byte on the host (src/backends/candle.rs:1281-1292): the
 * sums compare a pool with its expected contents without copying it back.
 * The launch splits the pages as the paged decode does, one page in flight
 * per wave, and does nothing else, so its duration is the time a decode
 * launch of that shape needs to read its K/V bytes. */
int rlse_kv_checksum(const void* k_pool, const void* v_pool, const int32_t* block_tables,
                     const int32_t* seq_lens, int batch, int num_kv_heads, int head_dim,
                     int max_blocks_per_seq, int num_blocks, int dtype, uint32_t* out,
                     rlse_stream_t stream);

/* The same sums, each wave's first page requested from plan (rlse_decode_plan
 * of the same tables and lengths, 16-byte aligned) before the launch builds
 * its block prefix, as a planned decode launch does: the read ceiling of
 * rlse_decode_step_planned. A plan of another step shape (a cascade or
 * grouped plan) is ignored and the walk builds its own descriptors; the
 * sums are the same either way. No counterpart in the reference. */
int rlse_kv_checksum_planned(const void* k_pool, const void* v_pool,
                             const int32_t* block_tables, const int32_t* seq_lens, int batch,
                             int num_kv_heads, int head_dim, int max_blocks_per_seq,
                             int num_blocks, int dtype, const void* plan, uint32_t* out,
                             rlse_stream_t stream);

/* Snapshot export: pool pages -> contiguous [num_layers][Hkv][len][head_dim]
 * K and V, the layout of Attention::get_kv_snapshot views and of the
 * cumulative prefix snapshots (src/backends/qwen2.rs:363-371;
 * src/cache/prefix_cache.rs:320-333). Layer l's pools are k_pool/v_pool +
 * l*layer_stride_elems. block_table is a device int32 array. */
int rlse_kv_gather(const void* k_pool, const void* v_pool, long long layer_stride_elems,
                   int num_layers, const int32_t* block_table, int len, void* k_out,
                   void* v_out, int num_kv_heads, int head_dim, int num_blocks, int dtype,
                   rlse_stream_t stream);

/* Snapshot restore: contiguous [num_layers][Hkv][len][head_dim] K/V ->
 * positions start..start+len-1 of the sequence whose table is block_table.
 * Replaces Attention::set_kv_snapshot (src/backends/qwen2.rs:373-377). */
int rlse_kv_scatter(const void* k_in, const void* v_in, void* k_pool, void* v_pool,
                    long long layer_stride_elems, int num_layers,
                    const int32_t* block_table, int start, int len, int num_kv_heads,
                    int head_dim, int num_blocks, int dtype, rlse_stream_t stream);

/* Copy-on-write: copy whole blocks src_blocks[i] -> dst_blocks[i] (device
 * int32 arrays) in every layer's K and V pools. Replaces the per-fork
 * snapshot copy of Model::set_kv_snapshot (src/backends/qwen2.rs:547-574)
 * for the last partial block; full blocks are shared by refcount instead. */
int rlse_kv_copy_blocks(void* k_pool, void* v_pool, long long layer_stride_elems,
                        int num_layers, const int32_t* src_blocks,
                        const int32_t* dst_blocks, int num_pairs, int num_kv_heads,
                        int head_dim, int num_blocks, int dtype, rlse_stream_t stream);

/* ------------------------------------------------------------------ */
/* GQA decode attention over the paged pool.                           */
/* q [batch][num_heads][head_dim], out same shape; query head h uses KV */
/* head h / (num_heads/num_kv_heads) (src/backends/qwen2.rs:192).       */
/* seq_lens[b] = keys attended (cached + appended). Result is          */
/* softmax(q K^T * scale) V per head, as decode_attention_gqa_zero_copy */
/* (src/backends/qwen2.rs:177-203) computes on contiguous buffers.     */
/* Rows with seq_len <= 0 produce zeros. A row with seq_len above      */
/* max_blocks_per_seq*16 is invalid: it produces zeros, nothing is     */
/* appended for it and RLSE_WS_ERR_LENGTH is raised in the workspace.  */
/* Blocks with ids outside [0, num_blocks) are not read and contribute */
/* nothing.                                                            */
/* ------------------------------------------------------------------ */

/* Bytes of split-K workspace needed by rlse_paged_gqa_decode on the
 * current device. */
int rlse_decode_workspace_size(int batch, int num_heads, int num_kv_heads, int head_dim,
                               size_t* bytes);

/* Split-K decode in one launch. workspace may be NULL, in which case a
 * library-owned per-device workspace is used (allocated and zero-filled on
 * first need). A caller workspace must be zero-filled once before its first
 * use and then left to the library: it holds sticky error flags
 * (rlse_workspace_check), per-wave launch counters and epoch-tagged
 * partial records, which never need clearing. One workspace serves calls
 * of any shape on its device. Launches that share a workspace, the
 * library-owned one included, must be ordered (same stream). */
int rlse_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, const int32_t* seq_lens, void* out,
                          int batch, int num_heads, int num_kv_heads, int head_dim,
                          int max_blocks_per_seq, int num_blocks, float scale, int dtype,
                          void* workspace, size_t workspace_bytes, rlse_stream_t stream);

/* Fused decode step of one layer: the front half of Attention::forward
 * and its decode branch (src/backends/qwen2.rs:291-328) in one launch.
 * For every sequence b the new token sits at position p = seq_lens[b]-1:
 * q [batch][num_heads][head_dim] and k_new/v_new [batch][num_kv_heads]
 * [head_dim] are the raw projections; q and k get q_norm/k_norm RMSNorm
 * (skipped when the weight is NULL, as for Qwen2) and NeoX RoPE at p; the
 * rotated k and raw v are appended to the pool at p; out receives the
 * attention over the seq_lens[b] keys, as rlse_paged_gqa_decode would give
 * after rlse_qk_norm_rope_append. cos/sin tables are [max_pos][head_dim/2]
 * with max_pos >= max_blocks_per_seq*16. Workspace rules as for
 * rlse_paged_gqa_decode. */
int rlse_decode_step(const void* q, const void* k_new, const void* v_new,
                     const void* q_norm_weight, const void* k_norm_weight, float eps,
                     const void* cos_table, const void* sin_table, int max_pos, void* k_pool,
                     void* v_pool, const int32_t* block_tables, const int32_t* seq_lens,
                     void* out, int batch, int num_heads, int num_kv_heads, int head_dim,
                     int max_blocks_per_seq, int num_blocks, float scale, int dtype,
                     void* workspace, size_t workspace_bytes, rlse_stream_t stream);

/* Per-step plan for rlse_decode_step_planned: the first block descriptors
 * of every wave of a decode launch (page id, valid rows, row, new-token
 * position) and the new-token positions of the rows its first query stage
 * covers, computed once from the step's block tables and lengths instead
 * of by every layer's launch. No counterpart in the reference: its decode
 * runs per sequence on contiguous buffers, with no page tables to walk.
 * plan: rlse_decode_plan_size bytes, 16-byte aligned. */
int rlse_decode_plan_size(size_t* bytes);
int rlse_decode_plan(const int32_t* block_tables, const int32_t* seq_lens, int batch,
                     int num_kv_heads, int max_blocks_per_seq, int num_blocks, void* plan,
                     size_t plan_bytes, rlse_stream_t stream);
/* rlse_decode_step with a plan that rlse_decode_plan built from the same
 * block_tables, seq_lens, batch, num_kv_heads, max_blocks_per_seq and
 * num_blocks (every layer of a decode step shares them): each wave's page
 * ids then arrive with its first load, its query and append loads go out
 * next and its first pages right after. Results are identical to rlse_decode_step's.
 * The plan carries a stamp of the step shape it was built for (plain, a
 * cascade's prefix_pages, prefix groups); a planned launch given a plan of
 * another shape raises RLSE_WS_ERR_PREFIX in the workspace.
 * flags: RLSE_DECODE_STREAM when no page of the batch is read by more than
 * one row (no sequence shares pages with another -- the caller's block
 * manager knows: no page with a refcount above 1): the pages are then read
 * with non-temporal loads that keep the per-launch data in the caches.
 * Without it (e.g. sequences forked from one cached prefix) the pages stay
 * cacheable, so a page read by many rows is served from the caches. Either
 * way the results are the same. */
#define RLSE_DECODE_STREAM 1
int rlse_decode_step_planned(const void* q, const void* k_new, const void* v_new,
                             const void* q_norm_weight, const void* k_norm_weight, float eps,
                             const void* cos_table, const void* sin_table, int max_pos,
                             void* k_pool, void* v_pool, const int32_t* block_tables,
                             const int32_t* seq_lens, void* out, int batch, int num_heads,
                             int num_kv_heads, int head_dim, int max_blocks_per_seq,
                             int num_blocks, float scale, int dtype, void* workspace,
                             size_t workspace_bytes, const void* plan, int flags,
                             rlse_stream_t stream);

/* Shared-prefix (cascade) decode step. No counterpart in the reference: its
 * decode attends every sequence's keys separately (src/backends/qwen2.rs:
 * 177-203), also when sequences were forked from one cached prefix
 * (src/backends/candle.rs:437-478). When the first prefix_pages entries of
 * every block table are the same pages and every new token lies past them
 * (seq_lens[b] - 1 >= 16 * prefix_pages), the prefix's keys are attended
 * once for all sequences -- a matrix-core tile of 16 query heads per KV head
 * -- into prefix_buf, and the decode launch that follows streams only each
 * sequence's own pages and combines the two softmax states per row. Same
 * arguments and results as rlse_decode_step_planned (within rounding: the
 * order of the sums over the keys changes), with a plan from
 * rlse_decode_plan_cascade for the same prefix_pages (or NULL: the
 * descriptors are derived in the launch, as in rlse_decode_step).
 * bf16/f16 only; 0 <= prefix_pages <= min(max_blocks_per_seq, 512), 0 being
 * the plain step. prefix_buf: rlse_decode_prefix_size bytes for the same
 * batch, num_heads, head_dim and prefix_pages, 16-byte aligned, overwritten
 * by every call (calls sharing one must be ordered: same stream). Pages of
 * the prefix are read by one workgroup per slice of about 16 pages and 16
 * query heads, in a launch ahead of the decode launch; the decode combines
 * the slices' states into each row. A batch that breaks the contract
 * raises RLSE_WS_ERR_PREFIX in the workspace; its outputs are then not its
 * attention. With a plan the contract is checked once, by
 * rlse_decode_plan_cascade (the plan carries its verdict), instead of by
 * every layer's launch. */
int rlse_decode_prefix_size(int batch, int num_heads, int head_dim, int prefix_pages,
                            size_t* bytes);
int rlse_decode_plan_cascade(const int32_t* block_tables, const int32_t* seq_lens, int batch,
                             int num_kv_heads, int max_blocks_per_seq, int num_blocks,
                             int prefix_pages, void* plan, size_t plan_bytes,
                             rlse_stream_t stream);
int rlse_decode_step_cascade(const void* q, const void* k_new, const void* v_new,
                             const void* q_norm_weight, const void* k_norm_weight, float eps,
                             const void* cos_table, const void* sin_table, int max_pos,
                             void* k_pool, void* v_pool, const int32_t* block_tables,
                             const int32_t* seq_lens, void* out, int batch, int num_heads,
                             int num_kv_heads, int head_dim, int max_blocks_per_seq,
                             int num_blocks, float scale, int dtype, void* workspace,
                             size_t workspace_bytes, const void* plan, int flags,
                             int prefix_pages, void* prefix_buf, size_t prefix_bytes,
                             rlse_stream_t stream);

/* Cascade decode step of a mixed batch: several prefix groups and unforked
 * sequences in one step. The batch the reference decodes in one
 * step_decode_batch (src/backends/qwen2.rs:628-764) holds sequences restored
 * from different cached prefixes and sequences with none
 * (src/backends/candle.rs:437-478, 602-640); here each group's shared pages
 * are attended once for its members and every other page once for its
 * sequence. seq_group (device int32 [batch]): the group of each sequence, -1
 * for none (its whole table is streamed). group_pages (device int32
 * [num_groups]): the number of leading table entries every member of group
 * g shares with the group's other members (the same pages, and each
 * member's new token lies past them), 1 .. min(max_blocks_per_seq, 512).
 * Members may sit anywhere in the batch. rlse_decode_plan_groups builds the
 * step's plan (one per step, read by every layer; required), including the
 * member lists and the prefix launch's work items (one per group column
 * tile and prefix slice); rlse_decode_step_groups then runs the prefix
 * launch over those items and the decode, with
 * max_group_pages >= every group's pages sizing both and prefix_buf
 * (rlse_decode_prefix_size with prefix_pages = max_group_pages). 1 <=
 * num_groups <= 64; num_heads / num_kv_heads <= 8; bf16/f16 only. Same
 * results as rlse_decode_step_planned within rounding. A group id or page
 * count out of range, a member whose leading entries differ from its
 * group's, a new token inside its group's pages, or a plan built for
 * another step shape (another group count or group size included) raise
 * RLSE_WS_ERR_PREFIX. */
int rlse_decode_plan_groups(const int32_t* block_tables, const int32_t* seq_lens,
                            const int32_t* seq_group, const int32_t* group_pages, int num_groups,
                            int batch, int num_heads, int num_kv_heads, int max_blocks_per_seq,
                            int num_blocks, void* plan, size_t plan_bytes, rlse_stream_t stream);
int rlse_decode_step_groups(const void* q, const void* k_new, const void* v_new,
                            const void* q_norm_weight, const void* k_norm_weight, float eps,
                            const void* cos_table, const void* sin_table, int max_pos,
                            void* k_pool, void* v_pool, const int32_t* block_tables,
                            const int32_t* seq_lens, void* out, int batch, int num_heads,
                            int num_kv_heads, int head_dim, int max_blocks_per_seq,
                            int num_blocks, float scale, int dtype, void* workspace,
                            size_t workspace_bytes, const void* plan, int flags, int num_groups,
                            int max_group_pages, void* prefix_buf, size_t prefix_bytes,
                            rlse_stream_t stream);

/* rlse_decode_step for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments and results
 * as rlse_decode_step, without a workspace: the split-K records live in a
 * static device array of 8.5 MB per device (room for 512 workgroups -- two
 * per compute unit on up to 256 CUs -- at group size <= 8, head_dim <= 128;
 * RLSE_ERR_INVALID_VALUE beyond that). The call allocates nothing and
 * calls no allocating routine. Every call on a device shares that array:
 * calls that overlap on one device (different streams or host threads)
 * race. Its error flags are read by rlse_workspace_check(NULL, ...). */
int rlse_decode_step_noalloc(const void* q, const void* k_new, const void* v_new,
                             const void* q_norm_weight, const void* k_norm_weight, float eps,
                             const void* cos_table, const void* sin_table, int max_pos,
                             void* k_pool, void* v_pool, const int32_t* block_tables,
                             const int32_t* seq_lens, void* out, int batch, int num_heads,
                             int num_kv_heads, int head_dim, int max_blocks_per_seq,
                             int num_blocks, float scale, int dtype, rlse_stream_t stream);

/* Chunked-prefill attention of one sequence: the prefill branch of
 * Attention::forward (src/backends/qwen2.rs:329-345) with the causal mask
 * of prepare_causal_attention_mask (src/backends/qwen2.rs:476-503), read
 * from the paged pool with GQA head mapping hq / (num_heads/num_kv_heads)
 * instead of repeat_kv. The chunk's num_tokens queries q [num_tokens]
 * [num_heads][head_dim] sit at positions ctx_len-num_tokens .. ctx_len-1;
 * their K/V must already be in the pool (appended as the reference appends
 * before attending). Query t sees keys 0 .. ctx_len-num_tokens+t of the
 * page list block_table[max_blocks] (ctx_len <= max_blocks*16); keys in
 * pages with ids outside [0, num_blocks) are skipped. out [num_tokens]
 * [num_heads][head_dim]. f32, bf16 or f16 (MFMA tiles: f32 products for
 * f32, the reference CPU path's dtype), head_dim 64 or 128. workspace:
 * rlse_prefill_workspace_size bytes (may be 0), or NULL
 * for a library-owned one per device. Calls that share a workspace, the
 * library-owned one included, must be ordered (same stream). */
int rlse_prefill_workspace_size(int num_tokens, int ctx_len, int num_heads, int num_kv_heads,
                                int head_dim, size_t* bytes);
int rlse_prefill_attn(const void* q, const void* k_pool, const void* v_pool,
                      const int32_t* block_table, int ctx_len, int num_tokens, void* out,
                      int num_heads, int num_kv_heads, int head_dim, int max_blocks,
                      int num_blocks, float scale, int dtype, void* workspace,
                      size_t workspace_bytes, rlse_stream_t stream);

/* ------------------------------------------------------------------ */
/* Normalisation and rotary embedding.                                 */
/* ------------------------------------------------------------------ */

/* RMSNorm over the last dim with Candle's cast order
 * (src/backends/qwen2.rs:68-75): y = dtype(x / sqrt(mean(x^2) + eps)) * w. */
int rlse_rmsnorm(const void* x, const void* weight, void* out, int rows, int n, float eps,
                 int dtype, rlse_stream_t stream);

/* Host-side RoPE tables [max_pos][head_dim/2] in dtype, built exactly as
 * RotaryEmbedding::new (src/backends/qwen2.rs:90-108). cos_out/sin_out are
 * HOST buffers of max_pos*head_dim/2 elements. */
int rlse_rope_tables(double theta, int head_dim, int max_pos, int dtype, void* cos_out,
                     void* sin_out);

/* In-place NeoX RoPE of q [num_tokens][num_heads][head_dim] and
 * k [num_tokens][num_kv_heads][head_dim] at positions[num_tokens]
 * (apply_rope / rotate_half, src/backends/qwen2.rs:125-142, 701-719).
 * Either q or k may be NULL. */
int rlse_rope(void* q, void* k, const void* cos_table, const void* sin_table,
              const int32_t* positions, int num_tokens, int num_heads, int num_kv_heads,
              int head_dim, int max_pos, int dtype, rlse_stream_t stream);

/* Fused Attention::forward front half (src/backends/qwen2.rs:291-313):
 * q_norm/k_norm RMSNorm (skipped when the weight pointer is NULL, as for
 * Qwen2), RoPE at positions, then append of the rotated k and raw v into
 * the pool (as rlse_kv_append), writing the rotated q to q_out.
 * q [num_tokens][num_heads][head_dim]; k, v [num_tokens][num_kv_heads][head_dim]. */
int rlse_qk_norm_rope_append(const void* q, const void* k, const void* v,
                             const void* q_norm_weight, const void* k_norm_weight,
                             float eps, const void* cos_table, const void* sin_table,
                             int max_pos, const int32_t* positions,
                             const int32_t* block_tables, int num_seqs,
                             const int32_t* seq_index,
                             int num_tokens, int num_heads, int num_kv_heads,
                             int head_dim, int max_blocks_per_seq, int num_blocks,
                             void* q_out, void* k_pool, void* v_pool, int dtype,
                             rlse_stream_t stream);

/* ------------------------------------------------------------------ */
/* Prototype-compatible launchers (same signatures and argument meaning */
/* as mini_serve_kernels.cu:247-296; default stream; head_dim fixed at */
/* 128; pools in the layout above; no block-id bounds check is possible */
/* because the signature carries no pool size).                       */
/* ------------------------------------------------------------------ */
int launch_rmsnorm_f32(const float* d_x, const float* d_w, float* d_out, int num_rows,
                       int hidden_size, float eps);
int launch_rmsnorm_f16(const void* d_x, const void* d_w, void* d_out, int num_rows,
                       int hidden_size, float eps);
int launch_rmsnorm_bf16(const void* d_x, const void* d_w, void* d_out, int num_rows,
                        int hidden_size, float eps);
int launch_paged_gqa_decode_tiled_f32(const float* d_q, const float* d_k_pool,
                                      const float* d_v_pool, const int* d_block_tables,
                                      const int* d_seq_lens, float* d_out, int batch_size,
                                      int num_heads, int num_kv_heads,
                                      int max_blocks_per_seq, float scale);
int launch_paged_gqa_decode_tiled_f16(const void* d_q, const void* d_k_pool,
                                      const void* d_v_pool, const int* d_block_tables,
                                      const int* d_seq_lens, void* d_out, int batch_size,
                                      int num_heads, int num_kv_heads,
                                      int max_blocks_per_seq, float scale);
int launch_paged_gqa_decode_tiled_bf16(const void* d_q, const void* d_k_pool,
                                       const void* d_v_pool, const int* d_block_tables,
                                       const int* d_seq_lens, void* d_out, int batch_size,
                                       int num_heads, int num_kv_heads,
                                       int max_blocks_per_seq, float scale);

/* ------------------------------------------------------------------ */
/* The rest of a batched decode step on the device: the ops of         */
/* ModelForCausalLM::step_decode_batch (src/backends/qwen2.rs:628-764) */
/* around rlse_decode_step, so activations and logits stay in HBM.     */
/* Element-wise ops round as Candle's per-op bf16/f16 arithmetic does. */
/* ------------------------------------------------------------------ */
/* embed_tokens (qwen2.rs:651-652): out[b] = table[ids[b]], rows of hidden
 * elements (hidden * dtype bytes a multiple of 16); an id outside [0, vocab)
 * gives a zero row. */
int rlse_embedding(const int32_t* ids, const void* table, void* out, int batch, int hidden,
                   int vocab, int dtype, rlse_stream_t stream);
/* A residual add followed by an RmsNorm (qwen2.rs:748-756, and the next
 * layer's input_layernorm :665-667): residual <- residual + x (rounded),
 * out <- RmsNorm(residual) * weight, RmsNorm::forward's cast order. With x
 * NULL the residual is only normalised (not written): RmsNorm::forward. */
int rlse_add_rmsnorm(const void* x, void* residual, const void* weight, void* out, int rows,
                     int n, float eps, int dtype, rlse_stream_t stream);
/* MLP activation (qwen2.rs:170-175): gate_up = [rows][2*inter], gate columns
 * then up columns; out = silu(gate) * up with silu(v) = v / (1 + exp(-v)). */
int rlse_silu_mul(const void* gate_up, void* out, int rows, int inter, int dtype,
                  rlse_stream_t stream);
/* Greedy branch of sample_token (src/backends/candle.rs:737-751) on the
 * device: per row the first maximum; NaNs never win, except a NaN at index
 * 0, which wins outright (the host Tensor::argmax scan). Two launches; the
 * workspace (rlse_argmax_workspace_size bytes, 8-byte aligned) holds one
 * partial per 4096 logits of a row and needs no clearing. */
int rlse_argmax_workspace_size(int rows, int vocab, size_t* bytes);
int rlse_argmax(const void* logits, int32_t* out, int rows, int vocab, int dtype,
                void* workspace, size_t workspace_bytes, rlse_stream_t stream);
/* Linear (q/k/v/o_proj, gate/up/down_proj, lm_head; qwen2.rs:233-252,
 * 153-158): y[rows][out] = x[rows][in] . W[out][in]^T with f32
 * accumulation, rounded once; bias (may be NULL) added after, rounded
 * again, as Candle's broadcast_add after the matmul. At most 64 rows (a
 * decode step's batch) with out a multiple of 16 run on the MFMA kernel of
 * the three calls below: bf16/f16 with in a multiple of 32, f32 (on f32
 * MFMAs) with in a multiple of 16 and 16-byte aligned buffers; other shapes
 * (prefill-sized products among them) go through rocBLAS gemm_ex. */
int rlse_linear(const void* x, const void* weight, const void* bias, void* y, int rows,
                int out_features, int in_features, int dtype, rlse_stream_t stream);
/* Packed weights (no counterpart in the reference, which multiplies its
 * row-major weights as loaded). OR-ed into the dtype argument of
 * rlse_linear, rlse_qkv_proj, rlse_linear_residual and rlse_gate_up_silu
 * (bf16/f16), it says the weight is in the order rlse_dense_pack writes:
 * per 16-row tile and 32-element k step, the 64 16-byte packets one MFMA
 * operand load takes, contiguous. Results are bit-identical to the
 * row-major weight's; each operand load reads one KiB instead of 64 bytes
 * from each of 16 rows. Packed, rlse_linear runs every row count on the
 * MFMA kernel (64 rows at a time). */
#define RLSE_DENSE_PACKED 0x100
/* Packed rows (no counterpart in the reference): OR-ed into the dtype of
 * rlse_add_rmsnorm, `out` is written, and OR-ed into the dtype of the four
 * projection calls, `x` is read, in the order of the MFMA kernel's B
 * operands: per 16-row tile and 32-element k step, 64 16-byte packets
 * (packet (t * in/32 + s) * 64 + r + 16j holds row 16t + r, elements
 * 32s + 8j .. +8). bf16/f16, the row length a multiple of 32; the buffer
 * holds whole 16-row tiles (rows rounded up to 16). Results are the
 * row-major ones, bit for bit. */
#define RLSE_PACKED_ROWS 0x200
/* OR-ed into the dtype of rlse_gate_up_silu: act is written in the packed
 * row order (inter a multiple of 32; act holds whole 16-row tiles), ready
 * for rlse_linear_residual's x with RLSE_PACKED_ROWS. */
#define RLSE_PACKED_OUT 0x400
/* Writes weight [out_features][in_features] (row-major) to packed in that
 * order (same size, not in place). gate_up_inter > 0: the stacked gate/up
 * weight of rlse_gate_up_silu ([2*gate_up_inter][in], gate rows then up
 * rows), whose tiles pair 8 gate rows with the matching 8 up rows; 0: any
 * other weight (out_features a multiple of 16). in_features a multiple of
 * 32, both buffers 16-byte aligned. */
int rlse_dense_pack(const void* weight, void* packed, int out_features, int in_features,
                    int gate_up_inter, int dtype, rlse_stream_t stream);
/* The three calls below are the decode step's projections fused with their
 * neighbours on MFMA (bf16/f16; in_features a multiple of 32; any rows,
 * taken 64 at a time; x and weights 16-byte, outputs 8-byte aligned).
 * workspace may be NULL; with rlse_dense_workspace_size bytes (for the
 * call's rows, total output features and in_features; zero-filled once
 * before its first use, then left to the library: error flags, launch
 * counters, epoch-tagged records) an output with few 16-feature tiles
 * splits K across workgroups so the whole chip streams the weights. Calls
 * that share a workspace must not overlap. */
int rlse_dense_workspace_size(int rows, int out_features, int in_features, size_t* bytes);
/* q/k/v_proj (qwen2.rs:668-679) in one launch over the stacked weights
 * w_qkv [q_features + 2*kv_features][hidden] (q rows, then k, then v) and
 * bias b_qkv (may be NULL; Qwen2): q [rows][q_features],
 * k/v [rows][kv_features], feature counts multiples of 16. */
int rlse_qkv_proj(const void* x, const void* w_qkv, const void* b_qkv, void* q, void* k,
                  void* v, int rows, int hidden, int q_features, int kv_features, int dtype,
                  void* workspace, size_t workspace_bytes, rlse_stream_t stream);
/* o_proj with `residual + attn_proj` (qwen2.rs:745-748) or down_proj with
 * `xs_mid + mlp_out` (:755-756): residual <- residual + x . W^T, the product
 * rounded, then the sum. out_features a multiple of 16. */
int rlse_linear_residual(const void* x, const void* weight, void* residual, int rows,
                         int out_features, int in_features, int dtype, void* workspace,
                         size_t workspace_bytes, rlse_stream_t stream);
/* MLP front (qwen2.rs:170-175): act = silu(gate_proj(x)) * up_proj(x) with
 * w_gate_up [2*inter][hidden] (gate rows, then up rows), the projections
 * rounded, then silu and the product as rlse_silu_mul. inter a multiple
 * of 8; the workspace is sized for out_features = 2*inter. */
int rlse_gate_up_silu(const void* x, const void* w_gate_up, void* act, int rows, int hidden,
                      int inter, int dtype, void* workspace, size_t workspace_bytes,
                      rlse_stream_t stream);

/* ------------------------------------------------------------------ */
/* Host block manager: the physical successor of KVCache               */
/* (src/cache/kv_cache.rs:15-145) with per-block refcounts for prefix  */
/* sharing. Ids pop in ascending order from a free stack (kv_cache.rs: */
/* 23-35); blocks_needed(t) = max(1, ceil(t/block_size)) (:53-59).     */
/* A block returns to the free stack when its last holder releases it. */
/* ------------------------------------------------------------------ */
typedef struct rlse_block_manager rlse_block_manager;

typedef struct rlse_cache_stats {
  int total_blocks;
  int allocated_blocks;
  int free_blocks;
  float utilization;   /* rounded to 3 decimals, kv_cache.rs:113-145 */
  float fragmentation; /* (free runs - 1) / free, rounded to 3 decimals */
} rlse_cache_stats;

int rlse_bm_create(int total_blocks, int block_size, rlse_block_manager** out);
int rlse_bm_destroy(rlse_block_manager* bm);
/* KVCache::blocks_needed (kv_cache.rs:53-59). Returns the count (>= 1) or -1. */
int rlse_bm_blocks_needed(const rlse_block_manager* bm, long long tokens);
int rlse_bm_free_count(const rlse_block_manager* bm);
/* KVCache::allocate (kv_cache.rs:61-84): RLSE_ERR_CACHE_PRESSURE with the
 * reference's message when too few blocks are free. Replaces any previous
 * allocation list of request_id, as the reference's HashMap insert does. */
int rlse_bm_allocate(rlse_block_manager* bm, const char* request_id, long long num_tokens,
                     int32_t* out_blocks, int capacity, int* num_out);
/* KVCache::allocate_block (kv_cache.rs:86-99). */
int rlse_bm_allocate_block(rlse_block_manager* bm, const char* request_id,
                           int32_t* out_block);
/* KVCache::release (kv_cache.rs:101-111); num_released = blocks the request held. */
int rlse_bm_release(rlse_block_manager* bm, const char* request_id, int* num_released);
/* Prefix fork: child_id gets parent_id's first ceil(num_tokens/16) blocks.
 * Full blocks are shared (refcount + 1); a trailing partial block is
 * copied-on-write into a fresh block, reported as (cow_src[i], cow_dst[i])
 * pairs for rlse_kv_copy_blocks. Fails before any change if the child
 * already holds blocks, the parent holds too few, or no block is free. */
int rlse_bm_fork(rlse_block_manager* bm, const char* parent_id, const char* child_id,
                 long long num_tokens, int32_t* cow_src, int32_t* cow_dst,
                 int cow_capacity, int* num_cow);
/* The request's block table (physical ids in logical order). */
int rlse_bm_block_table(const rlse_block_manager* bm, const char* request_id,
                        int32_t* out_blocks, int capacity, int* num_out);
int rlse_bm_refcount(const rlse_block_manager* bm, int block);
int rlse_bm_stats(const rlse_block_manager* bm, rlse_cache_stats* out);
/* Releases every request's blocks, in request-id order: the KV side of
 * quarantine (src/backends/candle.rs:689-697 clears every model state). */
int rlse_bm_release_all(rlse_block_manager* bm, int* num_requests);

/* ------------------------------------------------------------------ */
/* Per-step block tables: successor of the scheduler's per-step block  */
/* reservation (src/scheduler/scheduler.rs:422-449) plus the upload of */
/* the tables the decode kernels read. Row i of the tables is request  */
/* i of the step's batch. Uploads send only what changed since the     */
/* previous upload of the same object: the whole row of a request new  */
/* to its row (or whose block list was replaced), else one (row, col,  */
/* page) triple per page added. Host object; one upload in flight per  */
/* staging buffer (two), uploads of one object on one stream.          */
/* ------------------------------------------------------------------ */
typedef struct rlse_step_tables rlse_step_tables;
int rlse_st_create(int max_batch, int max_blocks_per_seq, rlse_step_tables** out);
int rlse_st_destroy(rlse_step_tables* st);
/* Forget what the device holds (the next upload sends every row whole),
 * e.g. after the device tables were reallocated. */
int rlse_st_reset(rlse_step_tables* st);
/* The reservation loop for a batch: request i grows to
 * blocks_needed(next_lens[i]) blocks (rlse_bm_allocate_block); a request
 * that cannot grow is released and gets status[i] = RLSE_ERR_CACHE_PRESSURE
 * (the reference's swap_remove + cancel + release), an unknown one
 * RLSE_ERR_UNKNOWN_REQUEST, one needing more than max_blocks_per_seq
 * blocks RLSE_ERR_INVALID_VALUE; their length is 0, which the decode
 * kernels answer with zeros. Then lays out the rows and lengths. */
int rlse_st_prepare(rlse_step_tables* st, rlse_block_manager* bm,
                    const char* const* request_ids, const long long* next_lens, int batch,
                    int* status);
/* Host image of this step: tables [max_batch][max_blocks_per_seq] (rows <
 * batch valid up to their block count), lengths, and the triples not yet
 * uploaded. */
int rlse_st_host(const rlse_step_tables* st, const int32_t** tables, const int32_t** seq_lens,
                 int* batch, const int32_t** pending, int* num_pending);
/* Copies the lengths and pending triples into device tables
 * [max_batch][max_blocks_per_seq] and seq_lens [max_batch] on stream: one
 * transfer from pinned memory plus one scatter kernel. Entries past a row's
 * block count are left as they were (never read). */
int rlse_st_upload(rlse_step_tables* st, int32_t* tables, int32_t* seq_lens,
                   rlse_stream_t stream);
/* For callers that copy the host image themselves: drops the pending
 * triples as if uploaded. */
int rlse_st_mark_uploaded(rlse_step_tables* st);

/* ------------------------------------------------------------------ */
/* Prefix cache over refcounted pages: successor of PrefixCache        */
/* (src/cache/prefix_cache.rs:58-394). Same chained SHA-256 chunk keys */
/* (:98-124), LRU refresh and eviction, lookup / lookup_kv / insert /  */
/* insert_kv rules and counters; a chunk holding KV keeps references  */
/* on its prefix's pages instead of a contiguous copy. Destroy the     */
/* cache before its block manager. Host only.                          */
/* ------------------------------------------------------------------ */
typedef struct rlse_prefix_cache rlse_prefix_cache;
typedef struct rlse_prefix_stats {
  long long hits, misses, tokens_saved; /* record_reuse counters (:368-380) */
  long long kv_evictions;               /* evicted chunks that held KV      */
  long long chunks, held_pages;         /* cached chunks, page references   */
  float hit_rate;                       /* percent, as hit_rate (:382-389)  */
} rlse_prefix_stats;

/* chunk_size: tokens per chunk, a multiple of the block manager's block size. */
int rlse_pc_create(rlse_block_manager* bm, int chunk_size, int max_chunks,
                   rlse_prefix_cache** out);
/* Releases every page reference the cache holds. */
int rlse_pc_destroy(rlse_prefix_cache* pc);
/* compute_chunk_hashes (:98-124): 64 hex digits + NUL per whole chunk. */
int rlse_pc_chunk_hashes(const uint32_t* tokens, long long num_tokens, int chunk_size,
                         char* out_hex, int capacity, int* num_chunks);
/* lookup (:126-155): matched tokens of the leading cached chunks. */
int rlse_pc_lookup(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens,
                   long long* matched_tokens);
/* insert (:198-203): metadata-only chunks. */
int rlse_pc_insert(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens);
/* insert_kv (:250-345): KV for every chunk boundary of tokens, from the
 * pages request_id holds (its first chunk_end/block_size pages); the chunk
 * ending exactly at num_tokens records the caller's logits handle when
 * has_logits. No bytes are copied. */
int rlse_pc_insert_kv(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens,
                      const char* request_id, int has_logits, long long logits_handle);
/* lookup_kv (:157-196): tokens covered by the longest cached chunk with KV;
 * has_logits / logits_handle only when that chunk ends at num_tokens. */
int rlse_pc_lookup_kv(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens,
                      long long* matched_tokens, int* has_logits, long long* logits_handle);
/* Restore of a prefix into child_id (the snapshot copy of set_kv_snapshot,
 * src/backends/candle.rs:437-478, 557-574): the child receives the cached
 * pages of the first restore_tokens tokens (<= the lookup_kv match), full
 * pages shared by refcount; a trailing partial page is copied on write --
 * one (src, dst) pair for rlse_kv_copy_blocks. */
int rlse_pc_fork(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens,
                 long long restore_tokens, const char* child_id, int32_t* cow_src,
                 int32_t* cow_dst, int cow_capacity, int* num_cow);
/* Evicts least recently used chunks until the block manager has at least
 * min_free_blocks free and, with a memory budget attached, room for that
 * many pages (the memory-pressure eviction of reserve_memory, :216-244);
 * RLSE_ERR_CACHE_PRESSURE if the cache empties first. */
int rlse_pc_reclaim(rlse_prefix_cache* pc, int min_free_blocks, int* evicted);
int rlse_pc_clear(rlse_prefix_cache* pc);
/* record_reuse (:368-376). */
int rlse_pc_record_reuse(rlse_prefix_cache* pc, long long skipped_tokens);
int rlse_pc_stats(const rlse_prefix_cache* pc, rlse_prefix_stats* out);
/* PrefixCache::reserve_memory (:229-244): try_reserve on the block
 * manager's budget, evicting least recently used chunks until the charge
 * fits; records a rejection and returns RLSE_ERR_CACHE_PRESSURE ("Tensor
 * memory budget exhausted") when the cache empties first. */
int rlse_pc_reserve_memory(rlse_prefix_cache* pc, long long active_kv_bytes,
                           long long execution_bytes, long long prefix_bytes, long long* lease);

/* ------------------------------------------------------------------ */
/* Tensor memory budget with page-based KV charges: successor of       */
/* TensorMemoryBudget (src/cache/tensor_memory.rs:41-125) and of       */
/* CandleBackend::memory_charge (src/backends/candle.rs:241-282).      */
/* The reference charges each request its whole contiguous capacity,   */
/* 2*layers*Hkv*d*(prompt+max_tokens)*bytes, at admission. A block     */
/* manager with an attached budget instead charges each page when it   */
/* leaves the free stack -- active KV while any request holds it,      */
/* retained prefix while only prefix-cache chunks hold it -- and       */
/* uncharges it when its last holder lets go. Host only; updates are   */
/* serialized by a mutex inside the budget, so workers may share one.  */
/* Destroy block managers (or detach them) before their budget.        */
/* ------------------------------------------------------------------ */
typedef struct rlse_memory_budget rlse_memory_budget;
typedef struct rlse_memory_stats {   /* TensorMemoryStats (:28-39)       */
  long long budget_bytes, headroom_bytes;
  long long active_kv_reserved_bytes;  /* leases + pages held by requests */
  long long execution_reserved_bytes;
  long long prefix_retained_bytes;     /* leases + pages held only by chunks */
  long long reserved_bytes, available_bytes, peak_reserved_bytes;
  long long rejections;
} rlse_memory_stats;
typedef struct rlse_model_shape {    /* the Config fields memory_charge reads */
  int num_layers, num_heads, num_kv_heads, head_dim;
  int hidden_size, intermediate_size, vocab_size;
  int dtype_bytes, context_length, block_size;
} rlse_model_shape;

/* TensorMemoryBudget::new (:48-67): 0 <= headroom < budget, else
 * RLSE_ERR_INVALID_VALUE; the headroom is reserved from the start. */
int rlse_mb_create(long long budget_bytes, long long headroom_bytes, rlse_memory_budget** out);
int rlse_mb_destroy(rlse_memory_budget* mb);
int rlse_mb_stats(rlse_memory_budget* mb, rlse_memory_stats* out);
/* try_reserve (:72-90): all or nothing; RLSE_ERR_CACHE_PRESSURE (no
 * rejection recorded) when the total does not fit or overflows. The lease
 * id is released with rlse_mb_release (MemoryReservation's Drop, :105-117). */
int rlse_mb_try_reserve(rlse_memory_budget* mb, long long active_kv_bytes,
                        long long execution_bytes, long long prefix_bytes, long long* lease);
int rlse_mb_release(rlse_memory_budget* mb, long long lease);
/* record_rejection (:92-94). */
int rlse_mb_record_rejection(rlse_memory_budget* mb);
/* Charges bm's pages to mb from now on (mb NULL: detach, uncharging them),
 * page_bytes per page -- 2*layers*Hkv*d*block_size*dtype_bytes, as
 * rlse_memory_charge reports. The pages held at attach time are charged at
 * once (all or nothing). With a budget attached, an allocation that does
 * not fit records a rejection and fails with RLSE_ERR_CACHE_PRESSURE before
 * any change. */
int rlse_bm_attach_budget(rlse_block_manager* bm, rlse_memory_budget* mb, long long page_bytes);
/* memory_charge (candle.rs:241-282) for paged KV, with the same checked
 * arithmetic and errors (RLSE_ERR_TOKEN_LIMIT for zero tokens or
 * prompt+max_tokens > context_length, RLSE_ERR_CACHE_PRESSURE on overflow):
 *   page_bytes = 2*layers*Hkv*d*block_size*B;
 *   kv_bytes   = ceil(T / block_size) * page_bytes, the most the request's
 *                pages can be charged (T = prompt + max_tokens);
 *   execution_bytes = 8*H*P*T*max(B,4) + 16*S*P*B + 8*I*P*B + 8*H*T*D*B
 *                + 16*V*max(B,4): the reference's estimate without its
 *                KV-sized staging term (pages are written in place). */
int rlse_memory_charge(const rlse_model_shape* shape, long long prompt_tokens,
                       long long max_tokens, long long* kv_bytes, long long* execution_bytes,
                       long long* page_bytes);

#ifdef __cplusplus
}
#endif

#endif /* RLSE_KV_H */
