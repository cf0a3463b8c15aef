/*
 * velokv.h -- C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * This library replaces the KV half of Velo-Core's Metal device runtime: the
 * K/V pools and block table owned by MetalMemoryRuntime / MetalKvStore and the
 * five KV kernels in kernels.metal. Everything above it (VeloEngine,
 * VeloScheduler, RadixCache, PagedAttentionBlockManager) stays in the host
 * program and talks to this ABI with plain pointers and sizes.
 *
 * Conventions
 *  - Every function returns an int32 status: VK_OK (0) or a negative VK_ERR_*.
 *    The message for the last failure on the calling thread is returned by
 *    vk_last_error(). Mirrors the Result<_, SpeculativeError::Model(String)>
 *    convention of the reference (speculative.rs, metal/runtime.rs:141-239).
 *  - Device pointers ("dev") are caller-owned unless a function says otherwise.
 *    The pool owns its HBM (K/V codes, scales, block table).
 *  - Compute entry points are asynchronous on the given stream (a hipStream_t
 *    passed as void*; NULL = the null stream). The reference blocks on every
 *    command buffer (metal/model.rs:141-142); callers that want that behaviour
 *    call vk_stream_sync().
 *  - The compute path is HIP only. There is no CPU fallback: a context whose
 *    code object is missing fails vk_ctx_create with VK_ERR_NOT_WIRED.
 *  - Threading: a context, its pools and block managers may be used from several
 *    host threads. Planning state (occupancy cache, workspace growth) is guarded
 *    inside the context. Compute calls on one pool that overlap in time (on
 *    different streams) must touch disjoint pages and, when they need split-K
 *    scratch, pass their own workspace: the context-owned one is shared, and
 *    overlapping calls that use it race on its contents (never on its lifetime:
 *    a workspace the context outgrows is freed only by vk_ctx_destroy). Block
 *    managers and radix caches are not internally locked: serialise calls on
 *    one of them, as the reference does with its mutexes (metal/backend.rs:142-144).
 *
 * Layout of one layer of a pool in HBM ("build layout"; the reference layout
 * is [blk][tok][head][D(+4)], kernels.metal:474,700). The unit is a tile of 16
 * tokens and 128 dims per KV head; a page of block_size = 16 k tokens is the
 * k tiles page * k .. (page + 1) * k - 1, so a flat slot
 * page * block_size + offset is also tile * 16 + offset % 16:
 *    K codes   [n_tiles][n_kv_heads][16][128] for F32 / F16;
 *              I8_*: [n_tiles][n_kv_heads][2][16][4][16] (dims 32c..32c+15 of
 *              token t at byte (4t + c)*16 of the tile, dims 32c+16..32c+31 at
 *              1024 + (4t + c)*16)
 *    V codes   [n_tiles][n_kv_heads][8][128][2]   (token pairs interleaved)
 *    scales    I8_BLK: fp16 pairs [n_tiles][n_kv_heads][2] (one K and one V
 *              scale per 16 tokens and head, K first: a (tile, head)'s two
 *              scales are one 4-byte word);
 *              I8_REF: fp32 [n_tiles][n_kv_heads][16] for K, then the same
 *              array for V
 * n_tiles = n_blocks * block_size / 16. A head_dim-64 pool has 64-dim tiles in
 * the same layouts at D = 64: [16][64] K, [8][64][2] V, and int8 K as
 * [2][16][2][16] (dims 32c..32c+15 of token t at byte (2t + c)*16, dims
 * 32c+16..32c+31 at 512 + (2t + c)*16); callers pass 64-dim rows.
 * Other head_dims (any multiple of 8 up to 128, kernels.metal:464) are stored in
 * the tiles of the next width, 64 dims for head_dim <= 64, else 128, with the
 * dims past head_dim held as zeros; callers pass head_dim-long rows (K, V, q,
 * out) and the softmax scale defaults to 1/sqrt(head_dim).
 * Element size: F32 4, F16 2, I8_* 1 byte.
 */
#ifndef VELOKV_H
#define VELOKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------
 * Each host-forcible failure of the reference boundary has its own code.    */
#define VK_OK                      0
#define VK_ERR_BAD_ARG            -1  /* argument out of range / null        */
#define VK_ERR_INVALID_BLOCK_SIZE -2  /* paged_attention.rs:104-106          */
#define VK_ERR_OUT_OF_PAGES       -3  /* paged_attention.rs:164-169          */
#define VK_ERR_TOO_MANY_PAGES     -4  /* metal/runtime.rs:296-302            */
#define VK_ERR_NO_FREE_SLOTS      -5  /* engine.rs:248-252                   */
#define VK_ERR_NOT_WIRED          -6  /* metal/backend.rs:79-83,130-140      */
#define VK_ERR_NO_DEVICE          -7  /* metal/runtime.rs:164 (no device)    */
#define VK_ERR_HIP                -8  /* a HIP runtime call failed           */
#define VK_ERR_UNSUPPORTED        -9  /* shape/dtype with no kernel          */
#define VK_ERR_UNKNOWN_HANDLE    -10  /* paged_attention.rs:189-192          */

/* ---- KV storage types ----------------------------------------------------
 * KvCacheType (paged_attention.rs:27-35) has Fp32 / Int8 / Fp8; Fp8 is routed
 * to the Int8 kernels (metal/model.rs:404,442), so it maps to VK_KV_I8_REF.  */
#define VK_KV_F32     0  /* KvCacheType::Fp32, kernels.metal:619-645 / 440-501 */
#define VK_KV_F16     1  /* fp16 KV (benchmark configurations 2 and 5)         */
#define VK_KV_I8_REF  2  /* KvCacheType::Int8: per-(token, head) fp32 scale,
                            truncating codes, kernels.metal:753-802           */
#define VK_KV_I8_BLK  3  /* per-(block, head) fp16 scale, round-half-even codes
                            clamped to +-127 (benchmark configuration 3)     */

/* element types of caller tensors (q, new K/V) */
#define VK_DT_F32 0
#define VK_DT_F16 1

typedef struct vk_ctx vk_ctx;
typedef struct vk_pool vk_pool;
typedef struct vk_block_manager vk_block_manager;

/* ---- context -------------------------------------------------------------- */

/* Last error message of the calling thread ("" if none). */
const char* vk_last_error(void);

/* Open `device`, load the gfx950 code object (NULL = velokv_gfx950.co next to
 * this library) and resolve every kernel.
 * Replaces MetalMemoryRuntime::new's device/queue/library setup
 * (metal/runtime.rs:141-186) and load_metal_library (metal/runtime.rs:29-60). */
int vk_ctx_create(int device, const char* code_object_path, vk_ctx** out);
int vk_ctx_destroy(vk_ctx* ctx);
/* Name of the GPU architecture the context runs on (e.g. "gfx950"). */
int vk_ctx_arch(const vk_ctx* ctx, char* buf, size_t cap);

/* No reference counterpart (the Metal encoder reports a bad threadgroup size
 * itself). Checks a workgroup of `threads` threads against what `kernel` was
 * compiled for (its __launch_bounds__, read once per kernel at vk_ctx_create)
 * without launching anything: VK_OK, VK_ERR_BAD_ARG naming the kernel and its
 * limit, or VK_ERR_NOT_WIRED for an unknown kernel. *max_threads (optional)
 * receives the limit (0 if unknown). Every launch of the library runs this
 * check first, so a wrong workgroup size is an error, not a device fault. */
int vk_kernel_launch_check(const vk_ctx* ctx, const char* kernel, int32_t threads, int32_t* max_threads);

/* No reference counterpart. Size in bytes the context's own split-K workspace
 * grows to when it holds `cur` bytes and a call needs `need` (callers that pass
 * no workspace): max(need, 2 * cur), 256-byte aligned; `cur` when need <= cur.
 * Outgrown buffers are kept until vk_ctx_destroy (a call on another host thread
 * may still have work queued on one), and doubling keeps their sum below the
 * live buffer's size. */
uint64_t vk_workspace_grow_bytes(uint64_t cur, uint64_t need);

/* Misuse the kernels detect without trapping. The work still completes on the
 * clamped input, a flag is or-ed into the context's device error word, and the
 * next vk_stream_sync or vk_ctx_check returns VK_ERR_BAD_ARG naming it (and
 * clears the word). The reference rejects the host-visible cases of the same
 * kind before dispatch (metal/runtime.rs:296-302); these inputs live in device
 * memory. Calls overlapping on several streams share the word; a flag is
 * reported by whichever check reads it first. */
#define VK_MISUSE_PAGE_OUT_OF_POOL 1u  /* an attention call read a block-table page id
                                          outside [0, n_blocks) (clamped into the pool) */
#define VK_MISUSE_BLK_SPLIT_RUN    2u  /* an I8_BLK append had tokens of one block that
                                          were not adjacent in the call (in
                                          vk_append_decode: two sequences' new
                                          tokens in one block)                        */
/* Waits for all work of the context's device, then reports and clears the misuse
 * flags (*flags = the flags read; NULL to skip): VK_OK when none were set. */
int vk_ctx_check(vk_ctx* ctx, uint32_t* flags);

/* Kernel family of vk_paged_decode: VK_DECODE_MFMA (QK and PV on
 * v_mfma_f32_16x16x{32,16}_f16 over fp16 / int8 KV, where an fp32 q is split
 * into fp16 hi + lo parts; on v_mfma_f32_16x16x4_f32 in fp32 throughout over
 * fp32 KV; over 64-dim heads in every pool type at group sizes up to 16,
 * kernels built for 64 dims), VK_DECODE_VALU (v_dot2_f32_f16, or fp32
 * arithmetic for an fp32 q or fp32 KV, on the vector ALUs; GQA group sizes
 * 1, 2, 4, 8 and head_dim 128, else the matrix cores run) or VK_DECODE_AUTO
 * (MFMA for int8 and fp32 KV and for fp32 queries, VALU for fp16 queries over
 * fp16 KV with fixed partitions: the faster one on MI355X for each; stream-K
 * batches run on the matrix cores). No reference counterpart. */
#define VK_DECODE_AUTO 0
#define VK_DECODE_VALU 1
#define VK_DECODE_MFMA 2
int vk_ctx_set_decode_kernel(vk_ctx* ctx, int kind);

/* Work schedule of vk_paged_decode when partition_tokens is 0: VK_SCHED_SPLIT
 * (units = fixed context partitions, sized to fill one round of resident waves;
 * kernel family per vk_ctx_set_decode_kernel; over int8 or fp32 KV with the
 * matrix cores, a batch whose
 * (sequence, KV head) pairs fill the GPU with at most 8 waves each runs one
 * workgroup per pair instead, its waves splitting the context and combining in
 * LDS, with no merge launch and no workspace), VK_SCHED_STREAM (stream-K on the matrix cores: one
 * wave per resident slot, each taking an equal share of all (sequence, KV head)
 * blocks, so ragged batches stay balanced; the split segments are combined by a
 * merge launch), VK_SCHED_PACKED (one workgroup of 8 waves per resident slot; the
 * (sequence, KV head) pairs, longest first, are dealt to the workgroups in snake
 * order so each gets a nearly equal share of blocks, and the waves of a workgroup
 * split its blocks evenly and combine split pairs in LDS: no merge launch and no
 * workspace; fp16 / int8 KV, at most 256 sequences, else stream-K) or VK_SCHED_AUTO (stream-K
 * unless vk_decode_args.sum_context_len says the batch is uniform, or the VALU
 * family was requested). A nonzero partition_tokens always uses fixed partitions. No
 * reference counterpart. */
#define VK_SCHED_AUTO 0
#define VK_SCHED_SPLIT 1
#define VK_SCHED_STREAM 2
#define VK_SCHED_PACKED 4  /* packed workgroup split (see below) */
int vk_ctx_set_decode_schedule(vk_ctx* ctx, int schedule);

/* ---- pools ---------------------------------------------------------------- */

typedef struct vk_pool_desc {
  int32_t n_layer;        /* MemoryRuntimeConfig::n_layer (runtime.rs:55)          */
  int32_t n_blocks;       /* MemoryRuntimeConfig::paged_total_pages (runtime.rs:53) */
  int32_t block_size;     /* MemoryRuntimeConfig::paged_block_size (runtime.rs:51):
                             16 k tokens per page, k = 1..16 (16, 32, 48 .. 256);
                             other sizes > 0 are VK_ERR_UNSUPPORTED, 0
                             VK_ERR_INVALID_BLOCK_SIZE */
  int32_t n_kv_heads;     /* ModelMeta::n_head_kv                                  */
  int32_t head_dim;       /* ModelMeta::head_dim: a multiple of 8 up to 128 (64- or
                             128-dim tiles, zero-padded past head_dim)            */
  int32_t kv_type;        /* VK_KV_*  (MemoryRuntimeConfig::kv_type)               */
  int32_t max_slots;      /* MemoryRuntimeConfig::max_slots (runtime.rs:59)        */
  int32_t max_pages_per_slot; /* row length of the slot block table; 0 = n_blocks
                                 (the reference sizes rows by paged_total_pages,
                                 metal/runtime.rs:222-223)                         */
} vk_pool_desc;

/* Device addresses of one layer, for callers that read or write the pool
 * directly (tests, KV migration). Scales are read in 16-bit units: unit e of
 * the K (V) scales is at k_scales (v_scales) + e * scale_step. VK_KV_I8_REF:
 * scale_step 2, each kind contiguous. VK_KV_I8_BLK: scale_step 4, the K and V
 * scale of one (block, head) share a 4-byte word (K low, V high: v_scales =
 * k_scales + 2), so a decode fetches both with one load. */
typedef struct vk_layer_view {
  void* k_codes;  void* v_codes;
  void* k_scales; void* v_scales;   /* NULL for F32 / F16 */
  uint64_t codes_bytes;             /* bytes of each of k_codes / v_codes  */
  uint64_t scales_bytes;            /* bytes of each kind's scales (units x 2) */
  uint32_t scale_step;              /* bytes between a kind's 16-bit scale units: 2, 4 (I8_BLK), 0 */
} vk_layer_view;

/* Allocate and zero the K and V pools of all layers plus the slot block table
 * (u32[max_slots][max_pages_per_slot], zero-filled).
 * Replaces MetalKvStore::new (metal/kv_store.rs:36-57) and the slot-mapping
 * buffer allocation (metal/runtime.rs:221-229), with one layer offset per layer
 * (the reference binds every layer at offset 0, metal/model.rs:409-410). */
int vk_pool_create(vk_ctx* ctx, const vk_pool_desc* desc, vk_pool** out);
int vk_pool_destroy(vk_pool* pool);
int vk_pool_get_desc(const vk_pool* pool, vk_pool_desc* out);
int vk_pool_layer_view(const vk_pool* pool, int32_t layer, vk_layer_view* out);
/* Device pointer of the slot block table and its row stride (in entries). */
int vk_pool_block_table(const vk_pool* pool, int32_t** table_dev, int32_t* row_stride);
/* Total HBM held by the pool. */
int vk_pool_bytes(const vk_pool* pool, uint64_t* out);

/* Write `pages` into row `slot` of the pool's block table and zero the rest of
 * the row; synchronous, like the reference's memcpy into shared memory.
 * MemoryRuntime::bind_slot (runtime.rs:34) / MetalMemoryRuntime::bind_slot
 * (metal/runtime.rs:294-319). Errors: VK_ERR_TOO_MANY_PAGES when n_pages
 * exceeds the row length, VK_ERR_BAD_ARG for a slot >= max_slots or a page id
 * >= n_blocks. */
int vk_bind_slot(vk_pool* pool, uint32_t slot, const uint32_t* pages, int32_t n_pages);

/* ---- hot path ------------------------------------------------------------- */

/* Per-token flat slot = table[row][pos / bs] * bs + pos % bs, where row is
 * seq_rows[i] (or i when seq_rows is NULL). All pointers are device pointers.
 * The slot derivation the reference performs inside kv_update
 * (kernels.metal:637-640, 770-774). */
int vk_slot_mapping(vk_ctx* ctx, vk_pool* pool, const int32_t* block_tables,
                    int32_t bt_stride, const int32_t* seq_rows,
                    const int32_t* positions, int32_t n_tok,
                    int64_t* slot_mapping_out, void* stream);

/* Append n_tok new tokens of one layer: k, v are dev [n_tok][n_kv_heads][head_dim]
 * of type in_dtype (VK_DT_*); slot_mapping is dev int64 [n_tok] (negative, or
 * at or past n_blocks * block_size = skip). Quantizes on the way in for the I8
 * types.
 * kv_update (kernels.metal:619-645) and kv_update_int8 (kernels.metal:753-802),
 * dispatched at metal/model.rs:399-434.
 * Order rule: tokens of one call are applied in index order. For VK_KV_I8_BLK a
 * token at block offset 0 starts a fresh block scale; a later token whose absmax
 * needs a larger scale re-quantizes the codes already in the block. Tokens of
 * one call that fall in the same block must be adjacent in the call (padding
 * slots may sit between them) and in increasing offset order; a call that
 * breaks adjacency is reported as VK_MISUSE_BLK_SPLIT_RUN. */
int vk_append(vk_ctx* ctx, vk_pool* pool, int32_t layer, const void* k,
              const void* v, int32_t in_dtype, const int64_t* slot_mapping,
              int32_t n_tok, void* stream);

/* ---- RoPE fused into the append -------------------------------------------
 * The reference rotates q and k in two ways that disagree: the Metal kernel
 * pairs dims (2i, 2i+1) (kernels.metal:103-131, the GPU path) and the CPU model
 * pairs (i, i + head_dim/2) (llama_cpu.rs:113-131). Both use the angle
 * pos * freq_base^(-2i/head_dim) for pair i; the caller picks the style its
 * weights were exported for. */
#define VK_ROPE_INTERLEAVED 1  /* pairs (2i, 2i+1): kernels.metal:103-131    */
#define VK_ROPE_HALF        2  /* pairs (i, i+D/2): llama_cpu.rs:113-131     */

/* Host: fill out[n_pos][head_dim/2][2] (fp32) with cos and sin of the angle
 * p * freq_base^(-2i/head_dim) of pair i at position p, evaluated in double
 * precision and rounded to fp32 once. Upload it once; vk_append_rope reads it
 * (the reference evaluates the angle in fp32 per call, llama_cpu.rs:124-125). */
int vk_rope_table(float* out, int32_t n_pos, int32_t head_dim, float freq_base);

/* vk_append with rotary position embedding fused in: each token's K row is
 * rotated by its position (positions: dev int32 [n_tok]) before it is stored
 * (and quantized for the I8 types); V is stored as is. When q is not NULL the
 * same launch rotates q in place (dev [n_tok][n_heads][head_dim] of q_dtype;
 * fp16 q is rounded to fp16 after the fp32 rotation). cos_sin is the dev table
 * of vk_rope_table with n_pos positions, 16-byte aligned (the kernels read it
 * in 16-byte chunks; VK_ERR_BAD_ARG otherwise); a token whose position is outside
 * [0, n_pos) is skipped like a negative slot (not appended, q not rotated).
 * Rotation: y0 = x0 c - x1 s, y1 = x0 s + x1 c in fp32, every product and sum
 * rounded separately, the reference's expression order (llama_cpu.rs:128-129).
 * Replaces the separate rope dispatch before kv_update (metal/model.rs:380-396)
 * and rope() of the CPU model (llama_cpu.rs:99-111, called at 249). */
int vk_append_rope(vk_ctx* ctx, vk_pool* pool, int32_t layer, void* q, int32_t q_dtype,
                   int32_t n_heads, const void* k, const void* v, int32_t in_dtype,
                   const int32_t* positions, const int64_t* slot_mapping, int32_t n_tok,
                   const float* cos_sin, int32_t n_pos, int32_t rope_style, void* stream);

typedef struct vk_decode_args {
  int32_t layer;
  const void* q;              /* dev [S][n_heads][head_dim] of q_dtype         */
  int32_t q_dtype;            /* VK_DT_F16: fp16 q. VK_DT_F32: over fp16 / int8
                                 KV the matrix-core kernels split q into fp16
                                 hi + lo (scores see q to ~2^-22); over fp32 KV
                                 and in the VALU kernels fp32 math */
  float* out;                 /* dev fp32 [S][n_heads][head_dim]               */
  const int32_t* block_tables;/* dev [rows][bt_stride]; NULL = the pool's slot table */
  int32_t bt_stride;          /* ignored when block_tables is NULL             */
  const int32_t* seq_rows;    /* dev [S] row of each sequence; NULL = 0..S-1   */
  const int32_t* context_lens;/* dev [S] tokens to attend (incl. the new one)  */
  int32_t n_seqs;             /* S                                             */
  int32_t n_heads;            /* query heads H (multiple of n_kv_heads)        */
  int32_t max_context_len;    /* host upper bound of context_lens              */
  float scale;                /* softmax scale; 0 = 1/sqrt(head_dim)           */
  int32_t partition_tokens;   /* split-K partition size in tokens; 0 = auto    */
  void* workspace;            /* dev scratch for split-K partials; NULL = owned by
                                 ctx (calls on one ctx that overlap in time must
                                 then pass their own). Needs no initialisation. */
  uint64_t workspace_bytes;
  int64_t sum_context_len;    /* host sum of context_lens if known, else 0: with
                                 VK_SCHED_AUTO a batch whose sum is within 3 % of
                                 n_seqs * max_context_len runs fixed partitions,
                                 any other (or unknown) batch runs stream-K    */
} vk_decode_args;

/* Bytes of workspace vk_paged_decode needs for these arguments. */
int vk_paged_decode_workspace(const vk_pool* pool, const vk_decode_args* a, uint64_t* bytes);

/* Name of the attention kernel vk_paged_decode would launch for these arguments
 * (for profiling and reports). No reference counterpart. */
int vk_paged_decode_kernel(const vk_pool* pool, const vk_decode_args* a, char* buf, size_t cap);

/* The schedule vk_paged_decode would run for these arguments (for tests,
 * profiling and reports). No reference counterpart. */
#define VK_SCHED_WORKGROUP 3   /* schedule value reported for the workgroup split */
typedef struct vk_decode_plan {
  char kernel[64];             /* attention kernel name                                */
  int32_t schedule;            /* VK_SCHED_SPLIT, _STREAM, _WORKGROUP or _PACKED       */
  int32_t wg_waves;            /* waves per workgroup of the attention launch
                                  (workgroup split, packed split, stream-K)          */
  int32_t partition_tokens;    /* fixed partitions: tokens per partition               */
  int32_t max_partitions;      /* fixed partitions: partitions of the longest context  */
  int32_t n_workers;           /* stream-K: workers (one wave each, wg_waves of them
                                  per workgroup); packed: workgroups                 */
  int32_t max_blocks_per_wave; /* the most blocks one wave can walk (<= 256)           */
  uint64_t workspace_bytes;    /* split-K scratch the call needs                       */
  int32_t merge_launch;        /* 1 when a merge launch follows the attention kernel   */
} vk_decode_plan;
int vk_paged_decode_plan(const vk_pool* pool, const vk_decode_args* a, vk_decode_plan* out);

/* Single-query paged decode attention for S sequences, with split-K over
 * context partitions and an online-softmax merge (a second launch, skipped
 * when every sequence fits one partition).
 * paged_attention_flash (kernels.metal:440-501), paged_attention_flash_int8
 * (kernels.metal:672-732); GQA map kv_head = h / (H / Hkv) (kernels.metal:456);
 * math of llama_cpu.rs:251-284. */
int vk_paged_decode(vk_ctx* ctx, vk_pool* pool, const vk_decode_args* a, void* stream);

/* One decode step of a layer: the new token of every sequence appended, then
 * decode attention over the context including it. k_new, v_new are dev
 * [S][n_kv_heads][head_dim] of in_dtype (VK_DT_*); the token of sequence s goes
 * to position min(context_lens[s], max_context_len) - 1 of its block-table row
 * (slot = table[row][pos / bs] * bs + pos % bs, as kv_update derives it,
 * kernels.metal:637-640, 770-774); a sequence with context 0 appends nothing,
 * and a page id outside the pool stores nothing (the decode reports it,
 * VK_MISUSE_PAGE_OUT_OF_POOL). The pool afterwards equals vk_append of those
 * slots followed by vk_paged_decode, bit for bit, and so do the outputs except
 * under the workgroup split, whose folding wave takes a few blocks fewer (the
 * outputs then agree to fp32 rounding of a different split). Over VK_KV_I8_BLK pools under the
 * workgroup-split or stream-K schedule, and over VK_KV_F16 pools under
 * stream-K, the decode launch appends the tokens itself (the
 * wave that holds a sequence's last block applies the append rule to it before
 * loading it; two sequences whose new tokens share a block are reported,
 * VK_MISUSE_BLK_SPLIT_RUN); otherwise the append kernel runs first, with the
 * slots derived in the kernel, then the decode.
 * The reference runs kv_update then the attention kernel per layer
 * (metal/model.rs:399-471). */
int vk_append_decode(vk_ctx* ctx, vk_pool* pool, const void* k_new, const void* v_new, int32_t in_dtype,
                     const vk_decode_args* a, void* stream);

/* One decode step of a layer with rotary position embedding: the reference's
 * rope -> kv_update -> attention (metal/model.rs:380-471). As vk_append_decode,
 * with the new K rows and every q row rotated at the new token's position
 * (context_len - 1) by the vk_rope_table rows cos_sin (16-byte aligned; style
 * VK_ROPE_INTERLEAVED or VK_ROPE_HALF), exactly as vk_append_rope rotates them;
 * a position outside [0, n_pos) rotates nothing and appends nothing. The
 * attention uses the rotated q; the caller's q buffer is left unchanged. Where
 * vk_append_decode folds the append into the decode launch and head_dim is 64
 * or 128, the rotation folds too (one launch per layer: the folding wave
 * rotates the new K row, every wave its q rows in registers); otherwise the
 * RoPE append runs first and writes the rotated q rows into the workspace,
 * whose size vk_append_rope_decode_workspace gives. The pool afterwards equals
 * vk_append_rope (positions context_len - 1) followed by vk_paged_decode on the
 * rotated q, bit for bit. No separate reference counterpart. */
int vk_append_rope_decode(vk_ctx* ctx, vk_pool* pool, const void* k_new, const void* v_new, int32_t in_dtype,
                          const float* cos_sin, int32_t n_pos, int32_t rope_style, const vk_decode_args* a,
                          void* stream);
int vk_append_rope_decode_workspace(const vk_pool* pool, const vk_decode_args* a, uint64_t* bytes);

/* vk_paged_decode that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops or harnesses that forbid hipMalloc). The split-K scratch comes
 * from a fixed array of VK_NOALLOC_SCRATCH_BYTES that the library holds on each
 * GPU it runs on until the process ends (its device address is resolved once
 * per device when a context is created); a->workspace must be NULL and
 * a->workspace_bytes 0. A call whose scratch would exceed the array fails with
 * VK_ERR_BAD_ARG (vk_paged_decode_plan reports the bytes a call needs). Every
 * call on one GPU shares that GPU's array and nothing in it needs clearing
 * between calls; calls that overlap in time on one GPU race on it. */
#define VK_NOALLOC_SCRATCH_BYTES (64ull << 20)
int vk_paged_decode_noalloc(vk_ctx* ctx, vk_pool* pool, const vk_decode_args* a, void* stream);

typedef struct vk_tree_args {
  int32_t layer;
  const void* q;              /* dev [S][n_nodes][n_heads][head_dim] of q_dtype */
  int32_t q_dtype;            /* VK_DT_F16, or VK_DT_F32 (split into fp16 hi +
                                 lo for the fp16 / int8 matrix-core kernels, each
                                 score taking both products, so q keeps about 22
                                 bits; kept in fp32 over fp32 KV) */
  float* out;                 /* dev fp32 [S][n_nodes][n_heads][head_dim]       */
  const int32_t* block_tables;/* dev [rows][bt_stride]; NULL = slot table        */
  int32_t bt_stride;
  const int32_t* seq_rows;    /* dev [S] or NULL                                 */
  const int32_t* context_lens;/* dev [S] committed tokens before the tree        */
  const uint32_t* tree_mask;  /* dev [S][n_nodes]: bit j of row i = node i sees node j */
  int32_t n_seqs;
  int32_t n_nodes;            /* 1..32; node j's K/V sit at position context_len + j */
  int32_t n_heads;
  int32_t max_context_len;    /* max over context_lens (committed tokens)        */
  float scale;                /* 0 = 1/sqrt(head_dim)                            */
  int32_t partition_tokens;   /* split-K partition, multiple of bs, <= 4096; 0 = auto */
  void* workspace;            /* dev split-K scratch or NULL (context-owned)     */
  uint64_t workspace_bytes;
  int32_t shared_blocks;      /* the first shared_blocks pages of every table row
                                 used by the call are the same fully written pages
                                 (a prefix shared through the radix cache), 0 if
                                 unknown; shared_blocks * block_size <=
                                 max_context_len. Over F16 and I8_BLK pools the
                                 prefix is attended once per KV head for all rows
                                 (the results are those of shared_blocks = 0 up to
                                 fp32 rounding); other pools ignore it. */
} vk_tree_args;

/* Bytes of split-K workspace vk_tree_verify needs for these arguments (0 when
 * one partition covers every sequence). */
int vk_tree_verify_workspace(const vk_pool* pool, const vk_tree_args* a, uint64_t* bytes);

/* What vk_tree_verify would launch for these arguments, launching nothing. No
 * reference counterpart (the reference's tree kernel has no caller). */
typedef struct vk_tree_plan {
  char kernel[64];             /* rest-of-context (or whole-context) tree kernel     */
  char prefix_kernel[64];      /* shared-prefix pass, "" when there is none          */
  int32_t prefix_chunks;       /* chunks the shared prefix is cut into (0 = no pass) */
  int32_t prefix_row_tiles;    /* prefix pass: 256-row tiles of query rows per KV head */
  int32_t row_tiles;           /* tree kernel: 16-row tiles per (sequence, KV head)   */
  int32_t rows_per_tile;       /* 16 or 32 (the kernel's row tiles per wave x 16)     */
  int32_t partition_tokens;    /* rest of the context: tokens per partition          */
  int32_t max_partitions;      /* partial slots per row, prefix chunks included      */
  uint64_t workspace_bytes;    /* split-K scratch the call needs                     */
  int32_t merge_launch;        /* 1 when vk_decode_merge follows                     */
} vk_tree_plan;
int vk_tree_verify_plan(const vk_pool* pool, const vk_tree_args* a, vk_tree_plan* out);

/* Multi-query tree-verify attention over fp32, fp16 or int8 pools: query row (node i,
 * head h) attends to the committed context (positions 0..context_len-1) and to
 * the tree nodes j its mask row selects (position context_len + j). Build
 * tree_mask with vk_tree_mask (ancestors and the node itself).
 * paged_attention_tree (kernels.metal:512-599) / forward_tree
 * (metal/model.rs:574-731). The reference places an ancestor at n_ctx + depth
 * and skips the node itself (kernels.metal:567-575); here every node has its own
 * position so sibling branches do not collide, and a node sees itself. */
int vk_tree_verify(vk_ctx* ctx, vk_pool* pool, const vk_tree_args* a, void* stream);

/* Ancestor mask of a draft tree given as parent indices (parents[0] = -1 for
 * the root, parents[i] < i otherwise): mask_out[i] has bit j set when node j is
 * node i or one of its ancestors. Host only.
 * SpeculativeTree (speculative.rs:48-95); ancestors_map of forward_tree
 * (metal/model.rs:615-632) as a bitmask. */
int vk_tree_mask(const int32_t* parents, int32_t n_nodes, uint32_t* mask_out);

/* Copy-on-write block copy: for each (src, dst) pair in the HOST array
 * src_dst_pairs[2*n_pairs], copy the K/V codes and scales of block src to block
 * dst in every layer. dst blocks must be distinct and must not appear as a src.
 * No counterpart in the reference (it has no COW); serves the prefix sharing of
 * RadixCache (radix_cache.rs:73-140). */
int vk_copy_blocks(vk_ctx* ctx, vk_pool* pool, const int32_t* src_dst_pairs,
                   int32_t n_pairs, void* stream);

/* Commit the accepted path of a verified draft tree in layers
 * [layer0, layer0 + n_layers): for sequence s with committed length
 * context_lens[s], the K/V of tree node accept[s][d] (position
 * context_lens[s] + accept[s][d]) move to position context_lens[s] + d, for
 * d < n_accept[s]. All pointers are device pointers; accept is
 * [n_seqs][accept_stride], each row strictly increasing with accept[s][d] >= d
 * and < 32. A row that breaks this, or whose positions fall outside its block
 * table row or the pool, is left untouched and reported in status (dev int32
 * [n_seqs], VK_COMMIT_*; NULL = not reported). Leading nodes already in place
 * (accept[s][d] == d) are not rewritten. The blocks written must belong to one
 * sequence only (copy-on-write before appending the tree makes them private).
 * F32 / F16 / I8_REF: the token rows (with their per-token scales) move
 * unchanged. I8_BLK: every moved token is first dequantized (code x block
 * scale, exact in fp32) from the pre-commit pool; the moved tokens are then
 * appended in order by vk_append's rule, so a destination at block offset 0
 * starts a fresh scale and a token that needs a larger scale re-quantizes the
 * codes before it.
 * Completes the tree-verify step: verify_tree (speculative.rs:217-242) accepts
 * a root-to-node path of SpeculativeTree (speculative.rs:48-130) whose K/V
 * were appended at context_len + node by the draft pass. */
#define VK_COMMIT_OK          0  /* committed (or nothing to move)                     */
#define VK_COMMIT_BAD_ROW     1  /* n_accept / accept row malformed, or context_len < 0 */
#define VK_COMMIT_PAST_TABLE  2  /* a position past the block-table row                */
#define VK_COMMIT_BAD_PAGE    3  /* a page id outside the pool                         */
int vk_tree_commit(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers,
                   const int32_t* block_tables, int32_t bt_stride,
                   const int32_t* context_lens, const int32_t* accept,
                   int32_t accept_stride, const int32_t* n_accept,
                   int32_t n_seqs, int32_t* status, void* stream);

/* ---- NIXL wire records of KV pages ------------------------------------------
 * Wire format of nixl.rs:24-61 (serialize_block / deserialize_block): a record
 * is [block_id u64 LE][token_len u32 LE][byte_len u32 LE][payload byte_len B].
 * The reference leaves the payload opaque (nixl.rs:365-367); here it is the
 * KV pages of one KvCacheHandle (radix_cache.rs:6-9) over a layer range
 * [layer0, layer0 + n_layers), n_pages = ceil(token_len / block_size):
 *    tiles   for page i, for layer l: K codes of the page's n_kv_heads tiles,
 *            then V codes (2 * n_kv_heads * tile bytes, in pool layout)
 *    scales  for page i, for layer l: K scales of the page, then V scales
 *            (I8 pools only; fp16 per head for I8_BLK, fp32 per token for I8_REF)
 * Whole pages travel, including the slots past token_len in the last page. */
#define VK_NIXL_HEADER_BYTES 16

typedef struct vk_nixl_item {
  uint64_t block_id;     /* KvCacheHandle.block_id                              */
  uint32_t token_len;    /* KvCacheHandle.token_len                             */
  int32_t first_page;    /* index into the pages array of this handle's first page */
  uint64_t wire_offset;  /* byte offset of the record in the wire buffer (16-aligned) */
} vk_nixl_item;

/* Per-record status written by pack / unpack (dev int32 [n_items]). The first
 * two are the cases where deserialize_block returns None (nixl.rs:50-58). */
#define VK_NIXL_OK               0
#define VK_NIXL_SHORT_HEADER     1  /* fewer than 16 bytes left in the wire      */
#define VK_NIXL_TRUNCATED        2  /* header + byte_len runs past the wire      */
#define VK_NIXL_HANDLE_MISMATCH  3  /* header block_id / token_len != the item   */
#define VK_NIXL_LENGTH_MISMATCH  4  /* byte_len != the payload for this pool     */
#define VK_NIXL_BAD_PAGE         5  /* a page id outside the pool                */

/* Payload bytes of one record (without the 16-byte header). */
int vk_nixl_payload_bytes(const vk_pool* pool, int32_t n_layers, uint32_t token_len,
                          uint64_t* bytes);

/* Serialise n_items handles into the wire buffer (dev, wire_bytes long).
 * items is a HOST array; pages is a dev int32 array of n_pages page ids (item i
 * uses pages[first_page .. first_page + ceil(token_len/bs))); status is dev
 * int32 [n_items]. A record whose pages are all in range gets its header and
 * payload and status VK_NIXL_OK; otherwise VK_NIXL_BAD_PAGE and its bytes are
 * not written. Records must fit in the wire buffer and not overlap
 * (VK_ERR_BAD_ARG otherwise); byte_len must fit in u32.
 * DmaBlockManager::write_and_serialize (nixl.rs:129-144) / serialize_block
 * (nixl.rs:36-43), done as one gather of pool pages in HBM. */
int vk_nixl_pack(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers,
                 const vk_nixl_item* items, int32_t n_items, const int32_t* pages,
                 int32_t n_pages, void* wire, uint64_t wire_bytes, int32_t* status,
                 void* stream);

/* Deserialise records from the wire buffer into pool pages: item i's record is
 * read at wire_offset and checked (status codes above, in that order); a
 * record that passes writes its payload into pages[first_page ..] of this pool
 * (which need not be the pages it was packed from), a record that fails writes
 * nothing. Destination pages must be distinct across items.
 * DmaBlockManager::receive_into (nixl.rs:147-155) / deserialize_block
 * (nixl.rs:49-61), done as one scatter into pool pages in HBM. */
int vk_nixl_unpack(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers,
                   const vk_nixl_item* items, int32_t n_items, const int32_t* pages,
                   int32_t n_pages, const void* wire, uint64_t wire_bytes,
                   int32_t* status, void* stream);

/* ---- host block manager ----------------------------------------------------
 * PagedAttentionBlockManager (paged_attention.rs:92-212): FIFO free list,
 * pages_for_tokens = ceil(len / bs), plus per-page reference counts for
 * prefix sharing (the reference has none; used by vk_bm_fork / vk_bm_cow). */
int vk_bm_create(int32_t block_size, int32_t total_pages, vk_block_manager** out);
int vk_bm_destroy(vk_block_manager* bm);
int vk_bm_free_pages(const vk_block_manager* bm, int32_t* out);
int vk_bm_block_size(const vk_block_manager* bm, int32_t* out);
/* allocate(handle, token_len): pops ceil(token_len/bs) pages; pages_out gets them. */
int vk_bm_allocate(vk_block_manager* bm, uint64_t handle, int64_t token_len,
                   uint32_t* pages_out, int32_t cap, int32_t* n_out);
/* release(handle): drops one reference of each page; pages reaching zero go
 * back to the free list in order. */
int vk_bm_release(vk_block_manager* bm, uint64_t handle);
/* materialize_span(handle). */
int vk_bm_pages(const vk_block_manager* bm, uint64_t handle, uint32_t* pages_out,
                int32_t cap, int32_t* n_out);
/* New handle `child` that shares the first ceil(shared_tokens/bs) pages of
 * `parent` (refcount + 1) and owns fresh pages for the rest of token_len. */
int vk_bm_fork(vk_block_manager* bm, uint64_t parent, uint64_t child,
               int64_t shared_tokens, int64_t token_len, uint32_t* pages_out,
               int32_t cap, int32_t* n_out);
/* Grow `handle` to cover token_len tokens: fresh pages are appended (FIFO);
 * a handle that already covers them is unchanged. For a sequence that outgrows
 * the pages its prompt was given (decode tokens, draft-tree slots); the
 * reference binds a slot's pages once at prefill (engine.rs:266-268). */
int vk_bm_extend(vk_block_manager* bm, uint64_t handle, int64_t token_len,
                 uint32_t* pages_out, int32_t cap, int32_t* n_out);
/* Before writing into page index `page_idx` of `handle`: if that page is
 * shared, replace it by a fresh page and report the (src, dst) copy to issue
 * through vk_copy_blocks; *copied = 0 when the page was already private. */
int vk_bm_cow(vk_block_manager* bm, uint64_t handle, int32_t page_idx,
              int32_t* src, int32_t* dst, int32_t* copied);
int vk_bm_refcount(const vk_block_manager* bm, uint32_t page, int32_t* out);

/* ---- prefix cache over page handles ------------------------------------------
 * RadixCache (radix_cache.rs:28-264): a radix tree of token edges whose nodes
 * hold KV handles, with the reference's insert / lookup / edge split, logical
 * clock and coldest-first eviction (same results as the reference on the same
 * calls). Handles are block-manager handles (vk_bm_*), token_len = the tokens
 * inserted. Created with a block manager, the cache owns the handles inserted
 * into it and releases replaced and evicted ones there (pages return to the
 * free list once no other handle references them); with bm = NULL handles are
 * opaque ids and nothing is released, as in the reference. Host only. */
typedef struct vk_radix vk_radix;
/* RadixCache::new / with_capacity_tokens (capacity_tokens < 0: no limit). */
int vk_radix_create(vk_block_manager* bm, int64_t capacity_tokens, vk_radix** out);
/* Releases every handle the cache holds (bound caches). */
int vk_radix_destroy(vk_radix* rc);
/* RadixCache::insert (radix_cache.rs:73-99): *has_replaced / *replaced report
 * the handle this prefix held before (released when bound). */
int vk_radix_insert(vk_radix* rc, const uint32_t* tokens, int32_t n_tokens, uint64_t handle,
                    uint64_t* replaced, int32_t* has_replaced);
/* RadixCache::lookup (radix_cache.rs:101-140): longest cached prefix. */
int vk_radix_lookup(vk_radix* rc, const uint32_t* tokens, int32_t n_tokens, int32_t* matched,
                    uint64_t* handle, int32_t* has_handle);
int vk_radix_len(const vk_radix* rc, int32_t* out);
int vk_radix_resident_tokens(const vk_radix* rc, int64_t* out);
int vk_radix_capacity_tokens(const vk_radix* rc, int64_t* out);   /* -1 = no limit */
int vk_radix_set_capacity(vk_radix* rc, int64_t capacity_tokens);
/* RadixCache::evict_coldest (radix_cache.rs:163-187); evicted handles in order. */
int vk_radix_evict_coldest(vk_radix* rc, int64_t tokens, uint64_t* evicted, int32_t cap,
                           int32_t* n_out);
/* The engine's prefill + cache_sequence (engine.rs:435-494) with the cached
 * prefix's pages aliased instead of allocated again: looks up the longest
 * cached prefix (matched tokens m), gives seq_handle the prefix's pages
 * (reference count + 1) and fresh pages for the rest of the prompt, and, when
 * the prompt continues inside a partially filled shared page, makes that page
 * private (*has_cow = 1: copy *cow_src to *cow_dst with vk_copy_blocks before
 * writing). When m < n_tokens the whole prompt is then cached under
 * cache_handle, a second handle on the same pages owned by the cache (the
 * reference caches the prompt only on a miss, engine.rs:437-441). pages_out
 * receives seq_handle's pages. Needs a bound cache. */
int vk_radix_cache_sequence(vk_radix* rc, const uint32_t* tokens, int32_t n_tokens,
                            uint64_t seq_handle, uint64_t cache_handle, int32_t* matched_tokens,
                            uint32_t* pages_out, int32_t cap, int32_t* n_pages, int32_t* cow_src,
                            int32_t* cow_dst, int32_t* has_cow);

/* ---- device memory and stream helpers for hosts without their own HIP ----- */
int vk_dev_alloc(vk_ctx* ctx, uint64_t bytes, void** out);
int vk_dev_free(vk_ctx* ctx, void* p);
int vk_memcpy_h2d(vk_ctx* ctx, void* dst, const void* src, uint64_t bytes);
int vk_memcpy_d2h(vk_ctx* ctx, void* dst, const void* src, uint64_t bytes);
int vk_memset_d(vk_ctx* ctx, void* dst, int value, uint64_t bytes);
int vk_stream_create(vk_ctx* ctx, void** out);
int vk_stream_destroy(vk_ctx* ctx, void* stream);
/* Waits for the stream, then reports misuse flags as vk_ctx_check does. */
int vk_stream_sync(vk_ctx* ctx, void* stream);
int vk_event_create(vk_ctx* ctx, void** out);
int vk_event_destroy(vk_ctx* ctx, void* ev);
int vk_event_record(vk_ctx* ctx, void* ev, void* stream);
int vk_event_elapsed_ms(vk_ctx* ctx, void* start, void* end, float* ms);

/* ---- synthetic-data utilities (benchmarks and full-size tests) ------------ */
/* dev[i] = fp16(N(0,1) * (outlier channel ? outlier_scale : 1)) from a
 * counter-based SplitMix64 stream; channel = i % row_len; a channel is an
 * outlier when SplitMix64(seed ^ OUTLIER_SALT ^ channel) % 100 == 0. */
int vk_fill_normal_f16(vk_ctx* ctx, void* dev, uint64_t n, uint64_t seed,
                       int32_t row_len, float outlier_scale, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* VELOKV_H */
