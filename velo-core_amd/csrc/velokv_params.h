// Kernel argument blocks shared by the host library and the gfx950 code object.
// Each kernel takes exactly one of these structs by value, so the host packs
// one pointer into hipModuleLaunchKernel's kernelParams.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define VK_HD __host__ __device__
#else
#define VK_HD
#endif

namespace velokv {

enum KvType : int32_t { KV_F32 = 0, KV_F16 = 1, KV_I8_REF = 2, KV_I8_BLK = 3 };
enum DType : int32_t { DT_F32 = 0, DT_F16 = 1 };

// Geometry of one layer of a pool (see include/velokv.h for the layout). The
// kernels work on blocks of 16 tokens ("tiles"); a pool whose pages hold
// 16 * page_tiles tokens stores page p as tiles p * page_tiles ..
// (p + 1) * page_tiles - 1, back to back, so a flat slot page * page_tokens +
// offset is also tile * 16 + offset % 16. The tile view (append, decode,
// commit) has n_blocks = tiles and block_size = 16; the page view (COW copy,
// NIXL) has n_blocks = pages, block_size = page tokens, page_tiles = 1 and the
// tile sizes of a whole page.
// I8_BLK scales: the K and V scale (fp16) of one (block, head) share one 4-byte
// word, K in the low half: entry (block b, head h) of a layer's scale array is
// the word b * n_kv_heads + h, so that a decode wave fetches both with one load
// (one 32-byte sector per (block, head) instead of two).
constexpr uint32_t kBlkScaleStep = 4;

struct PoolGeom {
  uint64_t layer_stride;   // bytes between layers
  uint64_t k_off, v_off;   // byte offsets of K / V codes inside a layer
  uint64_t ks_off, vs_off; // byte offsets of K / V scales inside a layer
  uint32_t tile_bytes;     // codes of one (block, head): block_size * head_dim * esz (head_dim = tile width)
  uint32_t stile_bytes;    // scales of one (block, head): 2 (I8_BLK, per 16 tokens), 4 per token (I8_REF), 0
  uint32_t s_step;         // bytes from one 16-bit unit of a kind's (K or V) scales to its next: 2 for
                           // I8_REF (contiguous), kBlkScaleStep for I8_BLK, 0 without scales
  int32_t n_blocks, n_kv_heads, block_size, head_dim, kv_type, n_layer;
  int32_t page_tiles;      // tile view: page tokens / 16
  int32_t io_hd;           // head_dim of the caller's K/V/q/out rows: any multiple of 8 up to
                           // 128; head_dim above is the tile width, 64 (io_hd <= 64) or 128,
                           // the dims past io_hd held as zeros
};

enum RopeStyle : int32_t { ROPE_NONE = 0, ROPE_INTERLEAVED = 1, ROPE_HALF = 2 };

// Misuse flags or-ed into a context's device error word (include/velokv.h
// VK_MISUSE_*); the kernels still run to completion on the clamped input.
enum Misuse : uint32_t { MISUSE_PAGE_OUT_OF_POOL = 1u, MISUSE_BLK_SPLIT_RUN = 2u };

// Append of n_tok tokens; grid (ceil(n_tok / tok_per_wg), Hkv + ceil(n_heads / 2)):
// workgroup x covers tokens [x T, x T + T) of the call, T = tok_per_wg; rows
// y < Hkv write K (wave 0) and V (wave 1) of KV head y; with RoPE, rows y >= Hkv
// rotate query heads 2(y - Hkv) and 2(y - Hkv) + 1 in place.
struct AppendParams {
  uint8_t* base;            // pool base (all layers)
  PoolGeom g;
  int32_t layer;
  int32_t in_dtype;
  const void* k;            // [n_tok][Hkv][D]
  const void* v;
  const int64_t* slot_mapping;
  int32_t n_tok;
  int32_t rope;             // RopeStyle; ROPE_NONE = plain append
  const int32_t* positions; // [n_tok] RoPE positions (rope only); null: the new token's, context_len - 1
  const float* cos_sin;     // [n_pos][D/2][2] cos, sin of pair i at each position
  int32_t n_pos;
  int32_t n_heads;          // query heads rotated (0 = none)
  void* q;                  // [n_tok][n_heads][D] of q_dtype, rotated in place unless q_out is given
  void* q_out;              // or the rotated rows go here (same shape and type), q left unchanged
  int32_t q_dtype;
  int32_t tok_per_wg;       // tokens per workgroup (1..64)
  uint32_t* err;            // the context's misuse word
  unsigned long long* claim;// I8_BLK: [n_blocks] (epoch << 32 | first token) of the last run per block
  uint32_t epoch;           // I8_BLK: this call's epoch (never 0)
  // slot_mapping == null: token m is the new token of sequence m, at position
  // min(context_lens[m], cap_tokens) - 1 of table row seq_rows[m] (or m)
  const int32_t* block_tables;
  const int32_t* seq_rows;
  const int32_t* context_lens;
  int32_t bt_stride, bt_rows, cap_tokens;
};

struct SlotMapParams {
  const int32_t* block_tables;
  const int32_t* seq_rows;
  const int32_t* positions;
  int64_t* out;
  int32_t bt_stride, block_size, n_tok, n_blocks;
};

// Paged attention over a block table. Decode: one query row per (sequence,
// head). Tree verify: n_nodes query rows per (sequence, head); node j's K/V sit
// at position context_len + j and row i sees them where bit j of tree_mask[s][i]
// is set (every row sees positions < context_len).
struct DecodeParams {
  const uint8_t* kc;        // K codes of the layer
  const uint8_t* vc;        // V codes of the layer
  const uint8_t* ks;        // K scales of the layer (or null)
  const uint8_t* vs;        // V scales
  const void* q;            // [S][N][H][D]
  float* out;               // [S][N][H][D]
  float* part_acc;          // [S][N][H][max_parts][D]
  float* part_ml;           // [S][N][H][max_parts][2] (running max in log2 units, sum)
  const int32_t* block_tables;
  const int32_t* seq_rows;
  const int32_t* context_lens;
  const uint32_t* tree_mask;// [S][N] (tree kernels only)
  uint32_t tile_bytes;
  uint32_t stile_bytes;
  int32_t bt_stride;
  int32_t bt_rows;          // rows of the block table when known (pool slot table), else 0
  int32_t n_seqs, n_heads, n_kv_heads;
  int32_t n_blocks;         // pages in the pool (block-table entries range)
  int32_t page_tiles;       // page tokens / 16: table entry p holds tiles p * page_tiles .. (p + 1) * page_tiles - 1
  int32_t io_hd;            // head_dim: q / out row length (a multiple of 8 up to 128)
  int32_t tile_hd;          // tile width, 64 or 128 (>= io_hd; the dims past io_hd hold zeros)
  int32_t max_parts;        // partitions per sequence in the grid
  int32_t part_tokens;      // tokens per partition (multiple of the block size)
  int32_t cap_tokens;       // tokens a table row can address: min(max_parts*part_tokens, bt_stride*bs)
  int32_t n_nodes;          // query rows per (sequence, head): 1 for decode
  int32_t n_rgroups;        // row groups per (sequence, KV head) in the grid (tree kernels)
  int32_t n_workers;        // stream-K: workers in the grid
  int32_t* sk_prefix;       // stream-K: [S + 1] first cost unit of each sequence, then the total C
  int32_t sk_penalty;       // stream-K: cost units charged to each segment ahead of its blocks
  float scale_log2;         // softmax scale * log2(e)
  // tree verify with a shared prefix: the first prefix_blocks pages of every
  // table row are the same pages; partial slots 0..prefix_chunks-1 of a row hold
  // the prefix pass, the partitions of the rest of the context follow
  int32_t prefix_blocks, prefix_chunks;
  uint32_t* err;            // the context's misuse word (page ids outside the pool)
  // vk_append_decode over an I8_BLK pool with the append folded into the decode
  // (null otherwise): the new K and V rows [n_seqs][n_kv_heads][io_hd] of
  // fold_dtype, the call's append epoch and the pool's per-tile claim words
  const void* fold_k;
  const void* fold_v;
  int32_t fold_dtype;
  uint32_t fold_epoch;
  unsigned long long* claim;
  int32_t fold_blocks;      // workgroup split: blocks' worth of time the append costs the wave that folds it
  // vk_append_rope_decode with the append folded in: RoPE of the new K rows (the
  // folding wave) and of every q row (each wave, in registers) at position
  // context_len - 1; positions outside [0, rope_n_pos) rotate nothing and append
  // nothing. Only with io_hd equal to the tile width (the half-split partner of
  // a q chunk sits in lane ^ 32).
  int32_t rope;             // RopeStyle
  const float* cos_sin;     // [rope_n_pos][io_hd / 2][2]
  int32_t rope_n_pos;
};

// Stream-K decode: waves per workgroup (each wave one worker, workers
// blockIdx.x * kSkWaves .. + kSkWaves - 1); fewer, larger workgroups than one
// wave each reach the device sooner.
constexpr int kSkWaves = 4;
constexpr int kMaxCopyPairs = 224;  // pairs per copy launch (kernarg limit)
// Shared-prefix pass of tree verify: pages per prefix chunk, whose page ids and
// block scales one workgroup stages in LDS (the host cuts longer prefixes into
// more chunks).
constexpr int kPfxMaxChunkBlocks = 1024;
// Its workgroup: kPfxWaves waves of kPfxRT 16-row tiles of query rows each.
constexpr int kPfxRT = 1;
constexpr int kPfxWaves = 16;
constexpr int kPfxRows = 16 * kPfxRT * kPfxWaves;  // query rows per workgroup
struct CopyParams {
  uint8_t* base;
  PoolGeom g;
  int32_t n_pairs;
  int32_t pairs[2 * kMaxCopyPairs];
};

// NIXL wire records (include/velokv.h): one launch covers up to kMaxNixlItems
// records. Work unit = (record, page i, layer l), numbered r = i * n_layers + l
// inside a record and cut into n_slices slices of kNixlSliceVecs 16-byte
// vectors (one workgroup each); unit_begin is the record's first slice in the
// launch.
constexpr int kMaxNixlItems = 80;  // kernarg limit
constexpr int kNixlSliceVecs = 256;  // 4 KB per workgroup of 256 lanes
struct NixlItemArg {
  uint64_t block_id;
  uint64_t wire_offset;  // record start (16-aligned)
  uint32_t token_len;
  int32_t first_page;    // index into pages[]
  uint32_t n_pages;      // ceil(token_len / bs)
  uint32_t unit_begin;
  uint32_t byte_len;     // payload bytes for this pool and layer range
  uint32_t pad;
};
struct NixlParams {
  uint8_t* base;         // pool base (all layers)
  PoolGeom g;
  const int32_t* pages;
  uint8_t* wire;         // written by pack, read by unpack
  uint64_t wire_bytes;
  int32_t* status;       // status of this launch's first record
  int32_t layer0, n_layers;
  int32_t unpack;        // 0: pool -> wire, 1: wire -> pool
  int32_t n_items;
  int32_t n_slices;      // slices per unit: ceil(2 * codes bytes of a page / 4 KB)
  NixlItemArg items[kMaxNixlItems];
};

// Accepted-path commit of a draft tree: grid (sequence, KV head, group of 8
// layers), two waves (K, V).
struct CommitParams {
  uint8_t* base;
  PoolGeom g;
  const int32_t* block_tables;
  const int32_t* context_lens;
  const int32_t* accept;
  const int32_t* n_accept;
  int32_t* status;          // [n_seqs] commit status per sequence, or null
  int32_t bt_stride, accept_stride, n_seqs, layer0, n_layers;
};

// Per-sequence status of a tree commit (include/velokv.h VK_COMMIT_*).
enum CommitStatus : int32_t { COMMIT_OK = 0, COMMIT_BAD_ROW = 1, COMMIT_PAST_TABLE = 2, COMMIT_BAD_PAGE = 3 };

struct MergeParams {
  const float* part_acc;
  const float* part_ml;
  const int32_t* context_lens;
  float* out;
  int32_t n_rows;           // output rows: S * rows_per_seq
  int32_t rows_per_seq;     // n_nodes * n_heads
  int32_t extra_tokens;     // tokens after context_len (tree nodes), 0 for decode
  int32_t max_parts, part_tokens, cap_tokens;
  // stream-K merge (vk_decode_merge_sk): partials indexed by (worker, slot, row of the group)
  const int32_t* sk_prefix;
  int32_t n_workers, n_kv_heads, n_seqs;
  int32_t sk_penalty;                    // stream-K cost units per segment (DecodeParams)
  int32_t prefix_blocks, prefix_chunks;  // tree verify with a shared prefix (DecodeParams)
  int32_t io_hd;                         // out row length (a multiple of 8 up to 128)
};

// Stream-K split of W cost units over nw workers of one wave each: worker w
// takes units [begin(w), begin(w + 1)), begin(w) = w W / nwe over
// nwe = min(nw, W) workers, so that no range is empty. A segment (sequence, KV
// head) of nb > 0 blocks occupies pen + nb units, its blocks after pen units
// that stand for the cost of starting a piece (a worker that starts a new
// segment gets that many fewer blocks); with pen = 0 units are blocks. The
// attention kernel and the merge derive ranges from these functions.
struct SkSplit {
  int64_t W;
  int32_t nw;  // workers with blocks
};
VK_HD inline SkSplit sk_split(int64_t W, int32_t nw) { return SkSplit{W, (int32_t)(W < nw ? W : nw)}; }
// First block of worker w (w <= nw; requires W > 0).
VK_HD inline int64_t sk_begin(const SkSplit& s, int32_t w) { return (int64_t)w * s.W / s.nw; }
// The worker whose range holds block x (0 <= x < W): the largest w with
// begin(w) <= x, i.e. ceil((x + 1) nw / W) - 1.
VK_HD inline int32_t sk_worker_of(const SkSplit& s, int64_t x) {
  return (int32_t)(((x + 1) * s.nw + s.W - 1) / s.W) - 1;
}

// Blocks [lo, hi) of the segment whose units start at seg0 (nb blocks, pen
// units ahead of them) that fall in the unit range [c0, c1); lo >= hi: none.
VK_HD inline void sk_piece(int64_t seg0, int32_t nb, int32_t pen, int64_t c0, int64_t c1, int32_t* lo, int32_t* hi) {
  const int64_t a = c0 - seg0 - pen, b = c1 - seg0 - pen;
  *lo = (int32_t)(a > 0 ? a : 0);
  *hi = (int32_t)(b < nb ? b : nb);
}
// The first and last worker holding blocks of that segment.
VK_HD inline void sk_segment_workers(const SkSplit& s, int64_t seg0, int32_t nb, int32_t pen, int32_t* w_lo,
                                     int32_t* w_hi) {
  *w_lo = sk_worker_of(s, seg0 + pen);
  *w_hi = sk_worker_of(s, seg0 + pen + nb - 1);
}

struct FillParams {
  uint16_t* dst;
  uint64_t n;
  uint64_t seed;
  int32_t row_len;
  float outlier_scale;
};

}  // namespace velokv
