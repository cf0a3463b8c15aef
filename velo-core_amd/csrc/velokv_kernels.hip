// velokv_kernels.hip -- hand-written gfx950 (CDNA4) kernels of the KV-cache hot path.
//
// Built with `hipcc --offload-arch=gfx950 --offload-device-only` into a code object
// that the host library loads with hipModuleLoad and launches with
// hipModuleLaunchKernel. Every kernel takes one argument struct (velokv_params.h).
//
// The kernels work on 16-token tiles (a page of 16 k tokens is k tiles back
// to back) and 128-dim rows in registers; a head_dim-64 pool stores 64-dim tiles,
// which the loaders read into the lower half of those rows (the upper half takes
// a copy of the lower one and meets zero q dims; outputs keep the lower half).
// The host rejects other shapes with VK_ERR_UNSUPPORTED.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#include "velokv_params.h"

using namespace velokv;

#define DEV static __device__ __forceinline__

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int BS = 16;    // tokens per block
constexpr int HD = 128;   // head_dim
constexpr int WAVE = 64;
constexpr float kNegInf = -__builtin_huge_valf();

template <typename T, typename F>
DEV T bitcast(F x) { return __builtin_bit_cast(T, x); }

DEV float h2f(uint16_t b) { return (float)bitcast<_Float16>(b); }
DEV uint16_t f2h(float x) { return bitcast<uint16_t>((_Float16)x); }  // IEEE RNE
DEV int lane_id() { return __lane_id(); }

// ---- cross-lane helpers (DPP inside a row of 16 lanes, ds_bpermute across rows)
template <int CTRL>
DEV float dpp(float x) {
  return bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(x), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int DPP_ROW_ROR4 = 0x124;
constexpr int DPP_ROW_ROR8 = 0x128;
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

DEV float shfl_xor(float x, int m) { return __shfl_xor(x, m, WAVE); }
// x of lane l ^ 32: v_permlane32_swap exchanges lanes 32..63 of its first
// operand with lanes 0..31 of its second (a VALU exchange, no LDS round trip);
// with both operands x, the second result holds x[l + 32] in lanes 0..31 and the
// first holds x[l - 32] in lanes 32..63.
DEV float xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(lane_id() < 32 ? r[1] : r[0]);
}

DEV float wave_max(float x) {
  x = fmaxf(x, dpp<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp<DPP_ROW_HALF_MIRROR>(x));
  x = fmaxf(x, dpp<DPP_ROW_MIRROR>(x));
  x = fmaxf(x, shfl_xor(x, 16));
  x = fmaxf(x, shfl_xor(x, 32));
  return x;
}
DEV float wave_sum(float x) {
  x += dpp<DPP_QUAD_XOR1>(x);
  x += dpp<DPP_QUAD_XOR2>(x);
  x += dpp<DPP_ROW_HALF_MIRROR>(x);
  x += dpp<DPP_ROW_MIRROR>(x);
  x += shfl_xor(x, 16);
  x += shfl_xor(x, 32);
  return x;
}
// Reductions over the 16 lanes that share (lane & 3).
DEV float max_same_quadpos(float x) {
  x = fmaxf(x, dpp<DPP_ROW_ROR4>(x));
  x = fmaxf(x, dpp<DPP_ROW_ROR8>(x));
  x = fmaxf(x, shfl_xor(x, 16));
  x = fmaxf(x, shfl_xor(x, 32));
  return x;
}
DEV float sum_same_quadpos(float x) {
  x += dpp<DPP_ROW_ROR4>(x);
  x += dpp<DPP_ROW_ROR8>(x);
  x += shfl_xor(x, 16);
  x += shfl_xor(x, 32);
  return x;
}
DEV float readlane_f(float x, int l) { return bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(x), l)); }
DEV int readlane_i(int x, int l) { return __builtin_amdgcn_readlane(x, l); }

// ---- int8 -> fp16 -----------------------------------------------------------
// Four signed int8 codes (little-endian bytes b0..b3) become two fp16 pairs that
// hold the codes exactly: (b0,b1) and (b2,b3). XOR 0x80 turns each byte into
// offset binary u = c + 128; v_perm_b32 places u under the exponent byte 0x64,
// which is the fp16 value 1024 + u; subtracting 1152 leaves c.
DEV void i8x4_to_h2x2(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = bitcast<uint32_t>(bitcast<half2v>(a) - bias);
  hi = bitcast<uint32_t>(bitcast<half2v>(b) - bias);
}
DEV float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(bitcast<half2v>(a), bitcast<half2v>(b), c, false);
}
DEV float byte_to_f(uint32_t w, int byte) { return (float)(int8_t)((w >> (8 * byte)) & 0xFFu); }
DEV float half_lo(uint32_t w) { return h2f((uint16_t)(w & 0xFFFFu)); }
DEV float half_hi(uint32_t w) { return h2f((uint16_t)(w >> 16)); }
// Two fp32 values to an fp16 pair, each rounded to nearest even: one
// v_cvt_pk_f16_f32.
typedef float f32x2 __attribute__((ext_vector_type(2)));
DEV uint32_t pack_h2(float a, float b) {
  const f32x2 x = {a, b};
  return bitcast<uint32_t>(__builtin_convertvector(x, half2v));
}

template <int KV> struct Esz;
template <> struct Esz<KV_F32> { static constexpr int v = 4; };
template <> struct Esz<KV_F16> { static constexpr int v = 2; };
template <> struct Esz<KV_I8_REF> { static constexpr int v = 1; };
template <> struct Esz<KV_I8_BLK> { static constexpr int v = 1; };

// Per-lane vector of N dwords loaded with as few instructions as possible. K/V
// tiles are read exactly once per decode, so the loads are marked non-temporal.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int N> struct DW { uint32_t d[N]; };
template <int N>
DEV DW<N> load_dw(const uint8_t* p) {
  DW<N> r;
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
      r.d[4 * i] = v.x; r.d[4 * i + 1] = v.y; r.d[4 * i + 2] = v.z; r.d[4 * i + 3] = v.w;
    }
  } else if constexpr (N == 2) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    r.d[0] = v.x; r.d[1] = v.y;
  } else {
    r.d[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
  }
  return r;
}

// =============================================================================
// Paged decode attention, split-K partial pass.
//
// One wave (= one workgroup) owns one unit (sequence s, KV head kvh, partition
// part of at most 256 blocks). The partition streams through a two-stage software
// pipeline: while the K and V tiles of batch b (CH blocks) are consumed, the loads
// of batch b+1 are already in flight.
//   scores  K tile [tok][D]: lane = (token lane>>2, 32-dim slice lane&3). Dot
//           products with the G query heads of the GQA group are summed over the
//           quad; the lane keeps the score of (its token, head (lane&3)+4k).
//   softmax running max M per head, updated lazily: only when some score of the
//           batch exceeds M by more than 2^4 is M raised to the exact batch max
//           and the accumulators rescaled, so p = 2^(score - M) <= 16 always.
//           p~ = p * v_scale goes to LDS as (token pair, head) pairs.
//   values  V tile [tok/2][D][2]: lane = (dims 2*lane, 2*lane+1), all 16 tokens;
//           acc[g][d] += p~_2j * v_2j[d] + p~_2j+1 * v_2j+1[d].
// FAST (q fp16 and fp16/int8 KV): v_dot2_f32_f16 on exact int8->fp16 codes and
// fp16 p~ pairs. Otherwise fp32 FMA on dequantized values.
// The unit writes unnormalised partials (acc, M in log2 units, l = sum p);
// vk_decode_merge combines the partitions of a sequence.
// Algorithm of kernels.metal:440-501 / 672-732 and llama_cpu.rs:255-284.
// =============================================================================
// ---- split-K: units with nparts > 1 store unnormalised partials (acc, M in log2
// units, l = sum p); vk_decode_merge combines them in a second launch. A device-
// scope release per unit would write back the XCD's whole L2 (buffer_wbl2), so
// the merge is not fused into this kernel.
// An empty context attends to nothing: the first partition unit writes zeros.
template <int G>
DEV void write_zero_rows(const DecodeParams& P, int s, int kvh) {
  const int64_t hrow0 = (int64_t)s * P.n_heads + (int64_t)kvh * G;
#pragma unroll
  for (int g = 0; g < G; ++g) reinterpret_cast<float2*>(P.out)[(hrow0 + g) * (HD / 2) + lane_id()] = make_float2(0.f, 0.f);
}

// GQA group size of a kernel: the template's G, or for G == 0 (the "_gx" kernels
// that serve any other ratio) the runtime n_heads / n_kv_heads.
template <int G>
DEV int group_size(const DecodeParams& P) { return G > 0 ? G : P.n_heads / P.n_kv_heads; }
// Rows of one (sequence, KV head) a workgroup holds in LDS for group size G:
// runtime group sizes are at most 16 (one 16-row tile).
template <int G>
constexpr int lds_rows() { return G > 0 ? G : 16; }
DEV void write_zero_rows_n(const DecodeParams& P, int s, int kvh, int g_n) {
  const int64_t hrow0 = (int64_t)s * P.n_heads + (int64_t)kvh * g_n;
  if (2 * lane_id() >= P.io_hd) return;
  for (int g = 0; g < g_n; ++g)
    reinterpret_cast<float2*>(P.out)[(hrow0 + g) * (P.io_hd / 2) + lane_id()] = make_float2(0.f, 0.f);
}

// Misuse is reported, not trapped: the kernel or-s a flag into the context's
// error word (a vector atomic) and carries on with the clamped input.
DEV void flag_misuse(uint32_t* err, uint32_t bit) {
  if (err) __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr float kRescaleThreshold = 4.0f;  // log2 units
// Block ids (and per-(block, head) scales) of a unit, held one per lane in up to
// kWin windows of 64 blocks: partitions of up to 256 blocks (4096 tokens).
constexpr int kWin = 4;
struct BlockIds {
  int b[kWin];
  uint32_t sw[kWin];  // I8_BLK: the (K, V) scale word of the lane's (block, head), K low, V high (fp16)
  uint32_t oob;       // bit k: the page of this lane's block in window k was outside the pool
};
// A page id outside [0, n_blocks) is clamped into the pool (the read stays in
// bounds) and reported as MISUSE_PAGE_OUT_OF_POOL. Tile u of a sequence (tokens
// 16u .. 16u + 15) is tile u % page_tiles of page bt[u / page_tiles]. Lanes
// past the piece's nblk blocks hold its last block. Every load is issued
// outside any branch (lanes past nblk read the last block's entries) and the
// scale words are kept as loaded: a load in a branch, or a use here, would wait
// for it, and the windows' table and scale loads would complete one after
// another before the piece's first tile loads go out.
template <bool BLK>
DEV void load_block_ids(BlockIds& w, const DecodeParams& P, const int32_t* bt, int blk0, int nblk, int kvh) {
  const int lane = lane_id();
  const uint32_t pt = (uint32_t)P.page_tiles;
  const int last = max(nblk - 1, 0);
  int raw[kWin];
#pragma unroll
  for (int k = 0; k < kWin; ++k) raw[k] = bt[(uint32_t)(blk0 + min(64 * k + lane, last)) / pt];
  bool bad = false;
  w.oob = 0u;
#pragma unroll
  for (int k = 0; k < kWin; ++k) {
    const int idx = 64 * k + lane;
    const int u = blk0 + min(idx, last);
    const bool out = idx < nblk && (raw[k] < 0 || raw[k] >= P.n_blocks);
    bad |= out;
    w.oob |= out ? 1u << k : 0u;
    w.b[k] = min(max(raw[k], 0), P.n_blocks - 1) * (int)pt + (int)((uint32_t)u % pt);
    w.sw[k] = 0u;
    if constexpr (BLK)  // the (K, V) scale word of the (block, head): one load
      w.sw[k] = *reinterpret_cast<const uint32_t*>(P.ks + ((int64_t)w.b[k] * P.n_kv_heads + kvh) * kBlkScaleStep);
  }
  if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) flag_misuse(P.err, MISUSE_PAGE_OUT_OF_POOL);
}
// Value of block i (wave-uniform) from a per-lane window array: each window is
// read at lane i % 64 and the window i / 64 is selected among the (scalar)
// results, so the array stays in registers (a select over the array elements
// themselves is turned into a dynamically indexed array in memory).
template <typename T>
DEV T window_at(const T (&a)[kWin], int i) {
  const int k = i >> 6, l = i & 63;
  int v = readlane_i(bitcast<int>(a[0]), l);
#pragma unroll
  for (int j = 1; j < kWin; ++j) {
    const int w = readlane_i(bitcast<int>(a[j]), l);
    v = (k == j) ? w : v;
  }
  return bitcast<T>(v);
}
// I8_BLK block scales of block i (wave-uniform) of a piece.
DEV float blk_kscale(const BlockIds& w, int i) { return half_lo(window_at(w.sw, i)); }
DEV float blk_vscale(const BlockIds& w, int i) { return half_hi(window_at(w.sw, i)); }

template <int KV>
struct Stage {
  static constexpr int ESZ = Esz<KV>::v;
  static constexpr int CH = (ESZ == 1) ? 2 : 1;  // blocks per pipeline stage
  DW<8 * ESZ> k[CH];
  DW<ESZ> v[CH][8];
  float ks[CH];  // VK_KV_I8_REF: K scale of the lane's token
  float vs[CH];  // VK_KV_I8_REF: V scale of the lane's token
};

// Buffer resource over one tile: base address and size in SGPRs, so the per-lane
// offset stays a fixed VGPR and address registers never alias load results.
// Word 3 = 0x00020000 (32-bit data format, the gfx9-family raw-buffer setting).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
DEV rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // the base is wave-uniform by construction; say so, so the descriptor lives in SGPRs
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  void* u = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, 0, (int)__builtin_amdgcn_readfirstlane((int)bytes), 0x00020000);
}
// A stage past the end of a piece (the pipeline issues one or two) or a block
// past the piece in a partly used stage takes a descriptor of zero bytes: its
// loads are issued as usual (the same instructions and wait counts on every
// path, so the pipeline keeps its loads in flight; a branch around them made the
// compiler wait for every outstanding load at the join) but are out of range,
// return zeros and move no bytes. Clamping them to the last block instead
// re-read up to four tiles per piece, 1.8 % of a ragged call's HBM traffic.
DEV uint32_t stage_bytes(int i, int nblk, uint32_t bytes) { return i < nblk ? bytes : 0u; }

// Cache policy of tile loads: V is streamed non-temporally. K rows are split
// over several load instructions (each covers a half (int8) or a quarter (fp16)
// of every 128-byte line of the tile), so K stays in the normal L2 policy unless
// its elements are bytes, where non-temporal measured faster.
constexpr int kAuxNT = 2;
template <int ESZ>
constexpr int k_aux() { return ESZ == 1 ? kAuxNT : 0; }
template <int N, int AUX = kAuxNT>
DEV DW<N> buf_load(rsrc_t r, uint32_t off) {
  DW<N> out;
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + 16 * i), 0, AUX);
      out.d[4 * i] = v.x; out.d[4 * i + 1] = v.y; out.d[4 * i + 2] = v.z; out.d[4 * i + 3] = v.w;
    }
  } else if constexpr (N == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, AUX);
    out.d[0] = v.x; out.d[1] = v.y;
  } else {
    out.d[0] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, AUX);
  }
  return out;
}

// Issue the loads of batch `b` (blocks b*CH .. b*CH+CH-1 of the unit; blocks past
// the unit load zeros through zero-size descriptors, so the tail needs no branch).
template <int KV>
DEV void stage_load(Stage<KV>& st, const DecodeParams& P, const BlockIds& bw, int b, int nblk, int kvh, int t) {
  constexpr int ESZ = Esz<KV>::v;
  constexpr int CH = Stage<KV>::CH;
  const int lane = lane_id();
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int i = min(b * CH + u, nblk - 1);
    const int blk = window_at(bw.b, i);
    const uint64_t tix = (uint64_t)blk * P.n_kv_heads + kvh;
    const uint32_t tb = stage_bytes(b * CH + u, nblk, P.tile_bytes);
    const rsrc_t kr = make_rsrc(P.kc + tix * P.tile_bytes, tb);
    const rsrc_t vr = make_rsrc(P.vc + tix * P.tile_bytes, tb);
    if constexpr (ESZ == 1) {  // lane 4t + c: pieces at 16 lane and 1024 + 16 lane (int8 K layout)
      const DW<4> lo = buf_load<4, k_aux<ESZ>()>(kr, lane * 16);
      const DW<4> hi = buf_load<4, k_aux<ESZ>()>(kr, 1024 + lane * 16);
#pragma unroll
      for (int w = 0; w < 4; ++w) { st.k[u].d[w] = lo.d[w]; st.k[u].d[4 + w] = hi.d[w]; }
    } else {
      st.k[u] = buf_load<8 * ESZ, k_aux<ESZ>()>(kr, lane * (32 * ESZ));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) st.v[u][j] = buf_load<ESZ>(vr, j * (HD * 2 * ESZ) + lane * (4 * ESZ));
    if constexpr (KV == KV_I8_REF) {
      const uint32_t sb = stage_bytes(b * CH + u, nblk, P.stile_bytes);
      const rsrc_t sr = make_rsrc(P.ks + tix * P.stile_bytes, sb);
      const rsrc_t svr = make_rsrc(P.vs + tix * P.stile_bytes, sb);
      st.ks[u] = bitcast<float>(__builtin_amdgcn_raw_buffer_load_b32(sr, t * 4, 0, 0));
      st.vs[u] = bitcast<float>(__builtin_amdgcn_raw_buffer_load_b32(svr, t * 4, 0, 0));
    }
  }
}

template <int KV, int G, int QT>
DEV void decode_unit(const DecodeParams& P) {
  constexpr int ESZ = Esz<KV>::v;
  constexpr bool FAST = (QT == DT_F16) && (KV != KV_F32);
  constexpr bool BLK = (KV == KV_I8_BLK);
  constexpr bool REF = (KV == KV_I8_REF);
  constexpr int CH = Stage<KV>::CH;
  constexpr int SPL = (G >= 4) ? G / 4 : 1;   // score slots per lane per block
  constexpr int QW = FAST ? 16 : 32;          // q registers per head
  constexpr int PW = FAST ? 1 : 2;            // LDS dwords per (pair, head)

  __shared__ uint32_t p_lds[CH * 8 * G * PW];

  const int lane = lane_id();
  const int t = lane >> 2;   // token of the K tile this lane reads
  const int c = lane & 3;    // 32-dim slice of the K tile

  const int unit = blockIdx.x;
  const int kvh = unit % P.n_kv_heads;
  const int rest = unit / P.n_kv_heads;
  const int part = rest % P.max_parts;
  const int s = rest / P.max_parts;
  if (s >= P.n_seqs) return;

  const int ctx = max(0, min(P.context_lens[s], P.cap_tokens));
  const int start = part * P.part_tokens;
  if (start >= ctx) {
    if (part == 0) write_zero_rows<G>(P, s, kvh);
    return;
  }
  const int end = min(start + P.part_tokens, ctx);
  const int nparts = (ctx + P.part_tokens - 1) / P.part_tokens;
  int row = P.seq_rows ? P.seq_rows[s] : s;
  if (P.bt_rows > 0) row = min(max(row, 0), P.bt_rows - 1);
  const int32_t* bt = P.block_tables + (int64_t)row * P.bt_stride;
  const int H = P.n_heads;
  const int Hkv = P.n_kv_heads;
  const int nblk = (end - start + BS - 1) / BS;   // <= 64 * kWin
  const int blk0 = start / BS;
  const int nbatch = (nblk + CH - 1) / CH;

  // block ids (and per-(block, head) scales) of the unit, one block per lane
  BlockIds bw;
  load_block_ids<BLK>(bw, P, bt, blk0, nblk, kvh);

  Stage<KV> sa, sb;
  stage_load<KV>(sa, P, bw, 0, nblk, kvh, t);

  // ---- query registers: 32 dims (slice c) of each head of the group ---------
  uint32_t qh[G][QW];
  {
    const int64_t qoff = ((int64_t)s * H + (int64_t)kvh * G) * HD + c * 32;
    if constexpr (QT == DT_F16) {
      const uint16_t* q16 = reinterpret_cast<const uint16_t*>(P.q) + qoff;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint4* q4 = reinterpret_cast<const uint4*>(q16 + g * HD);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 v = q4[i];
          if constexpr (FAST) {
            qh[g][4 * i + 0] = v.x; qh[g][4 * i + 1] = v.y;
            qh[g][4 * i + 2] = v.z; qh[g][4 * i + 3] = v.w;
          } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              qh[g][8 * i + 2 * k] = bitcast<uint32_t>(half_lo(w[k]));
              qh[g][8 * i + 2 * k + 1] = bitcast<uint32_t>(half_hi(w[k]));
            }
          }
        }
      }
    } else {
      const float* q32 = reinterpret_cast<const float*>(P.q) + qoff;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint4* q4 = reinterpret_cast<const uint4*>(q32 + g * HD);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint4 v = q4[i];
          qh[g][4 * i + 0] = v.x; qh[g][4 * i + 1] = v.y;
          qh[g][4 * i + 2] = v.z; qh[g][4 * i + 3] = v.w;
        }
      }
    }
  }

  // head held by score slot k of this lane, and whether the lane owns it
  auto slot_head = [&](int k) -> int { return (G >= 4) ? c + 4 * k : c % G; };
  const bool owner = (G >= 4) || (c < G);

  float M[G];        // running max per head (log2 units), wave-uniform
  float Mlane[SPL];  // M of the head of each slot of this lane
  float lrun[SPL];   // per-lane partial softmax denominators
  float acc[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) { M[g] = kNegInf; acc[g][0] = 0.f; acc[g][1] = 0.f; }
#pragma unroll
  for (int k = 0; k < SPL; ++k) { lrun[k] = 0.f; Mlane[k] = kNegInf; }
  const int last_valid = (end - start) - (nblk - 1) * BS;  // valid tokens in the last block

  auto compute = [&](const Stage<KV>& st, int b) {
    float sc[CH][SPL];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = b * CH + u;
      float a[G];
#pragma unroll
      for (int g = 0; g < G; ++g) a[g] = 0.f;
      if constexpr (FAST) {
        if constexpr (ESZ == 1) {
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            uint32_t lo, hi;
            i8x4_to_h2x2(st.k[u].d[w], lo, hi);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              a[g] = dot2(qh[g][2 * w], lo, a[g]);
              a[g] = dot2(qh[g][2 * w + 1], hi, a[g]);
            }
          }
        } else {
#pragma unroll
          for (int w = 0; w < 16; ++w)
#pragma unroll
            for (int g = 0; g < G; ++g) a[g] = dot2(qh[g][w], st.k[u].d[w], a[g]);
        }
      } else {
        float kf[32];
#pragma unroll
        for (int d = 0; d < 32; ++d) {
          if constexpr (ESZ == 1) kf[d] = byte_to_f(st.k[u].d[d >> 2], d & 3);
          else if constexpr (ESZ == 2) kf[d] = (d & 1) ? half_hi(st.k[u].d[d >> 1]) : half_lo(st.k[u].d[d >> 1]);
          else kf[d] = bitcast<float>(st.k[u].d[d]);
        }
#pragma unroll
        for (int d = 0; d < 32; ++d)
#pragma unroll
          for (int g = 0; g < G; ++g) a[g] = fmaf(bitcast<float>(qh[g][d]), kf[d], a[g]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        a[g] += dpp<DPP_QUAD_XOR1>(a[g]);
        a[g] += dpp<DPP_QUAD_XOR2>(a[g]);
      }
      float kscale = P.scale_log2;
      if constexpr (BLK) kscale *= blk_kscale(bw, min(i, nblk - 1));
      if constexpr (REF) kscale *= st.ks[u];
      const bool valid = (i < nblk) && (start + i * BS + t < end);
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        float v;
        if constexpr (G >= 4) {
          v = a[4 * k];
          v = (c == 1) ? a[4 * k + 1] : v;
          v = (c == 2) ? a[4 * k + 2] : v;
          v = (c == 3) ? a[4 * k + 3] : v;
        } else if constexpr (G == 2) {
          v = (c & 1) ? a[1] : a[0];
        } else {
          v = a[0];
        }
        sc[u][k] = valid ? v * kscale : kNegInf;
      }
    }

    // lazy running max: rescale only when a score passes M + threshold
    bool need = false;
#pragma unroll
    for (int u = 0; u < CH; ++u)
#pragma unroll
      for (int k = 0; k < SPL; ++k) need |= sc[u][k] > Mlane[k] + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      float mb[SPL];
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        float m = sc[0][k];
#pragma unroll
        for (int u = 1; u < CH; ++u) m = fmaxf(m, sc[u][k]);
        mb[k] = max_same_quadpos(m);
      }
      float alpha[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float m;
        if constexpr (G >= 4) m = readlane_f(mb[g / 4], g % 4);
        else if constexpr (G == 2) m = readlane_f(mb[0], g);
        else m = readlane_f(mb[0], 0);
        const float Mn = fmaxf(M[g], m);
        alpha[g] = __builtin_amdgcn_exp2f(M[g] - Mn);  // 0 while M is -inf
        M[g] = Mn;
        acc[g][0] *= alpha[g];
        acc[g][1] *= alpha[g];
      }
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        float al = alpha[0], ml = M[0];
#pragma unroll
        for (int g = 1; g < G; ++g) {
          al = (slot_head(k) == g) ? alpha[g] : al;
          ml = (slot_head(k) == g) ? M[g] : ml;
        }
        lrun[k] *= al;
        Mlane[k] = ml;
      }
    }

    // p and p~ = p * v_scale into LDS as (token pair, head) pairs
    const int jp = t >> 1, e = t & 1;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = b * CH + u;
      if (i < nblk) {
        float vscale = 1.f;
        if constexpr (BLK) vscale = blk_vscale(bw, i);
        if constexpr (REF) vscale = st.vs[u];
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
          const float p = __builtin_amdgcn_exp2f(sc[u][k] - Mlane[k]);
          if (owner) {
            lrun[k] += p;
            const int g = slot_head(k);
            if constexpr (FAST)
              reinterpret_cast<uint16_t*>(p_lds)[(((u * 8 + jp) * G + g) << 1) + e] = f2h(p * vscale);
            else
              reinterpret_cast<float*>(p_lds)[(((u * 8 + jp) * G + g) << 1) + e] = p * vscale;
          }
        }
      }
    }
    __asm__ volatile("" ::: "memory");

    // values
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = b * CH + u;
      if (i < nblk) {
        const bool partial = (i == nblk - 1) && (last_valid < BS);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint32_t pp[G * PW];
          const uint32_t* src = p_lds + (u * 8 + j) * G * PW;
          if constexpr (G * PW >= 4) {
#pragma unroll
            for (int q4 = 0; q4 < G * PW / 4; ++q4) {
              const uint4 v = reinterpret_cast<const uint4*>(src)[q4];
              pp[4 * q4] = v.x; pp[4 * q4 + 1] = v.y; pp[4 * q4 + 2] = v.z; pp[4 * q4 + 3] = v.w;
            }
          } else if constexpr (G * PW == 2) {
            const uint2 v = reinterpret_cast<const uint2*>(src)[0];
            pp[0] = v.x; pp[1] = v.y;
          } else {
            pp[0] = src[0];
          }
          const bool z0 = partial && (2 * j >= last_valid);
          const bool z1 = partial && (2 * j + 1 >= last_valid);
          if constexpr (FAST) {
            uint32_t v0, v1;
            if constexpr (ESZ == 1) i8x4_to_h2x2(st.v[u][j].d[0], v0, v1);
            else { v0 = st.v[u][j].d[0]; v1 = st.v[u][j].d[1]; }
            if (partial) {
              const uint32_t m = (z0 ? 0u : 0xFFFFu) | (z1 ? 0u : 0xFFFF0000u);
              v0 &= m; v1 &= m;
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
              acc[g][0] = dot2(pp[g], v0, acc[g][0]);
              acc[g][1] = dot2(pp[g], v1, acc[g][1]);
            }
          } else {
            float v00, v01, v10, v11;  // v[d][tok]
            if constexpr (ESZ == 1) {
              const uint32_t w = st.v[u][j].d[0];
              v00 = byte_to_f(w, 0); v01 = byte_to_f(w, 1); v10 = byte_to_f(w, 2); v11 = byte_to_f(w, 3);
            } else if constexpr (ESZ == 2) {
              v00 = half_lo(st.v[u][j].d[0]); v01 = half_hi(st.v[u][j].d[0]);
              v10 = half_lo(st.v[u][j].d[1]); v11 = half_hi(st.v[u][j].d[1]);
            } else {
              v00 = bitcast<float>(st.v[u][j].d[0]); v01 = bitcast<float>(st.v[u][j].d[1]);
              v10 = bitcast<float>(st.v[u][j].d[2]); v11 = bitcast<float>(st.v[u][j].d[3]);
            }
            if (z0) { v00 = 0.f; v10 = 0.f; }
            if (z1) { v01 = 0.f; v11 = 0.f; }
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const float pe = bitcast<float>(pp[2 * g]);
              const float po = bitcast<float>(pp[2 * g + 1]);
              acc[g][0] = fmaf(po, v01, fmaf(pe, v00, acc[g][0]));
              acc[g][1] = fmaf(po, v11, fmaf(pe, v10, acc[g][1]));
            }
          }
        }
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  // two-stage pipeline over the batches of the unit
  for (int b = 0; b < nbatch; b += 2) {
    stage_load<KV>(sb, P, bw, b + 1, nblk, kvh, t);
    compute(sa, b);
    if (b + 1 >= nbatch) break;
    stage_load<KV>(sa, P, bw, b + 2, nblk, kvh, t);
    compute(sb, b + 1);
  }

  // ---- partials of this unit ----
  float lsum[G];
#pragma unroll
  for (int k = 0; k < SPL; ++k) lrun[k] = sum_same_quadpos(lrun[k]);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if constexpr (G >= 4) lsum[g] = readlane_f(lrun[g / 4], g % 4);
    else lsum[g] = readlane_f(lrun[0], g);
  }
  const int64_t hrow0 = (int64_t)s * H + (int64_t)kvh * G;
  if (nparts == 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float inv = 1.f / lsum[g];
      reinterpret_cast<float2*>(P.out)[(hrow0 + g) * (HD / 2) + lane] = make_float2(acc[g][0] * inv, acc[g][1] * inv);
    }
    return;
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t pr = (hrow0 + g) * P.max_parts + part;
    reinterpret_cast<float2*>(P.part_acc + pr * HD)[lane] = make_float2(acc[g][0], acc[g][1]);
    if (lane == g) reinterpret_cast<float2*>(P.part_ml)[pr] = make_float2(M[g], lsum[g]);
  }
}

// =============================================================================
// Paged attention on the matrix cores: decode (one query row per head) and tree
// verify (one row per (node, head)), with the unit, partials and pool layout of
// decode_unit; fp16 (or fp32, rounded) q with fp16 or int8 KV.
//
// Scores, transposed: S^T[t][r] = v_mfma_f32_16x16x32_f16(A = K block, B = q^T)
//   over 4 chunks of 32 dims: rows = the 16 tokens of a block, columns = 16 query
//   rows (heads of the GQA group, or (node, head) pairs, zero-padded). Lane l
//   (n = l&15, g = l>>4) feeds K[token n][dims 32g..32g+31] and
//   q[row n][dims 32g..32g+31]: both operands see the same dim permutation, so
//   each lane reads 32 contiguous bytes of one token row. Lane l gets S for
//   tokens 4g..4g+3 of query row n -- exactly the A operand p[row n][tokens
//   4g..4g+3] of the value product, so p never leaves the registers, and each
//   lane keeps the softmax state (running max, sums) of one row.
// Values: out[r][d] += v_mfma_f32_16x16x16f16 per block and per 16-dim tile; the
//   B operand is V[tokens 4g..4g+3][dim 8n + tile] taken from the token pairs 2g
//   and 2g+1 of the block (16 contiguous bytes each). Lane l gets
//   out[rows 4g..4g+3][dims 8n..8n+7].
// int8 codes enter the matrix cores as fp16 (1152 + c) without the subtraction;
//   sum_d q_d (1152 + c_d) - 1152 sum_d q_d and sum_t p~_t (1152 + c_t) -
//   1152 sum_t p~_t remove the bias exactly up to fp32 rounding.
// Softmax: lazy running max as in decode_unit (rescale only when a score exceeds
//   the row's max by more than 2^4).
// =============================================================================
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

// D: the dims a kernel is built for, 128 or 64. A 64-dim kernel gives each lane
// half the dims (K: 16 per token, V: 4 per token pair), so a block takes two
// score and four value products instead of four and eight.
template <int KV, int D = HD>
struct MStage {
  static constexpr int ESZ = Esz<KV>::v;
  // blocks per pipeline stage: two int8 blocks or one fp16 block at 128 dims (8 KB
  // of K and V), two blocks at 64 dims (measured: four int8 blocks per stage at
  // two waves per SIMD lost to two at three waves per SIMD; one fp16 block lost
  // to two)
  static constexpr int CH = (ESZ == 1 || D < HD) ? 2 : 1;
  DW<(D / 16) * ESZ> k[CH];     // token n, dims 32g..32g+31 (D = 64: 16g..16g+15)
  DW<(D / 32) * ESZ> v[CH][2];  // token pairs 2g, 2g+1; dims 8n..8n+7 (D = 64: 4n..4n+3)
  float4 ks[CH];                // VK_KV_I8_REF: scales of tokens 4g..4g+3
  float4 vs[CH];
};

// Tiles of a head_dim-64 pool are 64 dims wide: lanes whose 32-dim chunk (K) or
// 8-dim group (V) lies past dim 63 read the same bytes as the lane 64 dims below
// (the chunk g & 1, the group n & 7), so a tile is fetched once; those K dims meet
// zero q dims and those output dims are dropped.
template <int KV, int DK = HD>
DEV void mstage_load(MStage<KV, DK>& st, const DecodeParams& P, const BlockIds& bw, int b, int nblk, int kvh, int n,
                     int g) {
  constexpr int ESZ = Esz<KV>::v;
  constexpr int CH = MStage<KV, DK>::CH;
  const int D = DK == HD ? P.tile_hd : DK;
  const int gk = g & (D / 32 - 1), nv = n & (D / 8 - 1);
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int i = min(b * CH + u, nblk - 1);
    const int blk = window_at(bw.b, i);
    const uint64_t tix = (uint64_t)blk * P.n_kv_heads + kvh;
    const uint32_t tb = stage_bytes(b * CH + u, nblk, P.tile_bytes);
    const rsrc_t kr = make_rsrc(P.kc + tix * P.tile_bytes, tb);
    const rsrc_t vr = make_rsrc(P.vc + tix * P.tile_bytes, tb);
    if constexpr (DK == 64) {
      // K dims 16g..16g+15 of token n: int8 half g & 1 of 32-dim chunk g >> 1
      // (byte 8 D h + (n D/32 + c) 16), fp16 32 contiguous bytes; V dims
      // 4n..4n+3 of token pairs 2g + r (8 elements of the pair row)
      if constexpr (ESZ == 1)
        st.k[u] = buf_load<4, k_aux<ESZ>()>(kr, (g & 1) * 8 * DK + (n * 2 + (g >> 1)) * 16);
      else
        st.k[u] = buf_load<8, k_aux<ESZ>()>(kr, (n * DK + 16 * g) * 2);
#pragma unroll
      for (int r = 0; r < 2; ++r) st.v[u][r] = buf_load<2 * ESZ>(vr, ((2 * g + r) * DK * 2 + 8 * n) * ESZ);
    } else {
      if constexpr (ESZ == 1) {  // pieces (n D/32 + g) of the two halves of 8 D bytes (int8 K layout)
        const DW<4> lo = buf_load<4, k_aux<ESZ>()>(kr, (n * (D / 32) + gk) * 16);
        const DW<4> hi = buf_load<4, k_aux<ESZ>()>(kr, 8 * D + (n * (D / 32) + gk) * 16);
#pragma unroll
        for (int w = 0; w < 4; ++w) { st.k[u].d[w] = lo.d[w]; st.k[u].d[4 + w] = hi.d[w]; }
      } else {
        st.k[u] = buf_load<8 * ESZ, k_aux<ESZ>()>(kr, (n * D + 32 * gk) * ESZ);
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) st.v[u][r] = buf_load<4 * ESZ>(vr, ((2 * g + r) * D * 2 + 16 * nv) * ESZ);
    }
    if constexpr (KV == KV_I8_REF) {
      const uint32_t sb = stage_bytes(b * CH + u, nblk, P.stile_bytes);
      const rsrc_t sr = make_rsrc(P.ks + tix * P.stile_bytes, sb);
      const rsrc_t svr = make_rsrc(P.vs + tix * P.stile_bytes, sb);
      st.ks[u] = bitcast<float4>(__builtin_amdgcn_raw_buffer_load_b128(sr, g * 16, 0, 0));
      st.vs[u] = bitcast<float4>(__builtin_amdgcn_raw_buffer_load_b128(svr, g * 16, 0, 0));
    }
  }
}

// ---- RoPE (fused into the append) --------------------------------------------
// Pair i of a head row at position p is rotated by the table's (cos, sin) of
// angle p * base^(-2i/D), D the caller's head_dim: ROPE_INTERLEAVED pairs dims (2i, 2i+1)
// (kernels.metal:103-131), ROPE_HALF pairs dims (i, i + D/2)
// (llama_cpu.rs:113-131). y0 = x0 c - x1 s, y1 = x0 s + x1 c in fp32 with
// every product and sum rounded separately (no fused multiply-add), the
// reference's expression order. Lane l holds dims 2l, 2l+1 of the row.
// D = any multiple of 4 up to 128 (the half-split partners of the lane's dims,
// d + D/2 or d - D/2, then sit together in lane l + D/4 or l - D/4): lanes
// 2l >= D hold zeros and stay zero.
// rope_rotate in two steps: rope_cs loads the 16-byte table chunk that holds
// the lane's (cos, sin) values, with no branch and no use (so that it can be
// issued with other loads and wait for nothing), and rope_apply takes the
// values from it and rotates. Interleaved: pair `lane` of the row (D/2 pairs of
// (cos, sin)) is in chunk lane / 2, .xy for even lanes, .zw for odd ones;
// half-split: pairs 2 lh, 2 lh + 1 of the lane's place lh in its half are chunk
// lh. Lanes past the row read chunk 0.
DEV float4 rope_cs(int style, const float* cos_sin, int pos, int D) {
  const int lane = lane_id();
  const int hl = D / 4;  // lanes of one half of the row
  const int lh = lane < hl ? lane : lane - hl;
  int c = style == ROPE_HALF ? lh : lane >> 1;
  c = 2 * lane < D ? c : 0;
  return reinterpret_cast<const float4*>(cos_sin + (int64_t)pos * D)[c];
}

DEV void rope_apply(int style, const float4 t, int D, float& x0, float& x1) {
#pragma clang fp contract(off)
  const int lane = lane_id();
  const int hl = D / 4;
  if (style == ROPE_INTERLEAVED) {
    if (2 * lane < D) {
      const float2 cs = (lane & 1) ? make_float2(t.z, t.w) : make_float2(t.x, t.y);
      const float y0 = x0 * cs.x - x1 * cs.y;
      const float y1 = x0 * cs.y + x1 * cs.x;
      x0 = y0;
      x1 = y1;
    }
  } else {
    const int lh = lane < hl ? lane : lane - hl;                             // the lane's place in its half
    const float p0 = __shfl(x0, lane < hl ? lane + hl : lh, WAVE);          // dims d -+ D/2
    const float p1 = __shfl(x1, lane < hl ? lane + hl : lh, WAVE);
    if (2 * lane >= D) return;
    if (lane < hl) {  // first half: y = x c - partner s
      const float y0 = x0 * t.x - p0 * t.y;
      const float y1 = x1 * t.z - p1 * t.w;
      x0 = y0;
      x1 = y1;
    } else {          // second half: y = partner s + x c
      const float y0 = p0 * t.y + x0 * t.x;
      const float y1 = p1 * t.w + x1 * t.z;
      x0 = y0;
      x1 = y1;
    }
  }
}

DEV void rope_rotate(int style, const float* cos_sin, int pos, int D, float& x0, float& x1) {
  rope_apply(style, rope_cs(style, cos_sin, pos, D), D, x0, x1);
}

// RoPE of a lane's q chunks in the matrix-core pieces (vk_append_rope_decode):
// chunk kc holds dims d0 = 8 (KC g + kc) .. d0 + 7 of row R (zeros when R is
// past the tile's rows). The rotation of rope_rotate at the table row of the new
// token's position (D = head_dim), in its expression order, every product and
// sum rounded separately: ROPE_INTERLEAVED pairs (2i, 2i + 1) within the chunk;
// ROPE_HALF pairs d with d + D/2, whose chunk is the same chunk of lane l ^ 32
// (lane group g ^ 2 holds the dims D/2 further on, at D = 64 and 128), fetched
// with one lane exchange per value. A position outside the table leaves q as it is.
// rope_q_issue issues every load of q and of the table, none in a branch,
// before the piece's first tile loads; rope_q_finish rotates while those are
// in flight (its waits count only the loads issued before them), both styles
// in one branch-free form (selects, not a branch on the style, so that no load
// is sunk into a branch and waited for behind the tile loads):
//   y_j = x_j c - p s   (interleaved, j even; half-split, first half)
//   y_j = p s + x_j c   (interleaved, j odd;  half-split, second half)
// with p the partner value (x_{j^1}, or lane l ^ 32's x_j).
template <int QT, int KC>
struct RopeQ {
  uint4 raw[KC][QT == DT_F32 ? 2 : 1];  // q chunks as loaded
  float4 t[KC][4];  // pairs 2h', 2h' + 1 of the chunk: interleaved h' = h / 2 (d0/2 + ..), half h' = h (df + ..)
  bool row_ok, rot;
};

// qoff: the lane's chunks of row R; qoff_ok: a row of q that exists, read by
// lanes past the rows (they then take zeros); pos: the new token's position.
template <int QT, int KC>
DEV void rope_q_issue(RopeQ<QT, KC>& r, const DecodeParams& P, int64_t qoff, int64_t qoff_ok, bool row_ok, int pos,
                      int g) {
  const int D = P.io_hd;
  const bool half = P.rope == ROPE_HALF;
  r.row_ok = row_ok;
  r.rot = pos >= 0 && pos < P.rope_n_pos;
  const float* csr = P.cos_sin + (int64_t)(r.rot ? pos : 0) * D;
  const int64_t qo = row_ok ? qoff : qoff_ok;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    if constexpr (QT == DT_F32) {
      const uint4* q32 = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(P.q) + qo) + 2 * kc;
      r.raw[kc][0] = q32[0];
      r.raw[kc][1] = q32[1];
    } else {
      r.raw[kc][0] = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.q) + qo)[kc];
    }
  }
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    const int d0 = 8 * (KC * g + kc);
    const int df = d0 < D / 2 ? d0 : d0 - D / 2;
#pragma unroll
    for (int h = 0; h < 4; ++h)
      r.t[kc][h] = *reinterpret_cast<const float4*>(half ? csr + 2 * df + 4 * h : csr + d0 + 4 * (h >> 1));
  }
}

template <int QT, int KC, bool QSPLIT>
DEV void rope_q_finish(const RopeQ<QT, KC>& r, const DecodeParams& P, int g, half8 (&qa)[KC], half8 (&qlo)[KC]) {
#pragma clang fp contract(off)
  const int D = P.io_hd;
  const bool half = P.rope == ROPE_HALF;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    float x[8];
    if constexpr (QT == DT_F32) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        x[4 * u + 0] = __uint_as_float(r.raw[kc][u].x);
        x[4 * u + 1] = __uint_as_float(r.raw[kc][u].y);
        x[4 * u + 2] = __uint_as_float(r.raw[kc][u].z);
        x[4 * u + 3] = __uint_as_float(r.raw[kc][u].w);
      }
    } else {
      const half8 h = bitcast<half8>(r.raw[kc][0]);
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (float)h[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = r.row_ok ? x[j] : 0.f;
    const bool first = 8 * (KC * g + kc) < D / 2;
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float ph = xor32(x[j]);
      const float p = half ? ph : x[j ^ 1];
      const float4 tt = r.t[kc][j >> 1];
      const bool zw = half ? (j & 1) != 0 : ((j >> 1) & 1) != 0;  // pair 2h' + 1 of t
      const float c = zw ? tt.z : tt.x, sn = zw ? tt.w : tt.y;
      const bool form1 = half ? first : (j & 1) == 0;
      y[j] = form1 ? x[j] * c - p * sn : p * sn + x[j] * c;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = r.rot ? y[j] : x[j];
    const uint4 v = make_uint4(pack_h2(x[0], x[1]), pack_h2(x[2], x[3]), pack_h2(x[4], x[5]), pack_h2(x[6], x[7]));
    qa[kc] = bitcast<half8>(v);
    qlo[kc] = bitcast<half8>(make_uint4(0, 0, 0, 0));
    if constexpr (QSPLIT) {
      const half8 h = qa[kc];
      qlo[kc] = bitcast<half8>(make_uint4(pack_h2(x[0] - (float)h[0], x[1] - (float)h[1]),
                                          pack_h2(x[2] - (float)h[2], x[3] - (float)h[3]),
                                          pack_h2(x[4] - (float)h[4], x[5] - (float)h[5]),
                                          pack_h2(x[6] - (float)h[6], x[7] - (float)h[7])));
    }
  }
}

// ---- KV append helpers (shared by the append kernels and the folded append) ----
DEV void load_x2(const void* src, int in_dtype, int64_t off, float& x0, float& x1) {
  if (in_dtype == DT_F16) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(src) + off)[0];
    x0 = half_lo(w); x1 = half_hi(w);
  } else {
    const float2 v = reinterpret_cast<const float2*>(reinterpret_cast<const float*>(src) + off)[0];
    x0 = v.x; x1 = v.y;
  }
}

// Byte offset inside a (block, head) tile of element (token, dim), D = head_dim
// (64 or 128):
//   V: [tok/2][D][2] (token pairs interleaved)
//   K, fp16 / fp32: [tok][D]
//   K, int8: [h][tok][D/32][16] with h = (d/16) % 2: the 32 codes of dims
//     32c..32c+31 of token t are two 16-byte pieces at (t D/32 + c)*16 and
//     8 D + (t D/32 + c)*16, so one 16-byte load per lane covers whole cache lines
template <bool IS_V>
DEV uint32_t tile_elem(int tok, int d, int esz, int D) {
  if (IS_V) return (uint32_t)(((tok >> 1) * D + d) * 2 + (tok & 1)) * esz;
  if (esz == 1) return (uint32_t)(((d >> 4) & 1) * 8 * D + (tok * (D >> 5) + (d >> 5)) * 16 + (d & 15));
  return (uint32_t)(tok * D + d) * esz;
}

DEV int clamp127(float r) { return (int)fminf(fmaxf(r, -127.f), 127.f); }

// The I8_BLK rule for one new token x (dims 2*lane, 2*lane + 1) at offset o of
// a block whose scale is s_old:
//   s_new = max(s_old, fp16(amax / 127))
//   if s_new > s_old: c' = clamp(rne((c * s_old) / s_new)) for tokens before o
//   c = s_new > 0 ? clamp(rne(x / s_new)) : 0
// s_new of the row; s_bits becomes its fp16 bits when it grows.
DEV float blk_scale(float s_old, uint16_t& s_bits, float x0, float x1) {
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const uint16_t cand = f2h(amax / 127.0f);
  if (h2f(cand) > s_old) {
    s_bits = cand;
    return h2f(cand);
  }
  return s_old;
}
DEV int blk_requant(int c, float s_old, float s_new) { return clamp127(__builtin_rintf(((float)c * s_old) / s_new)); }
DEV int blk_code(float x, float s_new) { return (s_new > 0.f) ? clamp127(__builtin_rintf(x / s_new)) : 0; }

// The rule over a block whose codes are in registers (cd) and whose scale is
// s_old (bits s_bits).
DEV void blk_put(int (&cd)[BS][2], int o, float& s_old, uint16_t& s_bits, float x0, float x1) {
  const float s_new = blk_scale(s_old, s_bits, x0, x1);
  if (s_new > s_old && o > 0) {
#pragma unroll
    for (int u = 0; u < BS; ++u) {
      if (u < o) {
#pragma unroll
        for (int k = 0; k < 2; ++k) cd[u][k] = blk_requant(cd[u][k], s_old, s_new);
      }
    }
  }
  const int c0 = blk_code(x0, s_new);
  const int c1 = blk_code(x1, s_new);
#pragma unroll
  for (int u = 0; u < BS; ++u)
    if (u == o) { cd[u][0] = c0; cd[u][1] = c1; }
  s_old = s_new;
}

// ---- the append of vk_append_decode inside the decode launch (I8_BLK; fp16
// pools under stream-K store the new rows as they are, fold_finish) ----------
// The piece that holds a sequence's last context token (position ctx - 1)
// appends the sequence's new K and V rows there before it loads that block: the
// rule of append_blk_run for a run of one token at offset o = (ctx - 1) % 16
// (s_old = 0 when o = 0), lane l holding dims 2l, 2l+1, then attends over the
// block as rewritten (its stores come before its own loads of the block in the
// wave's program order). fold_issue issues the loads of the new rows and the
// stored scales beside the piece's first loads; fold_finish applies the rule
// and stores the new token's codes, and when the scale grows loads, requantizes
// and stores the codes of the tokens before o. A page id outside the pool
// appends nothing (the decode reports it), as the append kernel drops such a
// slot. For I8_BLK the block's codes come with the first loads too (whole
// 16-byte pieces, and the V token pair of o), so that a requantization waits
// for no load: K pieces hold one token each and are rewritten whole when that
// token is before o; V pieces hold a token pair and are rewritten whole when
// both are before o; the pair holding o is stored by the lanes of the rule
// (dims 2 lane, 2 lane + 1) as one word with token o's codes, so no two stores
// of the call overlap.
struct FoldIn {
  uint32_t w[2][2];       // [K, V] new-token dims 2 lane, 2 lane + 1 as loaded (fp16: both in w[e][0])
  float x[2][2];          // the same as fp32 (fold_finish)
  float4 cs;              // RoPE: the lane's table chunk at ctx - 1 (rope_cs)
  uint32_t sw;            // I8_BLK: the block's scale word as loaded (K low, V high)
  uint4 kq[2], vq[2];     // I8_BLK: 16-byte pieces lane + 64 j of the K and V tiles (j < D / 64)
  uint32_t vpair;         // I8_BLK: V codes of tokens 2P, 2P + 1 (P = o / 2) at dims 2 lane, 2 lane + 1
  unsigned long long claim_old;
  uint64_t tix;           // (tile, KV head) index of the block
  int o;
  bool on;
};

// Loads of the folded append of sequence s, KV head kvh, whose piece holds nblk
// blocks (window bw), the last one holding position ctx - 1 (I8_BLK: also the
// block's stored scales; fp16 pools store the new rows as they are). Every load
// is issued whether or not the append happens (f.on), from an address that
// exists, and none is used here: a use here, or a load in a branch, would wait
// for them (and, vector loads completing in order, for nothing more) before the
// piece's first tile loads go out, on the folding wave's critical path.
template <int KV, int D, bool ROPE = false>
DEV void fold_issue(FoldIn& f, const DecodeParams& P, const BlockIds& bw, int nblk, int s, int kvh, int ctx) {
  const int i = nblk - 1;
  f.on = ((readlane_i((int)bw.oob, i & 63) >> (i >> 6)) & 1) == 0;
  // with RoPE, a position outside the table appends nothing (as the RoPE append skips it)
  if constexpr (ROPE) {
    if (ctx - 1 < 0 || ctx - 1 >= P.rope_n_pos) f.on = false;
  }
  const int tile_id = f.on ? window_at(bw.b, i) : 0;
  f.tix = (uint64_t)tile_id * P.n_kv_heads + kvh;
  f.o = (ctx - 1) & (BS - 1);
  // the claim of the block (one run per block and call), checked after the piece
  f.claim_old = 0;
  if (P.claim && f.on && kvh == 0 && lane_id() == 0)
    f.claim_old = __hip_atomic_exchange(&P.claim[tile_id], ((unsigned long long)P.fold_epoch << 32) | (uint32_t)s,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the new rows are io_hd long; lanes past it read dim 0 and take zeros (fold_finish)
  const int d0 = 2 * lane_id();
  const int64_t row = ((int64_t)s * P.n_kv_heads + kvh) * P.io_hd + (d0 < P.io_hd ? d0 : 0);
  const bool f16 = P.fold_dtype == DT_F16;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t* src = f16 ? reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(e ? P.fold_v : P.fold_k) + row)
                              : reinterpret_cast<const uint32_t*>(reinterpret_cast<const float*>(e ? P.fold_v : P.fold_k) + row);
    f.w[e][0] = src[0];
    f.w[e][1] = src[f16 ? 0 : 1];
  }
  // RoPE of the new K row: the table chunk now, the rotation in fold_finish
  if constexpr (ROPE) f.cs = rope_cs(P.rope, P.cos_sin, f.on ? ctx - 1 : 0, P.io_hd);
  if constexpr (KV == KV_I8_BLK) {
    f.sw = *reinterpret_cast<const uint32_t*>(P.ks + f.tix * kBlkScaleStep);
    const uint4* kt = reinterpret_cast<const uint4*>(P.kc + f.tix * P.tile_bytes);
    const uint4* vt = reinterpret_cast<const uint4*>(P.vc + f.tix * P.tile_bytes);
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      f.kq[j] = kt[lane_id() + 64 * j];
      f.vq[j] = vt[lane_id() + 64 * j];
    }
    f.vpair = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(vt) +
                                                 tile_elem<true>(f.o & ~1, d0 & (D - 1), 1, D));
  }
}

DEV int byte_at(uint32_t w, int k) { return (int)(int8_t)(uint8_t)(w >> (8 * k)); }

// The rule for K (IS_V false) or V; returns the block's new scale (fp16 bits). Lanes past a
// 64-dim row read the codes 64 dims below and store nothing. K codes of token u
// at dims 2 lane, 2 lane + 1 are two adjacent bytes; V codes of the token pair
// 2p, 2p + 1 are four (dim 2 lane: tokens 2p, 2p + 1; then dim 2 lane + 1).
DEV uint32_t blk_requant4(uint32_t w, float s_old, float s_new) {
  uint32_t r = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) r |= (uint32_t)(blk_requant(byte_at(w, k), s_old, s_new) & 0xFF) << (8 * k);
  return r;
}
DEV uint4 blk_requant16(uint4 v, float s_old, float s_new) {
  return make_uint4(blk_requant4(v.x, s_old, s_new), blk_requant4(v.y, s_old, s_new), blk_requant4(v.z, s_old, s_new),
                    blk_requant4(v.w, s_old, s_new));
}

template <bool IS_V, int D>
DEV uint32_t fold_finish_one(FoldIn& f, const DecodeParams& P) {
  const int e = IS_V ? 1 : 0;
  const int o = f.o;
  const int lane = lane_id();
  const int d0 = 2 * lane, da = d0 & (D - 1);
  const bool st = d0 < D;
  const uint16_t stored = (uint16_t)(e ? f.sw >> 16 : f.sw & 0xFFFFu);
  const float s_old = (o == 0) ? 0.f : h2f(stored);
  uint16_t s_bits = (o == 0) ? (uint16_t)0 : stored;
  const float s_new = blk_scale(s_old, s_bits, f.x[e][0], f.x[e][1]);
  const bool grew = s_new > s_old && o > 0;  // requantize the tokens before o
  uint8_t* tile = const_cast<uint8_t*>(IS_V ? P.vc : P.kc) + f.tix * P.tile_bytes;
  const int c0 = blk_code(f.x[e][0], s_new), c1 = blk_code(f.x[e][1], s_new);
  if constexpr (!IS_V) {
    if (grew) {
#pragma unroll
      for (int j = 0; j < D / 64; ++j) {
        const int q = lane + 64 * j;
        if ((q % (D / 2)) / (D / 32) < o)  // the piece's token
          reinterpret_cast<uint4*>(tile)[q] = blk_requant16(f.kq[j], s_old, s_new);
      }
    }
    if (st)
      *reinterpret_cast<uint16_t*>(tile + tile_elem<false>(o, da, 1, D)) = (uint16_t)((c0 & 0xFF) | ((c1 & 0xFF) << 8));
  } else {
    if (grew) {
#pragma unroll
      for (int j = 0; j < D / 64; ++j) {
        const int q = lane + 64 * j;
        if (q / (D / 8) < (o >> 1))  // the piece's token pair
          reinterpret_cast<uint4*>(tile)[q] = blk_requant16(f.vq[j], s_old, s_new);
      }
    }
    if (st) {  // bytes: (2P, d0), (2P + 1, d0), (2P, d0 + 1), (2P + 1, d0 + 1)
      uint32_t w = f.vpair;
      if (o & 1) {  // token o - 1 (requantized when the scale grew), then token o
        int a0 = byte_at(w, 0), a1 = byte_at(w, 2);
        if (grew) {
          a0 = blk_requant(a0, s_old, s_new);
          a1 = blk_requant(a1, s_old, s_new);
        }
        w = (uint32_t)(a0 & 0xFF) | ((uint32_t)(c0 & 0xFF) << 8) | ((uint32_t)(a1 & 0xFF) << 16) |
            ((uint32_t)(c1 & 0xFF) << 24);
      } else {      // token o, then token o + 1 as it was (not yet written)
        w = (uint32_t)(c0 & 0xFF) | (w & 0xFF00u) | ((uint32_t)(c1 & 0xFF) << 16) | (w & 0xFF000000u);
      }
      *reinterpret_cast<uint32_t*>(tile + tile_elem<true>(o & ~1, da, 1, D)) = w;
    }
  }
  if (lane == 0)
    *reinterpret_cast<uint16_t*>(const_cast<uint8_t*>(IS_V ? P.vs : P.ks) + f.tix * kBlkScaleStep) = s_bits;
  return s_bits;  // h2f(s_bits) == s_new
}

// One run per block and call, as in append_blk: a second sequence whose new
// token lands in the same block (claimed in this call) is reported. Checked
// after the piece, when the claim's old value has long arrived.
DEV void fold_claim_check(const FoldIn& f, const DecodeParams& P, int s) {
  if (f.on && P.claim && lane_id() == 0 && f.tix % P.n_kv_heads == 0) {
    const unsigned long long me = ((unsigned long long)P.fold_epoch << 32) | (uint32_t)s;
    if ((uint32_t)(f.claim_old >> 32) == P.fold_epoch && f.claim_old != me) flag_misuse(P.err, MISUSE_BLK_SPLIT_RUN);
  }
}

// The rule, the stores, and the block's new scales in bw.
template <int KV, int D, bool ROPE = false>
DEV void fold_finish(FoldIn& f, const DecodeParams& P, BlockIds& bw, int nblk, int s) {
  if (!f.on) return;
  const int lane = lane_id();
  const bool in_row = 2 * lane < P.io_hd;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    if (P.fold_dtype == DT_F16) {
      f.x[e][0] = half_lo(f.w[e][0]);
      f.x[e][1] = half_hi(f.w[e][0]);
    } else {
      f.x[e][0] = __uint_as_float(f.w[e][0]);
      f.x[e][1] = __uint_as_float(f.w[e][1]);
    }
    f.x[e][0] = in_row ? f.x[e][0] : 0.f;
    f.x[e][1] = in_row ? f.x[e][1] : 0.f;
  }
  // RoPE of the new K row before the append rule, as the RoPE append rotates it
  if constexpr (ROPE) rope_apply(P.rope, f.cs, P.io_hd, f.x[0][0], f.x[0][1]);
  if constexpr (KV == KV_F16) {  // the new rows rounded to fp16 (RNE), as vk_append_kv1 stores them
    const int d0 = 2 * lane;
    if (d0 < D) {
      uint8_t* kt = const_cast<uint8_t*>(P.kc) + f.tix * P.tile_bytes;
      uint8_t* vt = const_cast<uint8_t*>(P.vc) + f.tix * P.tile_bytes;
      *reinterpret_cast<uint16_t*>(kt + tile_elem<false>(f.o, d0, 2, D)) = f2h(f.x[0][0]);
      *reinterpret_cast<uint16_t*>(kt + tile_elem<false>(f.o, d0 + 1, 2, D)) = f2h(f.x[0][1]);
      *reinterpret_cast<uint16_t*>(vt + tile_elem<true>(f.o, d0, 2, D)) = f2h(f.x[1][0]);
      *reinterpret_cast<uint16_t*>(vt + tile_elem<true>(f.o, d0 + 1, 2, D)) = f2h(f.x[1][1]);
    }
    return;
  }
  const uint32_t ks = fold_finish_one<false, D>(f, P);
  const uint32_t vs = fold_finish_one<true, D>(f, P);
  const int i = nblk - 1;
#pragma unroll
  for (int k = 0; k < kWin; ++k) {
    if (k == (i >> 6) && lane == (i & 63)) bw.sw[k] = ks | (vs << 16);
  }
}

// Tokens of a sequence with ctx committed tokens that a shared prefix of pb
// pages covers: whole pages only, so that the rest of the context starts on a
// page boundary.
DEV int prefix_tokens_of(int ctx, int pb) { return min(ctx / BS, pb) * BS; }

// Four int8 codes -> two fp16 pairs holding 1152 + c exactly (no subtraction).
DEV void i8x4_to_h2x2_biased(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

DEV float f4_at(const float4& v, int r) { return r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w; }

// Rows of a unit: RT tiles of 16 query rows. Row R of the (sequence, KV head)
// pair is (node R / G, head kvh*G + R % G); decode has one node.
// An fp32 q (QT == DT_F32) is split into fp16 hi + lo parts for the matrix cores.
// One piece of work: tokens [start, end) of (sequence s, KV head kvh), row group
// rg, committed context ctx_c. direct: the piece is the whole context and writes
// normalised rows; otherwise it writes the unnormalised partial (acc, M, l) of
// row R at index TREE ? out_row(R) * max_parts + pbase : pbase + R * pstride of
// pacc ([.][HD] fp32) and pml ([.][2] fp32), in HBM or in LDS.
template <int KV, int G, int RT, bool TREE, int QT, int D = HD, bool FOLD = false, bool ROPE = false>
DEV void attn_piece(const DecodeParams& P, int s, int kvh, int rg, int start, int end, int ctx_c, bool direct,
                    int64_t pbase, int pstride, float* pacc, float* pml, int npre = 0) {
  constexpr int ESZ = Esz<KV>::v;
  constexpr bool I8 = (ESZ == 1);
  constexpr bool BLK = (KV == KV_I8_BLK);
  constexpr bool REF = (KV == KV_I8_REF);
  constexpr int CH = MStage<KV, D>::CH;
  constexpr float kBias = 1152.0f;
  constexpr int KC = D / 32;   // score products per block (8 dims of each lane group each)
  constexpr int NT = D / 16;   // value tiles: lane n holds output dims (128 / D) 4 n + nt
  constexpr int DL = D / 16;   // output dims per lane

  const int lane = lane_id();
  const int n = lane & 15;   // K token (A operand) / query row (scores, p) / dim group (values)
  const int g = lane >> 4;   // dim slice (operands) / token group (scores, p, values) / row group (results)
  const int N = TREE ? P.n_nodes : 1;
  int row = P.seq_rows ? P.seq_rows[s] : s;
  if (P.bt_rows > 0) row = min(max(row, 0), P.bt_rows - 1);
  const int32_t* bt = P.block_tables + (int64_t)row * P.bt_stride;
  const int H = P.n_heads;
  const int nblk = (end - start + BS - 1) / BS;
  const int blk0 = start / BS;
  const int nbatch = (nblk + CH - 1) / CH;
  const int Gn = group_size<G>(P);
  const int nrows = N * Gn;
  const int row0 = rg * 16 * RT;
  const int plain_end = min(end, ctx_c);  // tokens below this need no validity or mask test
  // output row of row R of this (sequence, KV head) pair
  auto out_row = [&](int R) -> int64_t { return ((int64_t)s * N + R / Gn) * H + (int64_t)kvh * Gn + R % Gn; };

  BlockIds bw;
  load_block_ids<BLK>(bw, P, bt, blk0, nblk, kvh);

  // vk_append_decode with the append folded in: this piece holds the last token
  // and appends it (after the first stage's loads and q, unless the block is in
  // the first stage)
  static_assert(!FOLD || ((BLK || KV == KV_F16) && !TREE), "the folded append is the I8_BLK and fp16 decode's");
  static_assert(!ROPE || FOLD, "RoPE folds with the folded append");
  // vk_append_decode with the append folded in: this piece holds the last token.
  // Its block in the first stage: append before any tile load; otherwise issue
  // the append's loads now and finish it after q, while the first stage is in
  // flight
  bool fold = false;
  if constexpr (FOLD) fold = P.fold_k != nullptr && end == ctx_c && nblk > 0;
  const bool fold_first = fold && nblk <= CH;
  FoldIn fin;
  if constexpr (FOLD) {
    if (fold) fold_issue<KV, D, ROPE>(fin, P, bw, nblk, s, kvh, ctx_c);
    if (fold_first) fold_finish<KV, D, ROPE>(fin, P, bw, nblk, s);
  }

  // vk_append_rope_decode: q rotated in registers at the new token's position
  // (ctx_c - 1), as the RoPE append would have rotated it in memory; its loads
  // go out before the first stage's
  static_assert(!ROPE || RT == 1, "the RoPE decode has one tile of rows");
  constexpr bool QSPLIT = (QT == DT_F32);
  RopeQ<QT, KC> rq;
  if constexpr (ROPE)
    rope_q_issue<QT, KC>(rq, P, out_row(row0 + n) * P.io_hd + 8 * KC * g, out_row(0) * P.io_hd + 8 * KC * g,
                         row0 + n < nrows, ctx_c - 1, g);

  MStage<KV, D> sa, sb;
  mstage_load<KV, D>(sa, P, bw, 0, nblk, kvh, n, g);

  // q^T as the B operand: row n of each tile (rows >= nrows are zero and their
  // results are dropped), dims 32g..32g+31 in 4 chunks (D = 64: 16g..16g+15 in 2). An fp32 q
  // is split as q = hi + lo, hi = fp16(q), lo = fp16(q - hi), and each score
  // takes two products (hi, then lo, into the same accumulator), so the scores
  // see q to about 2^-22 instead of fp16's 2^-11.
  half8 qa[RT][KC];
  half8 qlo[RT][KC];
  // int8 K enters the score products as fp16 1152 + c (two v_perm per four
  // codes) and the decode subtracts qb = 1152 * sum_d q[row n][d] (of hi + lo
  // when split) from each score; its fp32 sums then carry 1152 sum q, rounded in
  // proportion to sum |q| (within the north-star tolerance for queries with x30
  // outlier channels). Tree verify subtracts 1152 from the codes in fp16 first
  // (exact) and needs no qb: its fp32 queries keep their precision.
  constexpr bool KBIAS = I8 && !TREE;
  float qb[RT];
  uint32_t mrow[RT];   // tree: mask row of row n's node
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int R = row0 + 16 * rt + n;
    float qsum = 0.f;
    // q rows are io_hd long (a multiple of 8): the 8-dim chunks past it are zero
    const int64_t qoff = out_row(R) * P.io_hd + 8 * KC * g;
    if constexpr (ROPE) {
      rope_q_finish<QT, KC, QSPLIT>(rq, P, g, qa[rt], qlo[rt]);
    } else {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        uint4 v = make_uint4(0, 0, 0, 0), vlo = make_uint4(0, 0, 0, 0);
        if (R < nrows && 8 * (KC * g + kc) < P.io_hd) {
          if constexpr (QT == DT_F32) {
            const float4* q32 = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(P.q) + qoff) + 2 * kc;
            const float4 x0 = q32[0], x1 = q32[1];
            v = make_uint4(pack_h2(x0.x, x0.y), pack_h2(x0.z, x0.w), pack_h2(x1.x, x1.y), pack_h2(x1.z, x1.w));
            if constexpr (QSPLIT) {
              const half8 h = bitcast<half8>(v);
              vlo = make_uint4(pack_h2(x0.x - (float)h[0], x0.y - (float)h[1]), pack_h2(x0.z - (float)h[2], x0.w - (float)h[3]),
                               pack_h2(x1.x - (float)h[4], x1.y - (float)h[5]), pack_h2(x1.z - (float)h[6], x1.w - (float)h[7]));
            }
          } else {
            v = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.q) + qoff)[kc];
          }
        }
        qa[rt][kc] = bitcast<half8>(v);
        qlo[rt][kc] = bitcast<half8>(vlo);
      }
    }
    if constexpr (KBIAS) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int j = 0; j < 8; ++j) qsum += QSPLIT ? (float)qa[rt][kc][j] + (float)qlo[rt][kc][j] : (float)qa[rt][kc][j];
    }
    qb[rt] = 0.f;
    if constexpr (KBIAS) {
      qsum += shfl_xor(qsum, 16);
      qsum += shfl_xor(qsum, 32);   // full sum of row n
      qb[rt] = kBias * qsum;
    }
    mrow[rt] = 0u;
    if constexpr (TREE) {
      if (R < nrows) mrow[rt] = P.tree_mask[(int64_t)s * N + R / Gn];
    }
  }
  if constexpr (FOLD) {
    if (fold && !fold_first) fold_finish<KV, D, ROPE>(fin, P, bw, nblk, s);
  }

  float M[RT], lrun[RT], psum[RT];   // state of row n (each lane holds a quarter of the row's sums)
  float4v acc[RT][NT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    M[rt] = kNegInf; lrun[rt] = 0.f; psum[rt] = 0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = float4v{0.f, 0.f, 0.f, 0.f};
  }
  const int last_valid = (end - start) - (nblk - 1) * BS;
  const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

  auto compute = [&](const MStage<KV, D>& st, int b) {
    // ---- S^T of every block of the stage (independent MFMA chains) ----
    float4v sc[RT][CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) sc[rt][u] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        uint32_t kb[4];
        if constexpr (I8) {
          i8x4_to_h2x2_biased(st.k[u].d[2 * kc], kb[0], kb[1]);
          i8x4_to_h2x2_biased(st.k[u].d[2 * kc + 1], kb[2], kb[3]);
          if constexpr (!KBIAS) {  // (1152 + c) - 1152 = c exactly
            const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
            for (int w = 0; w < 4; ++w) kb[w] = bitcast<uint32_t>(bitcast<half2v>(kb[w]) - bias);
          }
        } else {
#pragma unroll
          for (int w = 0; w < 4; ++w) kb[w] = st.k[u].d[4 * kc + w];
        }
        const u32x4 kbv = {kb[0], kb[1], kb[2], kb[3]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          sc[rt][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<half8>(kbv), qa[rt][kc], sc[rt][u], 0, 0, 0);
        if constexpr (QSPLIT) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            sc[rt][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<half8>(kbv), qlo[rt][kc], sc[rt][u], 0, 0, 0);
        }
      }
    }
    // ---- scaled scores (log2 units) of tokens 4g..4g+3, row n ----
    float sv[RT][CH][4];
    bool need = false;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = b * CH + u;
      const int tpos0 = start + i * BS + 4 * g;
      // wave-uniform: every token of the block is committed context inside the partition
      const bool plain = (i < nblk) && (start + (i + 1) * BS <= plain_end);
      float kscale = P.scale_log2;
      if constexpr (BLK) kscale *= blk_kscale(bw, min(i, nblk - 1));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float ksr = kscale;
          if constexpr (REF) ksr *= f4_at(st.ks[u], r);
          float x = KBIAS ? (sc[rt][u][r] - qb[rt]) * ksr : sc[rt][u][r] * ksr;
          if (!plain) {
            const int tpos = tpos0 + r;
            bool ok = (i < nblk) && tpos < end;
            if constexpr (TREE) {
              const int j = tpos - ctx_c;  // tree node of this token when >= 0 (< N <= 32)
              ok = ok && (j < 0 || ((mrow[rt] >> (j & 31)) & 1u));
            }
            x = ok ? x : kNegInf;
          }
          sv[rt][u][r] = x;
          need |= x > M[rt] + kRescaleThreshold;
        }
    }
    // ---- lazy running max of row n ----
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float m = sv[rt][0][0];
#pragma unroll
        for (int u = 0; u < CH; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) m = fmaxf(m, sv[rt][u][r]);
        m = fmaxf(m, shfl_xor(m, 16));
        m = fmaxf(m, shfl_xor(m, 32));  // max over the stage's tokens of row n
        const float Mn = fmaxf(M[rt], m);
        const float alpha = (Mn == kNegInf) ? 1.f : __builtin_amdgcn_exp2f(M[rt] - Mn);
        M[rt] = Mn;
        lrun[rt] *= alpha;
        psum[rt] *= alpha;
        // acc holds rows 4g..4g+3: their factors live in lanes 4g..4g+3
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * g + r, WAVE);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[rt][nt][r] *= ar;
        }
      }
    }
    // ---- p = 2^(s - M), p~ = fp16(p * v_scale): the A operand of the value product ----
    half4 pa[RT][CH];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float Ms = (M[rt] == kNegInf) ? 0.f : M[rt];  // a row that has seen nothing keeps p = 0
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int i = b * CH + u;
        float vscale = 1.f;
        if constexpr (BLK) vscale = blk_vscale(bw, min(i, nblk - 1));
        float ph[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(sv[rt][u][r] - Ms);
          lrun[rt] += p;
          float vsr = vscale;
          if constexpr (REF) vsr = f4_at(st.vs[u], r);
          ph[r] = p * vsr;
        }
        const uint32_t lo = pack_h2(ph[0], ph[1]), hi = pack_h2(ph[2], ph[3]);
        if constexpr (I8) psum[rt] = dot2(hi, bitcast<uint32_t>(ones), dot2(lo, bitcast<uint32_t>(ones), psum[rt]));
        pa[rt][u] = bitcast<half4>(make_uint2(lo, hi));
      }
    }
    // ---- values ----
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = b * CH + u;
      if (i < nblk) {
        const bool partial = (i == nblk - 1) && (last_valid < BS);
#pragma unroll
        for (int w = 0; w < KC * ESZ; w += ESZ) {
          uint32_t b0[2], b1[2];   // [pair row] for tiles nt0, nt1
          int nt0, nt1;
          if constexpr (I8) {
            i8x4_to_h2x2_biased(st.v[u][0].d[w], b0[0], b1[0]);
            i8x4_to_h2x2_biased(st.v[u][1].d[w], b0[1], b1[1]);
            nt0 = 2 * w; nt1 = 2 * w + 1;
          } else {
            b0[0] = st.v[u][0].d[w]; b1[0] = st.v[u][0].d[w + 1];
            b0[1] = st.v[u][1].d[w]; b1[1] = st.v[u][1].d[w + 1];
            nt0 = w; nt1 = w + 1;
            if (partial) {  // fp16 bytes past the context may be anything, NaN included
#pragma unroll
              for (int r = 0; r < 2; ++r) {
                const int t0 = 4 * g + 2 * r;
                const uint32_t m = (t0 < last_valid ? 0xFFFFu : 0u) | (t0 + 1 < last_valid ? 0xFFFF0000u : 0u);
                b0[r] &= m; b1[r] &= m;
              }
            }
          }
          const uint2 v0 = make_uint2(b0[0], b0[1]), v1 = make_uint2(b1[0], b1[1]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            acc[rt][nt0] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[rt][u], bitcast<half4>(v0), acc[rt][nt0], 0, 0, 0);
            acc[rt][nt1] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[rt][u], bitcast<half4>(v1), acc[rt][nt1], 0, 0, 0);
          }
        }
      }
    }
  };

  if constexpr (BLK && !TREE && !QSPLIT) {
    // three-stage pipeline: two stages in flight while one is consumed (the tree
    // kernels read mostly cached prefix pages and keep two stages so that two
    // waves fit per SIMD; an I8_REF stage also carries the per-token scales, and
    // the lo parts of a split fp32 q take the registers of a third stage)
    MStage<KV, D> sc2;
    mstage_load<KV, D>(sb, P, bw, 1, nblk, kvh, n, g);
    for (int b = 0; b < nbatch; b += 3) {
      mstage_load<KV, D>(sc2, P, bw, b + 2, nblk, kvh, n, g);
      compute(sa, b);
      if (b + 1 >= nbatch) break;
      mstage_load<KV, D>(sa, P, bw, b + 3, nblk, kvh, n, g);
      compute(sb, b + 1);
      if (b + 2 >= nbatch) break;
      mstage_load<KV, D>(sb, P, bw, b + 4, nblk, kvh, n, g);
      compute(sc2, b + 2);
    }
  } else {
    for (int b = 0; b < nbatch; b += 2) {
      mstage_load<KV, D>(sb, P, bw, b + 1, nblk, kvh, n, g);
      compute(sa, b);
      if (b + 1 >= nbatch) break;
      mstage_load<KV, D>(sa, P, bw, b + 2, nblk, kvh, n, g);
      compute(sb, b + 1);
    }
  }

  // ---- one shared-prefix chunk (the common fold): its partials of every row
  // this lane writes are loaded at once, before the first output store, so the
  // fold waits for one round trip (loads issued row by row each waited for the
  // previous row's loads and stores: vector memory counts both) ----
  const bool fold1 = direct && npre == 1;  // wave-uniform
  float2 pm1[RT][4];
  float4 pa1[RT][4][DL / 4];
  if (fold1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int R = min(row0 + 16 * rt + 4 * g + r, nrows - 1);  // rows past the last are not stored
        const int64_t pr = out_row(R) * P.max_parts;
        pm1[rt][r] = reinterpret_cast<const float2*>(P.part_ml)[pr];
        const float4* src = reinterpret_cast<const float4*>(P.part_acc + pr * HD + DL * n);
#pragma unroll
        for (int q4 = 0; q4 < DL / 4; ++q4) pa1[rt][r][q4] = src[q4];
      }
  }

  // ---- partials: acc rows 16 rt + 4g + r, dims DL n .. DL n + DL - 1 ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float l = lrun[rt], ps = psum[rt];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);     // row n
    if constexpr (I8) {
      ps += shfl_xor(ps, 16);
      ps += shfl_xor(ps, 32);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int src = 4 * g + r;  // the lane that holds row 4g + r's state
      const float lr = __shfl(l, src, WAVE);
      const float psr = I8 ? __shfl(ps, src, WAVE) : 0.f;
      const float Mr = __shfl(M[rt], src, WAVE);
      const int R = row0 + 16 * rt + 4 * g + r;
      if (R < nrows) {
        const int64_t orow = out_row(R);
        float o[DL];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[nt] = I8 ? fmaf(-kBias, psr, acc[rt][nt][r]) : acc[rt][nt][r];
        if (direct) {
          float L = lr;
          if (fold1) {
            //   out = (2^(Mr-M) o + 2^(M_0-M) acc_0) / (2^(Mr-M) lr + 2^(M_0-M) l_0)
            const float2 mk = pm1[rt][r];
            const float Mt = fmaxf(Mr, mk.x);
            const float es = (Mr == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(Mr - Mt);
            const float e = (mk.x == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(mk.x - Mt);
            L = fmaf(e, mk.y, lr * es);
#pragma unroll
            for (int q4 = 0; q4 < DL / 4; ++q4) {
              const float4 a4 = pa1[rt][r][q4];
              o[4 * q4] = fmaf(e, a4.x, o[4 * q4] * es); o[4 * q4 + 1] = fmaf(e, a4.y, o[4 * q4 + 1] * es);
              o[4 * q4 + 2] = fmaf(e, a4.z, o[4 * q4 + 2] * es); o[4 * q4 + 3] = fmaf(e, a4.w, o[4 * q4 + 3] * es);
            }
          } else if (npre > 0) {
            // fold in the shared-prefix partials of the row (slots 0..npre-1):
            //   out = (2^(Mr-M) o + sum_k 2^(M_k-M) acc_k) / (2^(Mr-M) lr + sum_k 2^(M_k-M) l_k)
            const float2* pm = reinterpret_cast<const float2*>(P.part_ml) + orow * P.max_parts;
            float Mt = Mr;
            for (int k = 0; k < npre; ++k) Mt = fmaxf(Mt, pm[k].x);
            const float es = (Mr == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(Mr - Mt);
            L = lr * es;
#pragma unroll
            for (int nt = 0; nt < DL; ++nt) o[nt] *= es;
            for (int k = 0; k < npre; ++k) {
              const float2 mk = pm[k];
              if (mk.x == kNegInf) continue;
              const float e = __builtin_amdgcn_exp2f(mk.x - Mt);
              L = fmaf(e, mk.y, L);
              const float4* src = reinterpret_cast<const float4*>(P.part_acc + (orow * P.max_parts + k) * HD + DL * n);
#pragma unroll
              for (int q4 = 0; q4 < DL / 4; ++q4) {
                const float4 a4 = src[q4];
                o[4 * q4] = fmaf(e, a4.x, o[4 * q4]); o[4 * q4 + 1] = fmaf(e, a4.y, o[4 * q4 + 1]);
                o[4 * q4 + 2] = fmaf(e, a4.z, o[4 * q4 + 2]); o[4 * q4 + 3] = fmaf(e, a4.w, o[4 * q4 + 3]);
              }
            }
          }
          const float inv = L > 0.f ? 1.f / L : 0.f;  // a tree row that sees no token attends to nothing
          if (DL * n < P.io_hd) {
            float4* dst = reinterpret_cast<float4*>(P.out + orow * P.io_hd + DL * n);
#pragma unroll
            for (int q4 = 0; q4 < DL / 4; ++q4)
              dst[q4] = make_float4(o[4 * q4] * inv, o[4 * q4 + 1] * inv, o[4 * q4 + 2] * inv, o[4 * q4 + 3] * inv);
          }
        } else {
          const int64_t pr = TREE ? orow * P.max_parts + pbase : pbase + (int64_t)R * pstride;
          float4* dst = reinterpret_cast<float4*>(pacc + pr * HD + DL * n);
#pragma unroll
          for (int q4 = 0; q4 < DL / 4; ++q4) dst[q4] = make_float4(o[4 * q4], o[4 * q4 + 1], o[4 * q4 + 2], o[4 * q4 + 3]);
          if (n == 0) reinterpret_cast<float2*>(pml)[pr] = make_float2(Mr, lr);
        }
      }
    }
  }
  if constexpr (FOLD) {
    if (fold) fold_claim_check(fin, P, s);
  }
}

// =============================================================================
// fp32 KV on the matrix cores (v_mfma_f32_16x16x4f32): the unit, partials and
// schedules of attn_piece, with q, K, p and V in fp32 end to end, as the
// reference computes over its default fp32 cache (kernels.metal:440-501,
// llama_cpu.rs:251-284). One block per pipeline stage (8 KB of K, 8 KB of V).
//   scores  S^T[t][r] in 32 instructions of 4 dims: lane (n, g) feeds K[token n]
//           and q[row n] at dims 16 j + 4 g + e (instruction 4 j + e), read as 8
//           16-byte pieces of the token row (the 4 lanes of a token cover 64
//           contiguous bytes per load), and gets S^T[tokens 4g..4g+3][row n]: the
//           layout of attn_piece, so the softmax is the same.
//   values  out[r][d] += sum_t p[r][t] V[t][d] in 4 instructions of 4 tokens per
//           16-dim tile: instruction i takes tokens 4 g + i, so A = the lane's own
//           p[row n][token 4 g + i]; B = V[token 4 g + i][dim 16 tile + n], from
//           the token pairs 2 g and 2 g + 1 (one 8-byte load each per tile, 128
//           contiguous bytes per 16 lanes); lane (n, g) accumulates rows 4g..4g+3,
//           dim 16 tile + n.
// =============================================================================
// DF: the tile width the piece is built for (128, or 64 for pools of 64-dim
// tiles: half the loads and products per block)
template <int DF = HD>
struct F32Stage {
  u32x4 k[DF / 16];      // token n, dims 16 j + 4 g .. + 3
  u32x2 v[DF / 16][2];   // tile t, token pair 2 g + r: dim 16 t + n of its two tokens
};

template <int DF = HD>
DEV void f32_stage_load(F32Stage<DF>& st, const DecodeParams& P, const BlockIds& bw, int i, int nblk, int kvh, int n,
                        int g) {
  const int blk = window_at(bw.b, min(i, nblk - 1));
  const uint64_t tix = (uint64_t)blk * P.n_kv_heads + kvh;
  const uint32_t tb = stage_bytes(i, nblk, P.tile_bytes);
  const rsrc_t kr = make_rsrc(P.kc + tix * P.tile_bytes, tb);
  const rsrc_t vr = make_rsrc(P.vc + tix * P.tile_bytes, tb);
  // K dims 16 j + 4 g .. + 3 of token n at 4 (n D + 16 j + 4 g); V dim 16 t + n of
  // token pair 2 g + r at 8 ((2 g + r) D + 16 t + n). A 64-dim tile: dims 64 and
  // up (j, t >= 4) read the bytes of the dims 64 below (they meet zero q dims and
  // their outputs are dropped). Two base offsets each, so that j and t stay
  // immediates; the pair r goes in the scalar offset.
  const int D = P.tile_hd;
  const int k0 = n * 4 * D + 16 * g, k1 = k0 - (D < HD ? 256 : 0);
  const int v0 = 16 * g * D + 8 * n, v1 = v0 - (D < HD ? 512 : 0);
#pragma unroll
  for (int j = 0; j < DF / 16; ++j) st.k[j] = __builtin_amdgcn_raw_buffer_load_b128(kr, (j < 4 ? k0 : k1) + 64 * j, 0, 0);
#pragma unroll
  for (int t = 0; t < DF / 16; ++t)
#pragma unroll
    for (int r = 0; r < 2; ++r)
      st.v[t][r] = __builtin_amdgcn_raw_buffer_load_b64(vr, (t < 4 ? v0 : v1) + 128 * t, r * 8 * D, kAuxNT);
}

template <int G, int RT, bool TREE, int QT, int DF = HD>
DEV void attn_piece_f32(const DecodeParams& P, int s, int kvh, int rg, int start, int end, int ctx_c, bool direct,
                        int64_t pbase, int pstride, float* pacc, float* pml) {
  constexpr int NJ = DF / 16;  // 16-dim groups: score chunks of 4 instructions, value tiles
  const int lane = lane_id();
  const int n = lane & 15, g = lane >> 4;
  const int N = TREE ? P.n_nodes : 1;
  int row = P.seq_rows ? P.seq_rows[s] : s;
  if (P.bt_rows > 0) row = min(max(row, 0), P.bt_rows - 1);
  const int32_t* bt = P.block_tables + (int64_t)row * P.bt_stride;
  const int H = P.n_heads;
  const int nblk = (end - start + BS - 1) / BS;
  const int blk0 = start / BS;
  const int Gn = group_size<G>(P);
  const int nrows = N * Gn;
  const int row0 = rg * 16 * RT;
  const int plain_end = min(end, ctx_c);
  auto out_row = [&](int R) -> int64_t { return ((int64_t)s * N + R / Gn) * H + (int64_t)kvh * Gn + R % Gn; };

  BlockIds bw;
  load_block_ids<false>(bw, P, bt, blk0, nblk, kvh);
  F32Stage<DF> sa, sb;
  f32_stage_load<DF>(sa, P, bw, 0, nblk, kvh, n, g);

  // q of row n of each tile at the lane's dims 16 j + 4 g + e (rows past the end are 0)
  float qf[RT][4 * NJ];
  uint32_t mrow[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int R = row0 + 16 * rt + n;
    const int64_t qoff = (R < nrows ? out_row(R) : 0) * P.io_hd + 4 * g;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (R < nrows && 16 * j + 4 * g < P.io_hd) {
        if constexpr (QT == DT_F32) {
          x = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(P.q) + qoff + 16 * j);
        } else {
          const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(P.q) + qoff + 16 * j);
          x = make_float4(half_lo(h.x), half_hi(h.x), half_lo(h.y), half_hi(h.y));
        }
      }
      qf[rt][4 * j] = x.x; qf[rt][4 * j + 1] = x.y; qf[rt][4 * j + 2] = x.z; qf[rt][4 * j + 3] = x.w;
    }
    mrow[rt] = 0u;
    if constexpr (TREE) {
      if (R < nrows) mrow[rt] = P.tree_mask[(int64_t)s * N + R / Gn];
    }
  }

  float M[RT], lrun[RT];
  float4v acc[RT][NJ];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    M[rt] = kNegInf; lrun[rt] = 0.f;
#pragma unroll
    for (int t = 0; t < NJ; ++t) acc[rt][t] = float4v{0.f, 0.f, 0.f, 0.f};
  }
  const int last_valid = (end - start) - (nblk - 1) * BS;

  auto compute = [&](const F32Stage<DF>& st, int i) {
    float4v sc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) sc[rt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          sc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(bitcast<float>(st.k[j][e]), qf[rt][4 * j + e], sc[rt], 0, 0, 0);
    const bool plain = (i < nblk) && (start + (i + 1) * BS <= plain_end);
    float sv[RT][4];
    bool need = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = sc[rt][r] * P.scale_log2;
        if (!plain) {
          const int tpos = start + i * BS + 4 * g + r;
          bool ok = (i < nblk) && tpos < end;
          if constexpr (TREE) {
            const int j = tpos - ctx_c;
            ok = ok && (j < 0 || ((mrow[rt] >> (j & 31)) & 1u));
          }
          x = ok ? x : kNegInf;
        }
        sv[rt][r] = x;
        need |= x > M[rt] + kRescaleThreshold;
      }
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float m = fmaxf(fmaxf(sv[rt][0], sv[rt][1]), fmaxf(sv[rt][2], sv[rt][3]));
        m = fmaxf(m, shfl_xor(m, 16));
        m = fmaxf(m, shfl_xor(m, 32));
        const float Mn = fmaxf(M[rt], m);
        const float alpha = (Mn == kNegInf) ? 1.f : __builtin_amdgcn_exp2f(M[rt] - Mn);
        M[rt] = Mn;
        lrun[rt] *= alpha;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * g + r, WAVE);
#pragma unroll
          for (int t = 0; t < NJ; ++t) acc[rt][t][r] *= ar;
        }
      }
    }
    float p[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float Ms = (M[rt] == kNegInf) ? 0.f : M[rt];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[rt][r] = __builtin_amdgcn_exp2f(sv[rt][r] - Ms);
        lrun[rt] += p[rt][r];
      }
    }
    if (i < nblk) {
      const bool partial = (i == nblk - 1) && (last_valid < BS);
#pragma unroll
      for (int t = 0; t < NJ; ++t) {
        float vv[4] = {bitcast<float>(st.v[t][0].x), bitcast<float>(st.v[t][0].y), bitcast<float>(st.v[t][1].x),
                       bitcast<float>(st.v[t][1].y)};
        if (partial) {  // bytes past the context may be anything, NaN included
#pragma unroll
          for (int r = 0; r < 4; ++r) vv[r] = (4 * g + r < last_valid) ? vv[r] : 0.f;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[rt][r], vv[r], acc[rt][t], 0, 0, 0);
      }
    }
  };

  for (int b = 0; b < nblk; b += 2) {
    f32_stage_load<DF>(sb, P, bw, b + 1, nblk, kvh, n, g);
    compute(sa, b);
    if (b + 1 >= nblk) break;
    f32_stage_load<DF>(sa, P, bw, b + 2, nblk, kvh, n, g);
    compute(sb, b + 1);
  }

  // ---- partials: acc rows 16 rt + 4g + r, dims 16 t + n ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float l = lrun[rt];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int src = 4 * g + r;
      const float lr = __shfl(l, src, WAVE);
      const float Mr = __shfl(M[rt], src, WAVE);
      const int R = row0 + 16 * rt + 4 * g + r;
      if (R < nrows) {
        const int64_t orow = out_row(R);
        if (direct) {
          const float inv = lr > 0.f ? 1.f / lr : 0.f;
#pragma unroll
          for (int t = 0; t < NJ; ++t)
            if (16 * t + n < P.io_hd) P.out[orow * P.io_hd + 16 * t + n] = acc[rt][t][r] * inv;
        } else {
          const int64_t pr = TREE ? orow * P.max_parts + pbase : pbase + (int64_t)R * pstride;
#pragma unroll
          for (int t = 0; t < NJ; ++t) pacc[pr * HD + 16 * t + n] = acc[rt][t][r];
          if (n == 0) reinterpret_cast<float2*>(pml)[pr] = make_float2(Mr, lr);
        }
      }
    }
  }
}

// attn_piece for every KV type: fp32 pools take the fp32 matrix-core piece.
template <int KV, int G, int RT, bool TREE, int QT, int D = HD, bool FOLD = false, bool ROPE = false>
DEV void attn_piece_kv(const DecodeParams& P, int s, int kvh, int rg, int start, int end, int ctx_c, bool direct,
                       int64_t pbase, int pstride, float* pacc, float* pml, int npre = 0) {
  if constexpr (KV == KV_F32) {
    attn_piece_f32<G, RT, TREE, QT, D>(P, s, kvh, rg, start, end, ctx_c, direct, pbase, pstride, pacc, pml);
  } else {
    attn_piece<KV, G, RT, TREE, QT, D, FOLD, ROPE>(P, s, kvh, rg, start, end, ctx_c, direct, pbase, pstride, pacc, pml, npre);
  }
}

// Split-K entry: unit = (row group, KV head, partition, sequence), kv head
// fastest. Partitions that start past the context exit; an empty decode context
// writes zero rows.
template <int KV, int G, int RT, bool TREE, int QT = DT_F16, int D = HD>
DEV void attn_unit_mfma(const DecodeParams& P) {
  int unit = blockIdx.x;
  int rg = 0;
  if constexpr (TREE) {
    rg = unit % P.n_rgroups;
    unit /= P.n_rgroups;
  }
  const int kvh = unit % P.n_kv_heads;
  const int rest = unit / P.n_kv_heads;
  const int gparts = P.max_parts - (TREE ? P.prefix_chunks : 0);  // partitions in the grid
  const int part = rest % gparts;
  const int s = rest / gparts;
  if (s >= P.n_seqs) return;
  const int N = TREE ? P.n_nodes : 1;
  const int ctx_c = max(0, min(P.context_lens[s], P.cap_tokens));  // committed tokens
  const int ctx = TREE ? min(ctx_c + N, P.cap_tokens) : ctx_c;      // committed + tree nodes
  // tree verify with a shared prefix: tokens below pre were covered by the
  // prefix pass (partial slots 0..C0-1); the partitions start at pre
  const int C0 = TREE ? P.prefix_chunks : 0;
  const int pre = C0 > 0 ? prefix_tokens_of(ctx_c, P.prefix_blocks) : 0;
  const int start = pre + part * P.part_tokens;
  if (start >= ctx) {
    if constexpr (!TREE) {
      if (part == 0) write_zero_rows_n(P, s, kvh, group_size<G>(P));
    }
    return;
  }
  const int end = min(start + P.part_tokens, ctx);
  const int nparts = C0 + (ctx - pre + P.part_tokens - 1) / P.part_tokens;
  const int64_t pbase =
      TREE ? C0 + part : ((int64_t)s * P.n_heads + (int64_t)kvh * group_size<G>(P)) * P.max_parts + part;
  // the rest of a context in one partition after a shared prefix writes the
  // output itself, folding in the prefix partials
  const bool fold = C0 > 0 && nparts == C0 + 1;
  attn_piece_kv<KV, G, RT, TREE, QT, D>(P, s, kvh, rg, start, end, ctx_c, nparts == 1 || fold, pbase, P.max_parts, P.part_acc,
                                  P.part_ml, fold ? C0 : 0);
}

// ---- stream-K decode -------------------------------------------------------
// The (sequence, KV head) segments in order form one range of cost units: a
// segment of nb > 0 blocks takes pen + nb units, pen units that stand for the
// cost of starting a piece and then one per block (sk_penalty; traces showed a
// worker whose range starts a second segment ending later by about that many
// blocks' time). Worker w (one wave) takes the w-th range of the stream-K split
// of all units (sk_split, velokv_params.h) and runs the blocks in it
// (sk_piece). A segment inside one worker's range is written directly; a
// split segment leaves one partial per worker: slot 1 for the worker where it
// starts, slot 0 for the workers that continue it. vk_decode_merge_sk combines
// them. Worker 0 also stores the per-sequence unit prefix and the total for
// the merge.
DEV int wave_sum_i(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, DPP_QUAD_XOR1, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_QUAD_XOR2, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_HALF_MIRROR, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_MIRROR, 0xF, 0xF, false);
  x += __shfl_xor(x, 16, WAVE);
  x += __shfl_xor(x, 32, WAVE);
  return x;
}
DEV int wave_incl_scan_i(int x) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < WAVE; d <<= 1) {
    const int y = __shfl_up(x, d, WAVE);
    if (lane >= d) x += y;
  }
  return x;
}
DEV int seq_blocks(const DecodeParams& P, int s) {
  return (max(0, min(P.context_lens[s], P.cap_tokens)) + BS - 1) / BS;
}

// Cost units of sequence s: Hkv segments of pen + nb units (none when empty).
DEV int seq_units(const DecodeParams& P, int s) {
  const int nb = seq_blocks(P, s);
  return nb > 0 ? P.n_kv_heads * (nb + P.sk_penalty) : 0;
}

template <int KV, int G, int QT = DT_F16, int D = HD, bool ROPE = false>
DEV void attn_streamk_mfma(const DecodeParams& P) {
  const int lane = lane_id();
  const int w = (int)blockIdx.x * ((int)blockDim.x / WAVE) + (int)threadIdx.x / WAVE;
  const int nw = P.n_workers;
  const int S = P.n_seqs, Hkv = P.n_kv_heads, pen = P.sk_penalty;
  int W = 0;
  for (int b = 0; b < S; b += WAVE) {
    const int s = b + lane;
    W += wave_sum_i(s < S ? seq_units(P, s) : 0);
  }
  if (w == 0) {  // unit prefix per sequence for the merge
    int off = 0;
    for (int b = 0; b < S; b += WAVE) {
      const int s = b + lane;
      const int nu = s < S ? seq_units(P, s) : 0;
      const int incl = wave_incl_scan_i(nu);
      if (s < S) P.sk_prefix[s] = off + incl - nu;
      off += readlane_i(incl, WAVE - 1);
    }
    if (lane == 0) P.sk_prefix[S] = W;
  }
  if (W == 0) return;
  const SkSplit sp = sk_split(W, nw);
  if (w >= sp.nw) return;  // workers past the split have no units
  const int64_t c0 = sk_begin(sp, w), c1 = sk_begin(sp, w + 1);
  // the sequence holding unit c0 and its first unit
  int s = -1, pre = 0;
  {
    int off = 0;
    for (int b = 0; b < S && s < 0; b += WAVE) {
      const int sl = b + lane;
      const int nu = sl < S ? seq_units(P, sl) : 0;
      const int incl = wave_incl_scan_i(nu);
      const uint64_t m = __builtin_amdgcn_ballot_w64(off + incl > c0);
      if (m != 0) {
        const int l = __builtin_ctzll(m);
        s = b + l;
        pre = off + readlane_i(incl - nu, l);
      }
      off += readlane_i(incl, WAVE - 1);
    }
  }
  int64_t x = c0;  // next unit to cover
  while (x < c1 && s < S) {
    const int ctx_s = max(0, min(P.context_lens[s], P.cap_tokens));
    const int nb = (ctx_s + BS - 1) / BS;
    if (nb == 0) { ++s; continue; }
    const int su = nb + pen;  // units per segment of this sequence
    const int kvh = (int)(x - pre) / su;
    const int64_t seg0 = pre + (int64_t)kvh * su;
    int o0, o1;
    sk_piece(seg0, nb, pen, x, c1, &o0, &o1);
    if (o0 < o1) {
      // under vk_append_decode (I8_BLK and fp16 pools) the piece that ends at the
      // context's last token appends the new token first (fold_issue,
      // fold_finish): no other piece of the launch reads that block
      const int slot = o0 > 0 ? 0 : 1;
      attn_piece_kv<KV, G, 1, false, QT, D, KV == KV_I8_BLK || KV == KV_F16, ROPE>(P, s, kvh, 0, o0 * BS, min(o1 * BS, ctx_s), ctx_s,
                                                            o0 == 0 && o1 == nb,
                                                            ((int64_t)w * 2 + slot) * group_size<G>(P), 1, P.part_acc,
                                                            P.part_ml);
    }
    x = seg0 + su;
    if (kvh == Hkv - 1) {
      pre += Hkv * su;
      ++s;
    }
  }
}

// ---- workgroup-split decode ------------------------------------------------
// One workgroup of NW = blockDim.x / 64 waves per (sequence, KV head), KV head
// fastest: wave w takes the w-th of NW equal block ranges of the context,
// leaves its unnormalised partial (acc, M, l) in LDS, and after one barrier the
// workgroup combines them into the output rows,
//   out = sum_w 2^(M_w - M) acc_w / sum_w 2^(M_w - M) l_w,  M = max_w M_w,
// so a uniform batch needs no partials in HBM and no merge launch.
constexpr int kWgMaxWaves = 8;
template <int KV, int G, int QT = DT_F16, int D = HD, bool ROPE = false>
DEV void attn_wg_mfma(const DecodeParams& P) {
  constexpr int GM = lds_rows<G>();
  __shared__ float wacc[kWgMaxWaves][GM][HD];
  __shared__ float wml[kWgMaxWaves][GM][2];
  const int Gn = group_size<G>(P);
  const int nw = (int)blockDim.x / WAVE;
  const int w = (int)threadIdx.x / WAVE;
  const int lane = lane_id();
  const int kvh = (int)blockIdx.x % P.n_kv_heads;
  const int s = (int)blockIdx.x / P.n_kv_heads;
  if (s >= P.n_seqs) return;  // the whole workgroup
  const int ctx = max(0, min(P.context_lens[s], P.cap_tokens));
  if (ctx == 0) {
    if (w == 0) write_zero_rows_n(P, s, kvh, Gn);
    return;
  }
  const int nb = (ctx + BS - 1) / BS;
  // under vk_append_decode (I8_BLK) the wave whose range ends at the context's
  // last token appends the new token first (fold_issue, fold_finish): the split
  // counts that append as fold_blocks more blocks of that wave's range
  const int fw = (KV == KV_I8_BLK && P.fold_k != nullptr) ? P.fold_blocks : 0;
  const int per = (nb + fw + nw - 1) / nw;
  const int b0 = min(nb, w * per), b1 = min(nb, b0 + per);
  if (b0 < b1) {
    attn_piece_kv<KV, G, 1, false, QT, D, KV == KV_I8_BLK, ROPE>(P, s, kvh, 0, b0 * BS, min(b1 * BS, ctx), ctx, false, 0, 1,
                                                           &wacc[w][0][0], &wml[w][0][0]);
  } else if (lane < Gn) {
    wml[w][lane][0] = kNegInf;
    wml[w][lane][1] = 0.f;
  }
  __syncthreads();
  const int64_t hrow0 = (int64_t)s * P.n_heads + (int64_t)kvh * Gn;
  const int IO = P.io_hd;  // output dims of a row; the partials are HD wide
  for (int i = (int)threadIdx.x; i < Gn * IO; i += (int)blockDim.x) {
    const int r = i / IO, d = i - r * IO;
    float M = kNegInf;
    for (int v = 0; v < nw; ++v) M = fmaxf(M, wml[v][r][0]);
    float L = 0.f, o = 0.f;
    for (int v = 0; v < nw; ++v) {
      const float mv = wml[v][r][0];
      if (mv == kNegInf) continue;  // a wave with no tokens (its acc row is not written)
      const float e = __builtin_amdgcn_exp2f(mv - M);
      L = fmaf(e, wml[v][r][1], L);
      o = fmaf(e, wacc[v][r][d], o);
    }
    P.out[(hrow0 + r) * IO + d] = L > 0.f ? o / L : 0.f;
  }
}

// ---- packed workgroup split (ragged batches) ---------------------------------
// The (sequence, KV head) items of the batch, longest first, are dealt to the B
// workgroups of the grid in snake order: item i goes to workgroup i mod B in even
// rounds r = i / B and to B - 1 - (i mod B) in odd ones, so a workgroup gets one
// of the longest items with one of the shortest, and so on, and the workgroups'
// sums of blocks come out nearly equal without a host round trip or an extra
// launch. Each workgroup ranks the sequences itself (rank of s = the sequences
// with more blocks, ties by index). Inside the workgroup the NW waves split the
// concatenated blocks of its items evenly, as stream-K does (sk_split over cost
// units: sk_penalty per item, then one per block). An item inside one wave's
// range is written directly; a split item leaves one partial per wave in LDS
// (slot 1 in the wave where it starts, slot 0 in the waves that continue it),
// combined into the output after one barrier. No partials in HBM, no merge
// launch. The host keeps every wave's range within 256 blocks.
constexpr int kPkMaxSeqs = 256;  // sequences a workgroup ranks (LDS)
constexpr int kPkMaxRounds = 16; // items per workgroup at most

template <int KV, int G, int QT = DT_F16>
DEV void attn_pk_mfma(const DecodeParams& P) {
  __shared__ int nb_l[kPkMaxSeqs];
  __shared__ int seq_at[kPkMaxSeqs];
  __shared__ float wacc[kWgMaxWaves][2][G][HD];
  __shared__ float wml[kWgMaxWaves][2][G][2];
  const int nw = (int)blockDim.x / WAVE;
  const int w = (int)threadIdx.x / WAVE;
  const int S = P.n_seqs, Hkv = P.n_kv_heads, pen = P.sk_penalty;
  const int B = (int)gridDim.x, bin = (int)blockIdx.x;
  const int NI = S * Hkv;
  for (int s = (int)threadIdx.x; s < S; s += (int)blockDim.x) nb_l[s] = seq_blocks(P, s);
  __syncthreads();
  for (int s = (int)threadIdx.x; s < S; s += (int)blockDim.x) {
    const int ns = nb_l[s];
    int r = 0;
    for (int t = 0; t < S; ++t) {
      const int nt = nb_l[t];
      r += (nt > ns) || (nt == ns && t < s);
    }
    seq_at[r] = s;
  }
  __syncthreads();
  // item of this workgroup in round r (or -1 past the last item)
  auto item = [&](int r) -> int {
    const int i = r * B + ((r & 1) ? B - 1 - bin : bin);
    return i < NI ? i : -1;
  };
  int T = 0;  // cost units of the workgroup's items
  for (int r = 0; r < kPkMaxRounds; ++r) {
    const int i = item(r);
    if (i < 0) break;
    const int nb = nb_l[seq_at[i / Hkv]];
    T += nb > 0 ? nb + pen : 0;
  }
  if (T > 0) {
    const SkSplit sp = sk_split(T, nw);
    if (w < sp.nw) {
      const int64_t c0 = sk_begin(sp, w), c1 = sk_begin(sp, w + 1);
      int64_t u = 0;  // first unit of the current item
      for (int r = 0; r < kPkMaxRounds && u < c1; ++r) {
        const int i = item(r);
        if (i < 0) break;
        const int s = seq_at[i / Hkv], kvh = i % Hkv;
        const int nb = nb_l[s];
        if (nb == 0) continue;
        int o0, o1;
        sk_piece(u, nb, pen, c0, c1, &o0, &o1);
        if (o0 < o1) {
          const int ctx_s = max(0, min(P.context_lens[s], P.cap_tokens));
          const int slot = o0 > 0 ? 0 : 1;
          attn_piece_kv<KV, G, 1, false, QT>(P, s, kvh, 0, o0 * BS, min(o1 * BS, ctx_s), ctx_s, o0 == 0 && o1 == nb,
                                             0, 1, &wacc[w][slot][0][0], &wml[w][slot][0][0]);
        }
        u += nb + pen;
      }
    }
  }
  __syncthreads();
  // split items: combine their pieces; empty items: zero rows
  int64_t u = 0;
  const SkSplit sp = sk_split(T > 0 ? T : 1, nw);
  for (int r = 0; r < kPkMaxRounds; ++r) {
    const int i = item(r);
    if (i < 0) break;
    const int s = seq_at[i / Hkv], kvh = i % Hkv;
    const int nb = nb_l[s];
    const int64_t hrow0 = (int64_t)s * P.n_heads + (int64_t)kvh * G;
    const int IO = P.io_hd;  // output dims of a row; the partials are HD wide
    if (nb == 0) {
      for (int e = (int)threadIdx.x; e < G * IO; e += (int)blockDim.x) P.out[hrow0 * IO + e] = 0.f;
      continue;
    }
    int w_lo, w_hi;
    sk_segment_workers(sp, u, nb, pen, &w_lo, &w_hi);
    u += nb + pen;
    if (w_lo == w_hi) continue;  // written by its wave
    for (int e = (int)threadIdx.x; e < G * IO; e += (int)blockDim.x) {
      const int g = e / IO, d = e - g * IO;
      float M = kNegInf;
      for (int v = w_lo; v <= w_hi; ++v) M = fmaxf(M, wml[v][v == w_lo ? 1 : 0][g][0]);
      float L = 0.f, o = 0.f;
      for (int v = w_lo; v <= w_hi; ++v) {
        const int sl = v == w_lo ? 1 : 0;
        const float mv = wml[v][sl][g][0];
        if (mv == kNegInf) continue;
        const float ev = __builtin_amdgcn_exp2f(mv - M);
        L = fmaf(ev, wml[v][sl][g][1], L);
        o = fmaf(ev, wacc[v][sl][g][d], o);
      }
      P.out[(hrow0 + g) * IO + d] = L > 0.f ? o / L : 0.f;
    }
  }
}

// ---- tree verify: shared-prefix pass ----------------------------------------
// When every sequence of a tree-verify call starts with the same pb pages (a
// prefix shared through the radix cache), attention over those pages is one
// dense product per KV head: all S * n_nodes * G query rows against the same
// keys. The prefix tiles are then read and converted once per workgroup of 256
// rows instead of once per (sequence, KV head). Workgroup (row tile, KV head,
// prefix chunk): 16 waves of one 16-row tile, four per SIMD (at 128 registers:
// with two waves per SIMD the chain scores -> softmax -> values of each wave
// left the matrix cores idle 70 % of the time). Each stage of 4 blocks is
// loaded by the first 8 waves, converted to fp16 (int8 codes become 1152 + c
// exactly, as in attn_piece) and written to LDS; every wave then runs its score
// and value products on the matrix cores against the staged tiles, two blocks
// at a time, with the lazy running max of attn_piece. int8 K is staged as the
// codes c themselves ((1152 + c) - 1152 in fp16, exact), so a score needs no
// bias term: with the biased codes of attn_piece the fp32 sums carry
// 1152 sum q, whose rounding grows with sum |q| (queries with outlier channels
// lost 0.1 and more of a score). Row r of sequence s sees
// prefix positions below prefix_tokens_of(ctx_s, pb). The chunk's unnormalised
// partial (acc, M, l) goes to partial slot `chunk` of the row; the tree kernel
// writes the rest of the context to the slots that follow and vk_decode_merge
// combines them.
//   scores  16x16x32: A = staged K (token n, dims 32kc + 8g .. +7), B = q^T (row
//           n, the same dims); lane (n, g) gets row n, tokens 4g..4g+3.
//   values  16x16x32 over a block pair (u0, u1): the 32 token slots of lane group
//           g are tokens 4g..4g+3 of u0 then of u1, in A = p (row n) and in
//           B = staged V (dim 16 nt + n); lane (n, g) accumulates rows 4g..4g+3,
//           dims 16 nt + n. int8 V is staged as fp16 c * v_scale (one rounding),
//           so the product needs no scale and no bias term.
//   softmax y = S a - M with a = scale_log2 * k_scale folded per block,
//           p = 2^y; l sums the fp16 p pairs with v_dot2.
// LDS: two stage buffers, one barrier per stage; a loader thread holds the
// next stage's raw bytes in registers while the current one is consumed. The
// chunk's page ids and block scales are staged in LDS once at the start, so the
// loaders take page ids from LDS: a global load of an id would wait for every
// tile load issued before it (vector loads return in order).
// gfx950 serves a 16-byte read for lanes {0-7, 16-23} (then
// {8-15, 24-31}, ...) in one pass over 64 four-byte banks: with lane (n, g)
// reading row n at word 4g, rows must start 8 (mod 16) words apart for the
// 16 lanes to cover the 64 banks once (measured: 72-word rows 0 conflict
// cycles, 68- or 20-word rows 4 per read).
//   K [tok][D + 16] fp16 (72-word rows at 128 dims, 40 at 64); the loader
//     writes 8 bytes per lane along a token row.
//   V per block pair [D][2 x 16 + 16] fp16 (24-word rows): a dim row holds, for
//     g = 0..3, tokens 4g..4g+3 of u0 then of u1, so that a lane's 8 token slots
//     are one 16-byte read. The loader writes 8 bytes (one dim, four tokens of
//     one block) per lane, gathered from two token-pair rows of the pool tile.
constexpr int kPfxLoadThreads = 512;      // the first 8 waves load the stages
constexpr int kPfxCH = 4;                 // blocks per stage (two pairs)
constexpr int kPfxVPitch = 2 * BS + 16;   // fp16 per staged V dim row of a block pair (24 words)

template <int KV, int QPT>
struct PfxRaw {  // this thread's share of one stage: QPT (block, quad) slots
  uint32_t k[QPT][Esz<KV>::v];  // 4 dims of one K token row (int8: 4 bytes, fp16: 8 bytes)
  uint32_t v[QPT][2];           // tokens 4t..4t+1 and 4t+2..4t+3 of one V dim (int8: 2 bytes each, fp16: 4)
};

// DP: the tile width the pass is built for, 128 or 64 dims (pools of 64-dim
// tiles: half the staged bytes, score products and value products per block).
template <int KV, int G, int QT, int DP = HD>
DEV void tree_prefix_mfma(const DecodeParams& P) {
  constexpr int RT = kPfxRT;
  constexpr bool I8 = (KV == KV_I8_BLK);
  constexpr int ESZ = Esz<KV>::v;
  constexpr int KC = DP / 32;    // 32-dim chunks of a score product
  constexpr int NT = DP / 16;    // 16-dim tiles of the value product
  constexpr int KP = DP + 16;    // fp16 per staged K row (8 mod 16 words: conflict-free reads)
  // (block, quad) slots per loader thread and stage: a block's K and V are 4 DP
  // quads each, spread over the kPfxLoadThreads loaders
  constexpr int QPT = kPfxCH * 4 * DP / kPfxLoadThreads;
  static_assert(QPT == kPfxCH || QPT * 2 == kPfxCH, "a loader thread takes every block or every other one");
  __shared__ __attribute__((aligned(16))) _Float16 kl[2][kPfxCH][BS * KP];
  __shared__ __attribute__((aligned(16))) _Float16 vl[2][kPfxCH / 2][DP * kPfxVPitch];
  // the chunk's tiles (page id * n_kv_heads + kvh) and (int8) block scales: K
  // scale times the softmax scale as fp32, V scale as fp16 bits
  __shared__ uint32_t pid[kPfxMaxChunkBlocks];
  __shared__ float pks[I8 ? kPfxMaxChunkBlocks : 1];
  __shared__ uint16_t pvs[I8 ? kPfxMaxChunkBlocks : 1];

  const int tid = (int)threadIdx.x;
  const int wave = tid / WAVE;
  const int lane = lane_id();
  const int n = lane & 15, g = lane >> 4;
  const int kvh = (int)blockIdx.y;
  const int chunk = (int)blockIdx.z, nchunks = (int)gridDim.z;
  const int N = P.n_nodes, H = P.n_heads;
  const int Gn = group_size<G>(P);
  const int RS = N * Gn;  // rows of one sequence for this KV head
  const int R = P.n_seqs * RS;
  const int wrow0 = (int)blockIdx.x * kPfxRows + wave * 16 * RT;
  const int PB = P.prefix_blocks;
  const int per = (PB + nchunks - 1) / nchunks;
  const int cb0 = min(PB, chunk * per), cb1 = min(PB, cb0 + per);
  const int nst = (cb1 - cb0 + kPfxCH - 1) / kPfxCH;
  int prow = P.seq_rows ? P.seq_rows[0] : 0;
  if (P.bt_rows > 0) prow = min(max(prow, 0), P.bt_rows - 1);
  const int32_t* bt = P.block_tables + (int64_t)prow * P.bt_stride;
  auto out_row = [&](int r) -> int64_t {
    const int s = r / RS, rem = r - s * RS;
    return ((int64_t)s * N + rem / Gn) * H + (int64_t)kvh * Gn + rem % Gn;
  };

  // ---- the chunk's page ids and scales into LDS, once: the stage loads then
  // take their page ids from LDS, so no global load of an id (which would wait
  // for every tile load issued before it) sits between the tile loads ----
  {
    bool bad = false;
    for (int i = tid; i < cb1 - cb0; i += (int)blockDim.x) {
      const int u = cb0 + i;
      const uint32_t pt = (uint32_t)P.page_tiles;
      const int raw = bt[(uint32_t)u / pt];
      bad |= raw < 0 || raw >= P.n_blocks;
      const int b = min(max(raw, 0), P.n_blocks - 1) * (int)pt + (int)((uint32_t)u % pt);
      const uint32_t tix = (uint32_t)b * (uint32_t)P.n_kv_heads + (uint32_t)kvh;
      pid[i] = tix;
      if constexpr (I8) {  // the (K, V) scale word of the (page, head)
        const uint32_t sw = *reinterpret_cast<const uint32_t*>(P.ks + (uint64_t)tix * kBlkScaleStep);
        pks[i] = P.scale_log2 * h2f((uint16_t)(sw & 0xFFFFu));
        pvs[i] = (uint16_t)(sw >> 16);
      }
    }
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) flag_misuse(P.err, MISUSE_PAGE_OUT_OF_POOL);
  }
  __syncthreads();

  // ---- q^T operands of rows wrow0 + 16 rt + n, and the prefix each row sees.
  // An fp32 q is split as q = hi + lo (fp16 each) and each score takes both
  // products, as in attn_piece ----
  constexpr bool QSPLIT = (QT == DT_F32);
  half8 qa[RT][KC];
  half8 qlo[RT][QSPLIT ? KC : 1];
  int lim[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = wrow0 + 16 * rt + n;
    const bool valid = r < R;
    const int64_t qoff = (valid ? out_row(r) : 0) * P.io_hd + 8 * g;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      uint4 v = make_uint4(0, 0, 0, 0), vlo = make_uint4(0, 0, 0, 0);
      if (valid && 32 * kc + 8 * g < P.io_hd) {
        if constexpr (QT == DT_F32) {
          const float4* q32 = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(P.q) + qoff + 32 * kc);
          const float4 x0 = q32[0], x1 = q32[1];
          v = make_uint4(pack_h2(x0.x, x0.y), pack_h2(x0.z, x0.w), pack_h2(x1.x, x1.y), pack_h2(x1.z, x1.w));
          const half8 h = bitcast<half8>(v);
          vlo = make_uint4(pack_h2(x0.x - (float)h[0], x0.y - (float)h[1]), pack_h2(x0.z - (float)h[2], x0.w - (float)h[3]),
                           pack_h2(x1.x - (float)h[4], x1.y - (float)h[5]), pack_h2(x1.z - (float)h[6], x1.w - (float)h[7]));
        } else {
          v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.q) + qoff + 32 * kc);
        }
      }
      qa[rt][kc] = bitcast<half8>(v);
      if constexpr (QSPLIT) qlo[rt][kc] = bitcast<half8>(vlo);
    }
    // rows past the end see the whole chunk (their results are dropped)
    lim[rt] = valid ? prefix_tokens_of(max(0, min(P.context_lens[r / RS], P.cap_tokens)), PB) : PB * BS;
  }
  // blocks below every row's limit need no mask (wave-uniform)
  int lmin = lim[0];
  for (int rt = 1; rt < RT; ++rt) lmin = min(lmin, lim[rt]);
  const int minlim = __builtin_amdgcn_readfirstlane((int)(-wave_max(-(float)lmin)));

  float M[RT], lrun[RT];
  float nMs[RT], thr[RT];  // -M (0 while M = -inf) and the rescale threshold (-inf while M = -inf)
  float4v acc[RT][NT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    M[rt] = kNegInf; lrun[rt] = 0.f;
    nMs[rt] = 0.f; thr[rt] = kNegInf;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = float4v{0.f, 0.f, 0.f, 0.f};
  }

  // ---- stage loader (threads 0..511): a thread reads 4 dims of K token kt and
  // 4 tokens of V dim vd (token group vq) of each block; int8 V is staged as
  // fp16 c * v_scale (the value product then needs no scale and no bias) ----
  // the thread's quad inside a block, and the blocks of its QPT slots
  const int qi = (QPT == kPfxCH) ? tid : (tid & (kPfxLoadThreads / 2 - 1));
  const int kt = qi / (DP / 4), kd = (qi % (DP / 4)) * 4;
  const int vd = qi % DP, vq = qi / DP;
  auto slot_block = [&](int i) { return (QPT == kPfxCH) ? i : 2 * i + (tid >> 8); };  // wave-uniform
  // A head_dim-64 tile is 64 dims wide: dims 64 and up are read from the dims 64
  // below (they meet zero q dims, and those output dims are dropped).
  const int D = P.tile_hd;
  const int kdt = kd & (D - 1), vdt = vd & (D - 1);
  // byte offset of K dims kd..kd+3 of token kt: int8 tiles hold dims 32c + 16h + j
  // of token t at byte 8 D h + (t D/32 + c) 16 + j
  const uint32_t koff = (ESZ == 1) ? (uint32_t)(((kdt >> 4) & 1) * 8 * D + (kt * (D >> 5) + (kdt >> 5)) * 16 + (kdt & 15))
                                   : (uint32_t)((kt * D + kdt) * 2);
  // V token pairs 2 vq and 2 vq + 1 of dim vd ([pair][D][2] tile)
  const uint32_t voff0 = (uint32_t)(((2 * vq) * D + vdt) * 2 * ESZ), voff1 = voff0 + D * 2 * ESZ;
  const uint32_t tile_b = (uint32_t)__builtin_amdgcn_readfirstlane((int)P.tile_bytes);  // uniform: SGPR descriptors
  // Loads are unconditional: a block past the chunk (or a stage past the last)
  // reads the chunk's first page, a written prefix page, whose tokens the
  // compute then skips or masks. (A zero fill on a branch let the compiler hoist
  // the first step of the int8 conversion right behind each load, which turned
  // the two-stage prefetch into waits.)
  auto gload = [&](PfxRaw<KV, QPT>& rw, int st) {
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int u = slot_block(i);
      const int b = cb0 + st * kPfxCH + u;
      const int bi = (st < nst && b < cb1) ? b - cb0 : 0;
      // wave-uniform tile address (SALU): tile index from LDS, tile bytes fixed;
      // buffer loads take the lane offsets as 32-bit VGPRs
      const uint32_t tix = (uint32_t)__builtin_amdgcn_readfirstlane((int)pid[bi]);
      // range: a 128-dim tile (a constant, so the descriptor stays in SGPRs); the
      // lane offsets stay inside the pool's own tile, 64 dims wide or 128
      constexpr uint32_t kTileMax = (uint32_t)BS * DP * ESZ;
      const rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(P.kc + (uint64_t)tix * tile_b), 0,
                                                          (int)kTileMax, 0x00020000);
      const rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(P.vc + (uint64_t)tix * tile_b), 0,
                                                          (int)kTileMax, 0x00020000);
      if constexpr (ESZ == 1) {
        rw.k[i][0] = __builtin_amdgcn_raw_buffer_load_b32(kr, (int)koff, 0, 0);
        rw.v[i][0] = __builtin_amdgcn_raw_buffer_load_b16(vr, (int)voff0, 0, 0);
        rw.v[i][1] = __builtin_amdgcn_raw_buffer_load_b16(vr, (int)voff1, 0, 0);
      } else {
        const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(kr, (int)koff, 0, 0);
        rw.k[i][0] = x.x; rw.k[i][1] = x.y;
        rw.v[i][0] = __builtin_amdgcn_raw_buffer_load_b32(vr, (int)voff0, 0, 0);
        rw.v[i][1] = __builtin_amdgcn_raw_buffer_load_b32(vr, (int)voff1, 0, 0);
      }
    }
  };
  auto lwrite = [&](int buf, int st, const PfxRaw<KV, QPT>& rw) {
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int u = slot_block(i);
      uint32_t kw0, kw1, vw0, vw1;
      if constexpr (ESZ == 1) {
        i8x4_to_h2x2_biased(rw.k[i][0], kw0, kw1);
        i8x4_to_h2x2_biased(rw.v[i][0] | (rw.v[i][1] << 16), vw0, vw1);
        // (1152 + c) - 1152 = c exactly (K), then one rounding of c * v_scale (V)
        const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
        kw0 = bitcast<uint32_t>(bitcast<half2v>(kw0) - bias);
        kw1 = bitcast<uint32_t>(bitcast<half2v>(kw1) - bias);
        const int b = cb0 + st * kPfxCH + u;
        const int bi = (st < nst && b < cb1) ? b - cb0 : 0;
        const _Float16 vsh = bitcast<_Float16>(pvs[bi]);
        const half2v vs2 = {vsh, vsh};
        vw0 = bitcast<uint32_t>((bitcast<half2v>(vw0) - bias) * vs2);
        vw1 = bitcast<uint32_t>((bitcast<half2v>(vw1) - bias) * vs2);
      } else {
        kw0 = rw.k[i][0]; kw1 = rw.k[i][1];
        vw0 = rw.v[i][0]; vw1 = rw.v[i][1];
      }
      *reinterpret_cast<u32x2*>(&kl[buf][u][kt * KP + kd]) = u32x2{kw0, kw1};
      *reinterpret_cast<u32x2*>(&vl[buf][u >> 1][vd * kPfxVPitch + 8 * vq + 4 * (u & 1)]) = u32x2{vw0, vw1};
    }
  };
  const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};
  // one block pair (u0 = up, u1 = up + 1) of stage buffer buf. Masks: row n sees
  // tokens 4g + r of block b0 + j for r < vis; a lane whose four tokens are all
  // hidden gets -inf in the score offset, and the per-token mask runs only when
  // some lane sees part of its four tokens (one block per row at most).
  auto pair_body = [&](int buf, int up, int b0, bool has1, bool plain) {
    float a[2];
    float4v scv[RT][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const _Float16* kb = &kl[buf][up + j][n * KP + 8 * g];
      half8 kop[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) kop[kc] = *reinterpret_cast<const half8*>(kb + 32 * kc);
      a[j] = I8 ? pks[min(b0 + j, cb1 - 1) - cb0] : P.scale_log2;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float4v sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kc], qa[rt][kc], sc, 0, 0, 0);
          if constexpr (QSPLIT) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kc], qlo[rt][kc], sc, 0, 0, 0);
        }
        scv[rt][j] = sc;
      }
    }
    // scores relative to the running max: y = S a - M (log2 units; nMs = -M,
    // 0 before the first score)
    float y[RT][2][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) y[rt][j][r] = fmaf(scv[rt][j][r], a[j], nMs[rt]);
    if (!plain) {  // tokens at or past a row's limit (or of a missing second block)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int vis = (j == 0 || has1) ? lim[rt] - (b0 + j) * BS - 4 * g : 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) y[rt][j][r] = (r < vis) ? y[rt][j][r] : kNegInf;
        }
    }
    bool need = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) need |= y[rt][j][r] > thr[rt];
    // lazy running max of row n (rare after the first blocks)
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float Ms = -nMs[rt];
        float m = y[rt][0][0];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) m = fmaxf(m, y[rt][j][r]);
        m = fmaxf(m, shfl_xor(m, 16));
        m = fmaxf(m, shfl_xor(m, 32));  // max over the pair's tokens of row n, relative to Ms
        const float Mn = fmaxf(M[rt], m + Ms);
        const float alpha = (Mn == kNegInf) ? 1.f : __builtin_amdgcn_exp2f(M[rt] - Mn);
        const float shift = (Mn == kNegInf) ? 0.f : Mn - Ms;
        M[rt] = Mn;
        nMs[rt] = (Mn == kNegInf) ? 0.f : -Mn;
        thr[rt] = (Mn == kNegInf) ? kNegInf : kRescaleThreshold;
        lrun[rt] *= alpha;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) y[rt][j][r] -= shift;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * g + r, WAVE);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[rt][nt][r] *= ar;
        }
      }
    }
    // p = 2^y in fp16 pairs (the A operand); l += sum p
    half8 pa[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      uint32_t pw[4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t lo = pack_h2(__builtin_amdgcn_exp2f(y[rt][j][0]), __builtin_amdgcn_exp2f(y[rt][j][1]));
        const uint32_t hi = pack_h2(__builtin_amdgcn_exp2f(y[rt][j][2]), __builtin_amdgcn_exp2f(y[rt][j][3]));
        lrun[rt] = dot2(hi, bitcast<uint32_t>(ones), dot2(lo, bitcast<uint32_t>(ones), lrun[rt]));
        pw[2 * j] = lo; pw[2 * j + 1] = hi;
      }
      pa[rt] = bitcast<half8>(u32x4{pw[0], pw[1], pw[2], pw[3]});
    }
    // values: B = V of dim 16 nt + n, tokens 4g..4g+3 of u0 then of u1
    const _Float16* vb = &vl[buf][up >> 1][n * kPfxVPitch + 8 * g];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const half8 vop = *reinterpret_cast<const half8*>(vb + 16 * nt * kPfxVPitch);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt], vop, acc[rt][nt], 0, 0, 0);
    }
  };
  auto compute = [&](int buf, int st) {
#pragma unroll
    for (int up = 0; up < kPfxCH; up += 2) {
      const int b0 = cb0 + st * kPfxCH + up;  // first block of the pair (wave-uniform)
      if (b0 < cb1) {
        const bool has1 = b0 + 1 < cb1;
        pair_body(buf, up, b0, has1, has1 && (b0 + 2) * BS <= minlim);
      }
    }
  };

  // ---- pipeline: LDS buffers alternate; ra holds the raw bytes of the stage
  // after the one being computed (an empty chunk, nst = 0 for the whole
  // workgroup, writes empty partials) ----
  if (nst > 0) {
    PfxRaw<KV, QPT> ra;
    const bool ld = tid < kPfxLoadThreads;
    if (ld) { gload(ra, 0); lwrite(0, 0, ra); gload(ra, 1); }
    __syncthreads();
    for (int st = 0; st < nst; st += 2) {
      compute(0, st);
      if (ld) { lwrite(1, st + 1, ra); gload(ra, st + 2); }
      __syncthreads();
      if (st + 1 >= nst) break;
      compute(1, st + 1);
      if (ld) { lwrite(0, st + 2, ra); gload(ra, st + 3); }
      __syncthreads();
    }
  }

  // ---- partials: rows 16 rt + 4g + r, dims 16 nt + n ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float l = lrun[rt];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int src = 4 * g + r;
      const float lr = __shfl(l, src, WAVE);
      const float Mr = __shfl(M[rt], src, WAVE);
      const int row = wrow0 + 16 * rt + 4 * g + r;
      if (row < R) {
        const int64_t pr = out_row(row) * P.max_parts + chunk;
        float* dst = P.part_acc + pr * HD + n;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) dst[16 * nt] = acc[rt][nt][r];
        if (n == 0) reinterpret_cast<float2*>(P.part_ml)[pr] = make_float2(Mr, lr);
      }
    }
  }
}

// Combine the partitions of one (sequence, head):
//   out = sum_p 2^(M_p - M) acc_p / sum_p 2^(M_p - M) l_p,  M = max_p M_p.
// One wave per (sequence, head); sequences with a single partition were
// finished by the decode kernel itself. Partial rows are loaded 8 at a time so
// the loads overlap.
// Combine np partials (index pr(k), k = 0..np-1) into one output row.
template <typename PR>
DEV void merge_row(const MergeParams& P, int64_t out_row, int np, PR pr) {
  const int lane = lane_id();
  const float2* ml = reinterpret_cast<const float2*>(P.part_ml);
  const float2* pa = reinterpret_cast<const float2*>(P.part_acc);
  float M = kNegInf;
  for (int p = lane; p < np; p += WAVE) M = fmaxf(M, ml[pr(p)].x);
  M = wave_max(M);
  float L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int p0 = 0; p0 < np; p0 += WAVE) {
    float w = 0.f;
    if (p0 + lane < np) {
      const float2 m = ml[pr(p0 + lane)];
      w = (m.x == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(m.x - M);
      L = fmaf(w, m.y, L);
    }
    const int cnt = min(WAVE, np - p0);
    for (int k0 = 0; k0 < cnt; k0 += 8) {
      float2 a[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        a[k] = (k0 + k < cnt) ? pa[pr(p0 + k0 + k) * (HD / 2) + lane] : make_float2(0.f, 0.f);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float wk = readlane_f(w, min(k0 + k, cnt - 1));
        if (k0 + k < cnt) {
          o0 = fmaf(wk, a[k].x, o0);
          o1 = fmaf(wk, a[k].y, o1);
        }
      }
    }
  }
  L = wave_sum(L);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (2 * lane < P.io_hd)
    reinterpret_cast<float2*>(P.out)[out_row * (P.io_hd / 2) + lane] = make_float2(o0 * inv, o1 * inv);
}

// Split-K merge: one wave per (sequence, row) with partials [row][max_parts]:
//   out = sum_p 2^(M_p - M) acc_p / sum_p 2^(M_p - M) l_p,  M = max_p M_p.
// Rows whose context fits one partition were finished by the attention kernel.
// With a shared prefix (tree verify), slots 0..prefix_chunks-1 hold the prefix
// pass and the partitions of the rest follow; a row whose rest fits one
// partition was finished by the tree kernel (it folds the prefix slots in).
__device__ void decode_merge(const MergeParams& P) {
  const int r = blockIdx.x * (blockDim.x / WAVE) + (threadIdx.x / WAVE);
  if (r >= P.n_rows) return;
  const int s = r / P.rows_per_seq;
  const int ctx_c = max(0, min(P.context_lens[s], P.cap_tokens));
  const int ctx = min(ctx_c + P.extra_tokens, P.cap_tokens);
  const int pre = P.prefix_chunks > 0 ? prefix_tokens_of(ctx_c, P.prefix_blocks) : 0;
  const int np = P.prefix_chunks + (ctx - pre + P.part_tokens - 1) / P.part_tokens;
  // one partition, or one after the prefix chunks: the attention kernel wrote the row
  if (np == P.prefix_chunks + 1) return;
  const int64_t base = (int64_t)r * P.max_parts;
  merge_row(P, r, np, [&](int k) -> int64_t { return base + k; });
}

// Stream-K merge: one wave per (sequence, head). The segment (s, kvh) starts at
// unit seg0 (its blocks after sk_penalty units); workers w_lo..w_hi hold its
// blocks: w_lo left slot 1, the others slot 0. Unsplit segments were written by
// their worker; empty contexts get zeros.
__device__ void decode_merge_sk(const MergeParams& P) {
  const int lane = lane_id();
  const int r = blockIdx.x * (blockDim.x / WAVE) + (threadIdx.x / WAVE);
  if (r >= P.n_rows) return;
  const int H = P.rows_per_seq;
  const int s = r / H, h = r - s * H;
  const int G = H / P.n_kv_heads;
  const int kvh = h / G, gi = h - kvh * G;
  const int nb = (max(0, min(P.context_lens[s], P.cap_tokens)) + BS - 1) / BS;
  if (nb == 0) {
    if (2 * lane < P.io_hd) reinterpret_cast<float2*>(P.out)[(int64_t)r * (P.io_hd / 2) + lane] = make_float2(0.f, 0.f);
    return;
  }
  const int64_t W = P.sk_prefix[P.n_seqs];
  const SkSplit sp = sk_split(W, P.n_workers);
  const int64_t seg0 = (int64_t)P.sk_prefix[s] + (int64_t)kvh * (nb + P.sk_penalty);
  int w_lo, w_hi;
  sk_segment_workers(sp, seg0, nb, P.sk_penalty, &w_lo, &w_hi);
  if (w_lo == w_hi) return;
  merge_row(P, r, w_hi - w_lo + 1, [&](int k) -> int64_t {
    return ((int64_t)(w_lo + k) * 2 + (k == 0 ? 1 : 0)) * G + gi;
  });
}

// =============================================================================
// KV append (kernels.metal:619-645 kv_update, 753-802 kv_update_int8).
// Workgroup (token n, KV head h) with two waves: wave 0 writes K, wave 1 writes V.
// Lane l owns dims 2l and 2l+1.
// =============================================================================
// RoPE position of token m: the caller's, or without a position array the new
// token's (context_len - 1, as its slot is derived).
DEV int rope_pos(const AppendParams& P, int m) {
  return P.positions ? P.positions[m] : min(P.context_lens[m], P.cap_tokens) - 1;
}

// Flat slot of token m, or -1 when it is padding (a negative slot, or one at or
// past the end of the pool) or, with RoPE, its position is outside the table.
DEV int64_t token_slot(const AppendParams& P, int m) {
  int64_t slot;
  if (P.slot_mapping) {
    slot = P.slot_mapping[m];
  } else {  // the new token of sequence m, at its last context position (kernels.metal:770-774)
    const int pos = min(P.context_lens[m], P.cap_tokens) - 1;
    const int ptok = BS * P.g.page_tiles;  // the page's tokens
    if (pos < 0 || pos / ptok >= P.bt_stride) return -1;
    int row = P.seq_rows ? P.seq_rows[m] : m;
    if (P.bt_rows > 0) row = min(max(row, 0), P.bt_rows - 1);
    slot = (int64_t)P.block_tables[(int64_t)row * P.bt_stride + pos / ptok] * ptok + pos % ptok;
  }
  if (slot < 0 || slot >= (int64_t)P.g.n_blocks * BS) return -1;
  if (P.rope != ROPE_NONE) {
    const int pos = rope_pos(P, m);
    if (pos < 0 || pos >= P.n_pos) return -1;
  }
  return slot;
}

// K/V row elements (dims 2l, 2l+1) of token m, head h, rotated for K when RoPE is on.
// Rows are io_hd long; lanes past it hold zeros (the tile's upper dims).
DEV void load_kv(const AppendParams& P, const void* src, bool is_v, int m, int h, float& x0, float& x1) {
  const int io = P.g.io_hd;
  x0 = x1 = 0.f;
  if (2 * lane_id() < io) load_x2(src, P.in_dtype, ((int64_t)m * P.g.n_kv_heads + h) * io + 2 * lane_id(), x0, x1);
  if (P.rope != ROPE_NONE && !is_v) rope_rotate(P.rope, P.cos_sin, rope_pos(P, m), io, x0, x1);
}

// VK_KV_I8_BLK: per-(block, head) fp16 scale, round-half-even codes clamped to +-127.
// A run = consecutive tokens of the call that fall in one block (padding slots
// in between skipped); the wave that holds the run's first token does the work
// for all of them, in order, keeping the block's codes in registers:
//   s_old = (offset == 0) ? 0 : stored scale
//   s_new = max(s_old, fp16(amax / 127))
//   if s_new > s_old: c' = clamp(rne((c * s_old) / s_new)) for tokens before offset
//   c = s_new > 0 ? clamp(rne(x / s_new)) : 0
// Slots are read 64 tokens at a time (lane j: token base + j) and runs are found
// with ballots; the K/V rows of up to 8 members are loaded together before the
// rule runs over them.

// Block of the nearest non-padding token before token n of the call, or -1.
DEV int prev_block(const AppendParams& P, int n) {
  const int lane = lane_id();
  for (int top = n - 1; top >= 0; top -= WAVE) {
    const int m = top - lane;
    const int64_t ps = m >= 0 ? token_slot(P, m) : -1;
    const uint64_t mask = __builtin_amdgcn_ballot_w64(ps >= 0);
    if (mask != 0) return readlane_i((int)(ps / BS), __builtin_ctzll(mask));
  }
  return -1;
}

// The run that starts at token w0 + j (slot `slot`), for KV head h; ms0 holds
// the slots of tokens w0 .. w0 + 63 (lane i: token w0 + i, -1 past the end), so
// the first step of the run's forward scan needs no load.
template <bool IS_V, int D>
DEV void append_blk_run(const AppendParams& P, const void* src, uint8_t* codes, uint16_t* scales, int w0, int j,
                        int64_t slot, int64_t ms0, int h) {
  const int lane = lane_id();
  const int64_t b = slot / BS;
  if (b >= P.g.n_blocks) return;
  const int Hkv = P.g.n_kv_heads;
  uint8_t* tile = codes + ((uint64_t)b * Hkv + h) * P.g.tile_bytes;
  uint16_t* sp = scales + ((uint64_t)b * Hkv + h) * (kBlkScaleStep / 2);
  const int d0 = 2 * lane;
  // lanes past the row (2 lane >= D) read the codes of the dims D below and never
  // write them back; their new-token values are zero, so the absmax is the row's
  const bool din = d0 < D;
  const int da = d0 & (D - 1);
  // element (u, d) sits at tile_elem(u, 0) + tile_elem(0, d) in both layouts:
  // one lane pointer and constant offsets per token
  uint8_t* const lp0 = tile + tile_elem<IS_V>(0, da, 1, D);

  // the lane's codes as whole words: K dims da, da + 1 of a token are adjacent
  // bytes (one 16-bit word per token); V dims da, da + 1 of a token pair are 4
  // adjacent bytes (tokens 2p, 2p + 1 of dim da, then of dim da + 1)
  int cd[BS][2];
  if constexpr (IS_V) {
#pragma unroll
    for (int p = 0; p < BS / 2; ++p) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(lp0 + tile_elem<true>(2 * p, 0, 1, D));
      cd[2 * p][0] = (int8_t)(uint8_t)w;
      cd[2 * p + 1][0] = (int8_t)(uint8_t)(w >> 8);
      cd[2 * p][1] = (int8_t)(uint8_t)(w >> 16);
      cd[2 * p + 1][1] = (int8_t)(uint8_t)(w >> 24);
    }
  } else {
#pragma unroll
    for (int u = 0; u < BS; ++u) {
      const uint32_t w = *reinterpret_cast<const uint16_t*>(lp0 + tile_elem<false>(u, 0, 1, D));
      cd[u][0] = (int8_t)(uint8_t)w;
      cd[u][1] = (int8_t)(uint8_t)(w >> 8);
    }
  }
  const uint16_t stored = *sp;
  float s_old = 0.f;
  uint16_t s_bits = 0;
  int hi_written = -1;
  bool first = true;
  for (int base = w0; base < P.n_tok; base += WAVE) {
    const int m = base + lane;
    // tokens before the run's first (lanes below j of the first window) are not part of it
    const int64_t ms = base == w0 ? (lane >= j ? ms0 : -1) : (m < P.n_tok ? token_slot(P, m) : -1);
    // the run ends at the first non-padding token of another block
    const uint64_t other = __builtin_amdgcn_ballot_w64(ms >= 0 && ms / BS != b);
    const int stop = other ? __builtin_ctzll(other) : WAVE;
    uint64_t mem = __builtin_amdgcn_ballot_w64(ms >= 0 && lane < stop);
    const int moff = (int)(ms >= 0 ? ms % BS : 0);
    while (mem != 0) {
      // up to 8 members: their rows loaded together, then the rule. What does
      // not depend on the member before (the absmax and candidate scale, and
      // once the running scales are known the new codes) is computed for all
      // members at once; only the running scale and the placement, with its
      // requantization when the scale grew, follow the members' order.
      constexpr int kBatch = 8;
      float xs[kBatch][2];
      int ok[kBatch];  // member offsets in the block (wave-uniform)
      int nb = 0;
      {
        uint64_t rest = mem;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          ok[k] = 0;
          if (rest != 0) {
            const int j = __builtin_ctzll(rest);
            rest &= rest - 1;
            ok[k] = readlane_i(moff, j);
            nb = k + 1;
            load_kv(P, src, IS_V, base + j, h, xs[k][0], xs[k][1]);
          }
        }
        mem = rest;
      }
      uint16_t cand[kBatch];  // fp16(amax / 127) of each member (wave-uniform)
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        cand[k] = 0;
        if (k < nb) {
          const float amax = wave_max(fmaxf(fabsf(xs[k][0]), fabsf(xs[k][1])));
          cand[k] = (uint16_t)__builtin_amdgcn_readfirstlane((int)f2h(amax / 127.0f));
        }
      }
      // the scale before (so) and after (sn) each member
      float so[kBatch], sn[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        so[k] = sn[k] = 0.f;
        if (k < nb) {
          const int o = ok[k];
          if (first) {
            s_old = (o == 0) ? 0.f : h2f(stored);
            s_bits = (o == 0) ? (uint16_t)0 : stored;
            first = false;
          } else if (o == 0) {
            s_old = 0.f;
            s_bits = 0;
          }
          so[k] = s_old;
          if (h2f(cand[k]) > s_old) {
            s_bits = cand[k];
            s_old = h2f(cand[k]);
          }
          sn[k] = s_old;
        }
      }
      int cc[kBatch][2];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        cc[k][0] = k < nb ? blk_code(xs[k][0], sn[k]) : 0;
        cc[k][1] = k < nb ? blk_code(xs[k][1], sn[k]) : 0;
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (k < nb) {
          const int o = ok[k];
          if (sn[k] > so[k] && o > 0) {
#pragma unroll
            for (int u = 0; u < BS; ++u) {
              if (u < o) {
                cd[u][0] = blk_requant(cd[u][0], so[k], sn[k]);
                cd[u][1] = blk_requant(cd[u][1], so[k], sn[k]);
              }
            }
          }
#pragma unroll
          for (int u = 0; u < BS; ++u)
            if (u == o) { cd[u][0] = cc[k][0]; cd[u][1] = cc[k][1]; }
          hi_written = max(hi_written, o);
        }
      }
    }
    if (other != 0) break;
  }
  // the same words back for the tokens up to the last one written (a V pair whose
  // second token is past it stores that token's codes as they were loaded)
  auto b8 = [](int c) { return (uint32_t)(uint8_t)(int8_t)c; };
  if constexpr (IS_V) {
#pragma unroll
    for (int p = 0; p < BS / 2; ++p)
      if (din && 2 * p <= hi_written)
        *reinterpret_cast<uint32_t*>(lp0 + tile_elem<true>(2 * p, 0, 1, D)) =
            b8(cd[2 * p][0]) | (b8(cd[2 * p + 1][0]) << 8) | (b8(cd[2 * p][1]) << 16) | (b8(cd[2 * p + 1][1]) << 24);
  } else {
#pragma unroll
    for (int u = 0; u < BS; ++u)
      if (din && u <= hi_written)
        *reinterpret_cast<uint16_t*>(lp0 + tile_elem<false>(u, 0, 1, D)) = (uint16_t)(b8(cd[u][0]) | (b8(cd[u][1]) << 8));
  }
  if (lane == 0) *sp = s_bits;
}

// The runs that start inside tokens [w0, w0 + T) of the call, in order. A token
// starts a run when it is not padding and the nearest non-padding token before
// it is in another block (or there is none).
template <bool IS_V, int D>
DEV void append_blk(const AppendParams& P, const void* src, uint8_t* codes, uint16_t* scales, int w0, int T) {
  const int lane = lane_id();
  const int h = blockIdx.y;
  const int m = w0 + lane;
  // slots of 64 tokens from w0: the window's T and what follows (reused by the runs' forward scans)
  const int64_t ms64 = m < P.n_tok ? token_slot(P, m) : -1;
  const int64_t ms = lane < T ? ms64 : -1;
  const int before = prev_block(P, w0);  // loads issued beside the window's
  const int mb = ms >= 0 ? (int)(ms / BS) : -1;
  const uint64_t valid = __builtin_amdgcn_ballot_w64(ms >= 0);
  if (valid == 0) return;
  const uint64_t low = valid & ((1ull << lane) - 1ull);
  const int pl = low ? 63 - __builtin_clzll(low) : 0;
  const int pb = __shfl(mb, pl, WAVE);
  const int prevb = low ? pb : before;
  uint64_t starts = __builtin_amdgcn_ballot_w64(ms >= 0 && prevb != mb);
  while (starts != 0) {
    const int j = __builtin_ctzll(starts);
    starts &= starts - 1;
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)ms, j);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)ms >> 32), j);
    const int64_t slot = (int64_t)(((uint64_t)hi << 32) | lo);
    // one run per block and call: a second run of this call on the same block
    // (its tokens not adjacent in the call) would requantize it concurrently.
    // The claim's old value is checked after the run, so that the exchange's
    // round trip overlaps the run's loads instead of preceding them.
    const bool claim = !IS_V && h == 0 && lane == 0 && P.claim;
    const unsigned long long me = ((unsigned long long)P.epoch << 32) | (uint32_t)(w0 + j);
    unsigned long long old = 0;
    if (claim) old = __hip_atomic_exchange(&P.claim[slot / BS], me, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    append_blk_run<IS_V, D>(P, src, codes, scales, w0, j, slot, ms64, h);
    if (claim && (uint32_t)(old >> 32) == P.epoch && old != me) flag_misuse(P.err, MISUSE_BLK_SPLIT_RUN);
  }
}

// VK_KV_I8_REF: per-(token, head) fp32 scale = amax/127, codes = trunc(x * (127/amax)).
template <bool IS_V>
DEV void append_ref(const AppendParams& P, const void* src, uint8_t* codes, float* scales, int n, int64_t slot) {
  const int lane = lane_id();
  const int h = blockIdx.y;
  if (slot < 0) return;
  const int64_t b = slot / BS;
  const int o = (int)(slot % BS);
  if (b >= P.g.n_blocks) return;
  const int Hkv = P.g.n_kv_heads;
  const int d0 = 2 * lane;
  float x0, x1;
  load_kv(P, src, IS_V, n, h, x0, x1);
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const float scale = amax / 127.0f;
  const float inv = amax > 0.f ? 127.0f / amax : 0.f;
  uint8_t* tile = codes + ((uint64_t)b * Hkv + h) * P.g.tile_bytes;
  const int D = P.g.head_dim;
  if (d0 < D) {
    tile[tile_elem<IS_V>(o, d0, 1, D)] = (uint8_t)(int8_t)(int)(x0 * inv);
    tile[tile_elem<IS_V>(o, d0 + 1, 1, D)] = (uint8_t)(int8_t)(int)(x1 * inv);
  }
  if (lane == 0) scales[((uint64_t)b * Hkv + h) * BS + o] = scale;
}

// VK_KV_F16 / VK_KV_F32: plain copy (with RNE conversion to fp16 when needed).
template <bool IS_V, int ESZ>
DEV void append_plain(const AppendParams& P, const void* src, uint8_t* codes, int n, int64_t slot) {
  const int lane = lane_id();
  const int h = blockIdx.y;
  if (slot < 0) return;
  const int64_t b = slot / BS;
  const int o = (int)(slot % BS);
  if (b >= P.g.n_blocks) return;
  const int Hkv = P.g.n_kv_heads;
  const int d0 = 2 * lane;
  uint8_t* tile = codes + ((uint64_t)b * Hkv + h) * P.g.tile_bytes;
  const int D = P.g.head_dim;
  if (ESZ == 2 && P.in_dtype == DT_F16 && (IS_V || P.rope == ROPE_NONE) && D == HD && P.g.io_hd == HD) {
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src) + ((int64_t)n * Hkv + h) * HD + d0;
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0, 2, HD)) = s16[0];
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0 + 1, 2, HD)) = s16[1];
    return;
  }
  float x0, x1;
  load_kv(P, src, IS_V, n, h, x0, x1);
  if (d0 >= D) return;
  if constexpr (ESZ == 2) {
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0, 2, D)) = f2h(x0);
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0 + 1, 2, D)) = f2h(x1);
  } else {
    *reinterpret_cast<float*>(tile + tile_elem<IS_V>(o, d0, 4, D)) = x0;
    *reinterpret_cast<float*>(tile + tile_elem<IS_V>(o, d0 + 1, 4, D)) = x1;
  }
}

// D: head_dim of the pool for the I8_BLK rule (a compile-time constant, so that
// the 16 tokens' tile offsets fold into the instructions; vk_append_kv3 / _d64).
template <int KV, int D = HD>
DEV void append_kernel(const AppendParams& P) {
  const int T = P.tok_per_wg;
  const int w0 = (int)blockIdx.x * T;
  const int w1 = min(w0 + T, P.n_tok);
  if ((int)blockIdx.y >= P.g.n_kv_heads) {  // RoPE of two query heads of the window's tokens
    const int head = 2 * ((int)blockIdx.y - P.g.n_kv_heads) + (int)(threadIdx.x / WAVE);
    if (head >= P.n_heads) return;
    void* qd = P.q_out ? P.q_out : P.q;
    for (int n = w0; n < w1; ++n) {
      const int pos = rope_pos(P, n);
      const int64_t off = ((int64_t)n * P.n_heads + head) * P.g.io_hd + 2 * lane_id();
      float x0 = 0.f, x1 = 0.f;
      const bool in = 2 * lane_id() < P.g.io_hd;
      if (in) load_x2(P.q, P.q_dtype, off, x0, x1);
      const bool rot = pos >= 0 && pos < P.n_pos;  // (wave-uniform)
      if (rot) rope_rotate(P.rope, P.cos_sin, pos, P.g.io_hd, x0, x1);
      if (!in || (!rot && !P.q_out)) continue;  // unrotated rows stay as they are (copied when q_out is given)
      if (P.q_dtype == DT_F16) {
        reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(qd) + off)[0] =
            (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
      } else {
        reinterpret_cast<float2*>(reinterpret_cast<float*>(qd) + off)[0] = make_float2(x0, x1);
      }
    }
    return;
  }
  const bool is_v = (threadIdx.x >= WAVE);
  uint8_t* L = P.base + (uint64_t)P.layer * P.g.layer_stride;
  const void* src = is_v ? P.v : P.k;
  uint8_t* codes = L + (is_v ? P.g.v_off : P.g.k_off);
  if constexpr (KV == KV_I8_BLK) {
    uint16_t* sc = reinterpret_cast<uint16_t*>(L + (is_v ? P.g.vs_off : P.g.ks_off));
    if (is_v) append_blk<true, D>(P, src, codes, sc, w0, T); else append_blk<false, D>(P, src, codes, sc, w0, T);
    return;
  }
  // one token at a time; the window's slots are read at once (lane j: token w0 + j)
  const int64_t ms = w0 + lane_id() < w1 ? token_slot(P, w0 + lane_id()) : -1;
  for (int n = w0; n < w1; ++n) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)ms, n - w0);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)ms >> 32), n - w0);
    const int64_t slot = (int64_t)(((uint64_t)hi << 32) | lo);
    if constexpr (KV == KV_I8_REF) {
      float* sc = reinterpret_cast<float*>(L + (is_v ? P.g.vs_off : P.g.ks_off));
      if (is_v) append_ref<true>(P, src, codes, sc, n, slot); else append_ref<false>(P, src, codes, sc, n, slot);
    } else if constexpr (KV == KV_F16) {
      if (is_v) append_plain<true, 2>(P, src, codes, n, slot); else append_plain<false, 2>(P, src, codes, n, slot);
    } else {
      if (is_v) append_plain<true, 4>(P, src, codes, n, slot); else append_plain<false, 4>(P, src, codes, n, slot);
    }
  }
}

// =============================================================================
// Small kernels: slot mapping, copy-on-write block copy, synthetic fill.
// =============================================================================
__device__ void slot_mapping_kernel(const SlotMapParams& P) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.n_tok) return;
  const int row = P.seq_rows ? P.seq_rows[i] : i;
  const int pos = P.positions[i];
  if (pos < 0 || pos / P.block_size >= P.bt_stride) { P.out[i] = -1; return; }
  const int blk = P.block_tables[(int64_t)row * P.bt_stride + pos / P.block_size];
  P.out[i] = (blk < 0 || blk >= P.n_blocks) ? -1 : (int64_t)blk * P.block_size + pos % P.block_size;
}

// grid = (n_pairs, n_layer, 2): z = 0 copies K codes + K scales, z = 1 V.
__device__ void copy_blocks_kernel(const CopyParams& P) {
  const int pi = blockIdx.x, layer = blockIdx.y;
  const bool is_v = blockIdx.z != 0;
  const int src = P.pairs[2 * pi], dst = P.pairs[2 * pi + 1];
  uint8_t* L = P.base + (uint64_t)layer * P.g.layer_stride;
  const uint64_t cb = (uint64_t)P.g.n_kv_heads * P.g.tile_bytes;   // codes per block
  const uint64_t sb = (uint64_t)P.g.n_kv_heads * P.g.stile_bytes;  // scale bytes per block, K or V
  const uint8_t* cs = L + (is_v ? P.g.v_off : P.g.k_off) + (uint64_t)src * cb;
  uint8_t* cdst = L + (is_v ? P.g.v_off : P.g.k_off) + (uint64_t)dst * cb;
  for (uint64_t i = threadIdx.x; i < cb / 16; i += blockDim.x)
    reinterpret_cast<uint4*>(cdst)[i] = reinterpret_cast<const uint4*>(cs)[i];
  if (sb) {  // the block's sb / 2 16-bit scale units of this kind, s_step bytes apart
    const uint64_t ne = sb / 2, st = P.g.s_step;
    const uint8_t* ss = L + (is_v ? P.g.vs_off : P.g.ks_off) + (uint64_t)src * ne * st;
    uint8_t* sd = L + (is_v ? P.g.vs_off : P.g.ks_off) + (uint64_t)dst * ne * st;
    for (uint64_t i = threadIdx.x; i < ne; i += blockDim.x)
      *reinterpret_cast<uint16_t*>(sd + i * st) = *reinterpret_cast<const uint16_t*>(ss + i * st);
  }
}

// ---- NIXL wire records (nixl.rs:24-61) ------------------------------------
// Status codes of include/velokv.h.
constexpr int kNixlOk = 0, kNixlShortHeader = 1, kNixlTruncated = 2, kNixlHandleMismatch = 3,
              kNixlLengthMismatch = 4, kNixlBadPage = 5;

// grid = records of the launch, 256 threads. Decides each record's status
// before any payload moves: unpack checks the header as deserialize_block does
// (nixl.rs:50-58: header present, payload within the buffer) and then that it
// names this item and this pool's payload size; both directions check that
// every page id is inside the pool. Pack writes the header of a good record.
__device__ void nixl_check_kernel(const NixlParams& P) {
  __shared__ int bad_page;
  const int it = blockIdx.x;
  const NixlItemArg& I = P.items[it];
  if (threadIdx.x == 0) bad_page = 0;
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < I.n_pages; i += blockDim.x) {
    const int32_t pg = P.pages[I.first_page + (int64_t)i];
    if (pg < 0 || pg >= P.g.n_blocks) bad_page = 1;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  int st = kNixlOk;
  if (P.unpack) {
    if (I.wire_offset > P.wire_bytes || P.wire_bytes - I.wire_offset < 16) {
      st = kNixlShortHeader;
    } else {
      const uint4 h = *reinterpret_cast<const uint4*>(P.wire + I.wire_offset);
      const uint64_t block_id = (uint64_t)h.x | ((uint64_t)h.y << 32);
      const uint32_t token_len = h.z, byte_len = h.w;
      if ((uint64_t)byte_len > P.wire_bytes - I.wire_offset - 16) st = kNixlTruncated;
      else if (block_id != I.block_id || token_len != I.token_len) st = kNixlHandleMismatch;
      else if (byte_len != I.byte_len) st = kNixlLengthMismatch;
    }
  }
  if (st == kNixlOk && bad_page) st = kNixlBadPage;
  P.status[it] = st;
  if (!P.unpack && st == kNixlOk) {
    // little-endian header: block_id, token_len, byte_len
    *reinterpret_cast<uint4*>(P.wire + I.wire_offset) =
        make_uint4((uint32_t)I.block_id, (uint32_t)(I.block_id >> 32), I.token_len, I.byte_len);
  }
}

// grid = work units of the launch x slices, 256 threads: unit = (record, page i,
// layer l), whose K and V codes of every KV head (two contiguous runs in the
// pool, one run in the record) are cut into 4 KB slices, one per workgroup and
// one 16-byte load per lane (many small workgroups copy fastest on MI355X);
// slice 0 also moves the unit's scales.
__device__ void nixl_copy_kernel(const NixlParams& P) {
  const uint32_t gid = blockIdx.x;
  int lo = 0, hi = P.n_items - 1;  // last record whose slices start at or before gid
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (P.items[mid].unit_begin <= gid) lo = mid; else hi = mid - 1;
  }
  const NixlItemArg& I = P.items[lo];
  if (P.status[lo] != kNixlOk) return;
  const uint32_t rs = gid - I.unit_begin;
  const uint32_t r = rs / (uint32_t)P.n_slices;          // i * n_layers + l
  const uint32_t slice = rs - r * (uint32_t)P.n_slices;
  const uint32_t i = r / (uint32_t)P.n_layers, l = r - i * (uint32_t)P.n_layers;
  const int64_t page = P.pages[I.first_page + (int64_t)i];
  uint8_t* L = P.base + (uint64_t)(P.layer0 + (int)l) * P.g.layer_stride;
  const uint64_t cb = (uint64_t)P.g.n_kv_heads * P.g.tile_bytes;   // codes of one page, K or V
  const uint64_t sb = (uint64_t)P.g.n_kv_heads * P.g.stile_bytes;  // scales of one page, K or V
  uint8_t* payload = P.wire + I.wire_offset + 16;
  const uint32_t nv = (uint32_t)(cb / 16);  // 16-byte vectors per K (or V) run
  const uint32_t j = slice * kNixlSliceVecs + threadIdx.x;
  if (j < 2 * nv) {
    uint8_t* wt = payload + (uint64_t)r * 2 * cb + (uint64_t)j * 16;
    uint8_t* pt = L + (j < nv ? P.g.k_off + (uint64_t)page * cb + (uint64_t)j * 16
                              : P.g.v_off + (uint64_t)page * cb + (uint64_t)(j - nv) * 16);
    const u32x4* src = reinterpret_cast<const u32x4*>(P.unpack ? wt : pt);
    u32x4* dst = reinterpret_cast<u32x4*>(P.unpack ? pt : wt);
    __builtin_nontemporal_store(__builtin_nontemporal_load(src), dst);
  }
  if (sb && slice == 0) {  // the record holds K's units, then V's, each kind contiguous
    uint16_t* ws = reinterpret_cast<uint16_t*>(payload + (uint64_t)I.n_pages * P.n_layers * 2 * cb + (uint64_t)r * 2 * sb);
    const uint32_t ne = (uint32_t)(sb / 2), st = P.g.s_step;  // units of one kind, bytes between them
    uint8_t* sk = L + P.g.ks_off + (uint64_t)page * ne * st;
    uint8_t* sv = L + P.g.vs_off + (uint64_t)page * ne * st;
    for (uint32_t e = threadIdx.x; e < 2 * ne; e += blockDim.x) {
      uint16_t* pe = reinterpret_cast<uint16_t*>(e < ne ? sk + (uint64_t)e * st : sv + (uint64_t)(e - ne) * st);
      if (P.unpack) *pe = ws[e]; else ws[e] = *pe;
    }
  }
}

// ---- accepted-path commit of a draft tree -----------------------------------
// grid (sequence, KV head, group of kCommitLayers layers), wave 0 = K, wave 1 =
// V, lane = two dims (2l, 2l+1, or for int8 K the pair stored at byte 2l of the
// token's two 64-byte runs). The row is validated once; then per layer every moved
// token is read (raw element bytes and its scale, 8 tokens' loads in flight at a
// time) into LDS before any write, so a write never changes a source still to
// be read; then the tokens are written in order: rows and per-token scales as
// they were, or for I8_BLK dequantized (code x block scale, exact in fp32) and
// put through the append rule (blk_put), one destination block at a time.
constexpr int kMaxCommit = 32;
constexpr int kCommitLayers = 8;

// One wave's share of a commit (K when IS_V is false, V when true): layers
// [l0, l1) of KV head h of sequence s, accepted tokens a (lane i: node of the
// i-th accepted token), d0 the first moved one, blocks blk_l (lane i: the i-th
// destination block from b_first).
template <int KV, bool IS_V, int D>
DEV void commit_wave(const CommitParams& P, uint8_t (&raw)[kMaxCommit][2 * WAVE * Esz<KV>::v], float (&xsc)[kMaxCommit],
                     int h, int l0, int l1, int ctx, int na, int a, int d0, int blk_l, int b_first) {
  constexpr int ESZ = Esz<KV>::v;
  const int lane = lane_id();
  const int Hkv = P.g.n_kv_heads;
  // the lane's two dims: 2 lane, 2 lane + 1; for int8 K the two dims whose codes
  // sit at bytes 8 D (lane / (D/4)) + (D/2) t + 2 (lane % (D/4)) of the tile (the
  // 16-byte piece layout), so that a wave reads and writes two contiguous runs of
  // D/2 bytes per token (every per-dim step below is independent of which dims a
  // lane has). Lanes 2 lane >= D repeat the lane D/2 below (the same bytes, so
  // the same absmax) and write nothing.
  const bool din = 2 * lane < D;
  const int la = lane & (D / 2 - 1);
  const int lq = la & (D / 4 - 1), lh = la / (D / 4);
  const int c0 = (ESZ == 1 && !IS_V) ? 32 * (lq >> 3) + 16 * lh + 2 * (lq & 7) : 2 * la;
  // element (u, d) of a tile sits at tile_elem(u, 0) + tile_elem(0, d)
  const uint32_t off0 = tile_elem<IS_V>(0, c0, ESZ, D), off1 = tile_elem<IS_V>(0, c0 + 1, ESZ, D);
  auto blk_of = [&](int pos) -> int64_t { return readlane_i(blk_l, pos / BS - b_first); };
  for (int layer = l0; layer < l1; ++layer) {
    uint8_t* L = P.base + (uint64_t)layer * P.g.layer_stride;
    uint8_t* codes = L + (IS_V ? P.g.v_off : P.g.k_off);
    uint8_t* scales = L + (IS_V ? P.g.vs_off : P.g.ks_off);
    // ---- read every moved token ----
    constexpr int RC = 8;
    for (int d = d0; d < na; d += RC) {
      uint32_t e[RC][2];
      float sv[RC];
#pragma unroll
      for (int k = 0; k < RC; ++k) {
        const int q = ctx + readlane_i(a, min(d + k, na - 1));  // past na: a valid token, result dropped
        const int64_t blk = blk_of(q);
        const uint8_t* t = codes + ((uint64_t)blk * Hkv + h) * P.g.tile_bytes + tile_elem<IS_V>(q % BS, 0, ESZ, D);
        if constexpr (ESZ == 4) {
          e[k][0] = *reinterpret_cast<const uint32_t*>(t + off0);
          e[k][1] = *reinterpret_cast<const uint32_t*>(t + off1);
        } else if constexpr (ESZ == 2) {
          e[k][0] = *reinterpret_cast<const uint16_t*>(t + off0);
          e[k][1] = *reinterpret_cast<const uint16_t*>(t + off1);
        } else {
          e[k][0] = t[off0];
          e[k][1] = t[off1];
        }
        sv[k] = 0.f;
        if constexpr (KV == KV_I8_BLK)
          sv[k] = h2f(*reinterpret_cast<const uint16_t*>(scales + ((uint64_t)blk * Hkv + h) * kBlkScaleStep));
        if constexpr (KV == KV_I8_REF) sv[k] = reinterpret_cast<const float*>(scales)[((uint64_t)blk * Hkv + h) * BS + q % BS];
      }
#pragma unroll
      for (int k = 0; k < RC; ++k) {
        if (d + k < na) {
          uint8_t* r = &raw[d + k][2 * lane * ESZ];
          if constexpr (ESZ == 4) *reinterpret_cast<uint2*>(r) = make_uint2(e[k][0], e[k][1]);
          else if constexpr (ESZ == 2) *reinterpret_cast<uint32_t*>(r) = e[k][0] | (e[k][1] << 16);
          else *reinterpret_cast<uint16_t*>(r) = (uint16_t)(e[k][0] | (e[k][1] << 8));
          if (ESZ == 1 && lane == 0) xsc[d + k] = sv[k];
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // ---- write them at context_len + d ----
    if constexpr (KV != KV_I8_BLK) {
      for (int d = d0; d < na; ++d) {
        const int p = ctx + d;
        const int64_t blk = blk_of(p);
        uint8_t* t = codes + ((uint64_t)blk * Hkv + h) * P.g.tile_bytes + tile_elem<IS_V>(p % BS, 0, ESZ, D);
        const uint8_t* r = &raw[d][2 * lane * ESZ];
        if (!din) {
        } else if constexpr (ESZ == 4) {
          *reinterpret_cast<uint32_t*>(t + off0) = reinterpret_cast<const uint32_t*>(r)[0];
          *reinterpret_cast<uint32_t*>(t + off1) = reinterpret_cast<const uint32_t*>(r)[1];
        } else if constexpr (ESZ == 2) {
          *reinterpret_cast<uint16_t*>(t + off0) = reinterpret_cast<const uint16_t*>(r)[0];
          *reinterpret_cast<uint16_t*>(t + off1) = reinterpret_cast<const uint16_t*>(r)[1];
        } else {
          t[off0] = r[0];
          t[off1] = r[1];
        }
        if constexpr (KV == KV_I8_REF) {
          if (lane == 0) reinterpret_cast<float*>(scales)[((uint64_t)blk * Hkv + h) * BS + p % BS] = xsc[d];
        }
      }
    } else {
      // one run per destination block: [ctx + d, ctx + dend)
      int d = d0;
      while (d < na) {
        const int p = ctx + d;
        const int dend = min(na, (p / BS + 1) * BS - ctx);
        const int64_t blk = blk_of(p);
        uint8_t* t = codes + ((uint64_t)blk * Hkv + h) * P.g.tile_bytes;
        uint8_t* const lp0 = t + off0;
        uint8_t* const lp1 = t + off1;
        uint16_t* sp = reinterpret_cast<uint16_t*>(scales + ((uint64_t)blk * Hkv + h) * kBlkScaleStep);
        int cd[BS][2];
#pragma unroll
        for (int u = 0; u < BS; ++u) {
          cd[u][0] = (int8_t)lp0[tile_elem<IS_V>(u, 0, 1, D)];
          cd[u][1] = (int8_t)lp1[tile_elem<IS_V>(u, 0, 1, D)];
        }
        const int o0 = p % BS;
        const uint16_t stored = *sp;
        float s_old = (o0 == 0) ? 0.f : h2f(stored);
        uint16_t s_bits = (o0 == 0) ? (uint16_t)0 : stored;
#pragma unroll 1
        for (int e = d; e < dend; ++e) {
          const uint8_t* r = &raw[e][2 * lane];
          const float sc = xsc[e];
          blk_put(cd, (ctx + e) % BS, s_old, s_bits, (float)(int8_t)r[0] * sc, (float)(int8_t)r[1] * sc);
        }
        const int hi_written = (ctx + dend - 1) % BS;
#pragma unroll
        for (int u = 0; u < BS; ++u) {
          if (din && u <= hi_written) {
            lp0[tile_elem<IS_V>(u, 0, 1, D)] = (uint8_t)(int8_t)cd[u][0];
            lp1[tile_elem<IS_V>(u, 0, 1, D)] = (uint8_t)(int8_t)cd[u][1];
          }
        }
        if (lane == 0) *sp = s_bits;
        d = dend;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  }
}

template <int KV>
DEV void tree_commit(const CommitParams& P) {
  constexpr int ESZ = Esz<KV>::v;
  __shared__ uint8_t raw[2][kMaxCommit][2 * WAVE * ESZ];  // [wave][token][lane's 2 elements]
  __shared__ float xsc[2][kMaxCommit];
  const int s = blockIdx.x, h = blockIdx.y;
  const int l0 = P.layer0 + (int)blockIdx.z * kCommitLayers;
  const int l1 = min(l0 + kCommitLayers, P.layer0 + P.n_layers);
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x / WAVE);  // 0: K, 1: V (wave-uniform)
  const int lane = lane_id();
  // the status of the row is reported once, by wave 0 of (s, KV head 0, layer group 0)
  const bool reporter = P.status && h == 0 && blockIdx.z == 0 && w == 0 && lane == 0;
  auto report = [&](int st) {
    if (reporter) P.status[s] = st;
  };
  const int ctx = P.context_lens[s];
  const int na = P.n_accept[s];
  if (ctx < 0 || na < 0 || na > min(P.accept_stride, kMaxCommit)) { report(COMMIT_BAD_ROW); return; }
  if (na == 0) { report(COMMIT_OK); return; }
  const int32_t* acc = P.accept + (int64_t)s * P.accept_stride;
  const int a = lane < na ? acc[lane] : 0;
  const int prev = __shfl_up(a, 1, WAVE);
  const bool bad = lane < na && (a < lane || a >= kMaxCommit || (lane > 0 && a <= prev));
  if (__builtin_amdgcn_ballot_w64(bad) != 0) { report(COMMIT_BAD_ROW); return; }
  const uint64_t moved = __builtin_amdgcn_ballot_w64(lane < na && a != lane);
  if (moved == 0) { report(COMMIT_OK); return; }  // every accepted node is already in place
  const int d0 = __builtin_ctzll(moved);
  const int last = ctx + readlane_i(a, na - 1);
  const int pt = P.g.page_tiles;
  if ((int64_t)last >= (int64_t)P.bt_stride * BS * pt) { report(COMMIT_PAST_TABLE); return; }
  const int32_t* bt = P.block_tables + (int64_t)s * P.bt_stride;
  const int b_first = (ctx + d0) / BS, nb = last / BS - b_first + 1;  // at most 3 tiles
  // tile b_first + lane: page bt[tile / page_tiles], tile (tile % page_tiles) of that page
  const int pg = lane < nb ? bt[(b_first + lane) / pt] : 0;
  if (__builtin_amdgcn_ballot_w64(lane < nb && (pg < 0 || pg >= P.g.n_blocks / pt)) != 0) {
    report(COMMIT_BAD_PAGE);
    return;
  }
  const int blk_l = pg * pt + (b_first + lane) % pt;
  report(COMMIT_OK);
  // D as a constant, so that tile offsets fold into the instructions
  if (P.g.head_dim == HD) {
    if (w == 0) commit_wave<KV, false, HD>(P, raw[0], xsc[0], h, l0, l1, ctx, na, a, d0, blk_l, b_first);
    else commit_wave<KV, true, HD>(P, raw[1], xsc[1], h, l0, l1, ctx, na, a, d0, blk_l, b_first);
  } else {
    if (w == 0) commit_wave<KV, false, HD / 2>(P, raw[0], xsc[0], h, l0, l1, ctx, na, a, d0, blk_l, b_first);
    else commit_wave<KV, true, HD / 2>(P, raw[1], xsc[1], h, l0, l1, ctx, na, a, d0, blk_l, b_first);
  }
}

DEV uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
constexpr uint64_t kOutlierSalt = 0x6F75746C69657273ull;

// dst[i] = fp16(N(0,1)) by Box-Muller on two counter-based SplitMix64 uniforms,
// times outlier_scale on outlier channels.
__device__ void fill_normal_kernel(const FillParams& P) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.n) return;
  const uint64_t r1 = splitmix64(P.seed ^ (2 * i));
  const uint64_t r2 = splitmix64(P.seed ^ (2 * i + 1));
  const float u1 = ((float)(r1 >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
  const float u2 = (float)(r2 >> 40) * (1.0f / 16777216.0f);           // [0, 1)
  float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
  const uint64_t ch = i % (uint64_t)P.row_len;
  if (splitmix64(P.seed ^ kOutlierSalt ^ ch) % 100 == 0) z *= P.outlier_scale;
  P.dst[i] = f2h(z);
}

// =============================================================================
// Exported kernels (extern "C" names are what the host resolves).
// =============================================================================
#define VK_DECODE(KV, G, QT)                                                        \
  extern "C" __global__ void __launch_bounds__(64)                                  \
      vk_decode_kv##KV##_g##G##_q##QT(const DecodeParams P) {                      \
    decode_unit<KV, G, QT>(P);                                                      \
  }
#define VK_DECODE_G(KV, QT) VK_DECODE(KV, 1, QT) VK_DECODE(KV, 2, QT) VK_DECODE(KV, 4, QT) VK_DECODE(KV, 8, QT)
VK_DECODE_G(0, 0) VK_DECODE_G(0, 1)
VK_DECODE_G(1, 0) VK_DECODE_G(1, 1)
VK_DECODE_G(2, 0) VK_DECODE_G(2, 1)
VK_DECODE_G(3, 0) VK_DECODE_G(3, 1)

#define VK_DECODE_MFMA(KV, G)                                                       \
  extern "C" __global__ void __launch_bounds__(64)                                  \
      vk_decode_mfma_kv##KV##_g##G(const DecodeParams P) {                          \
    attn_unit_mfma<KV, G, 1, false>(P);                                             \
  }
#define VK_DECODE_MFMA_G(KV) VK_DECODE_MFMA(KV, 1) VK_DECODE_MFMA(KV, 2) VK_DECODE_MFMA(KV, 4) VK_DECODE_MFMA(KV, 8)
VK_DECODE_MFMA_G(0) VK_DECODE_MFMA_G(1) VK_DECODE_MFMA_G(2) VK_DECODE_MFMA_G(3)
// fp32 q (split into fp16 hi + lo over fp16 / int8 KV, fp32 over fp32 KV): suffix _q0
#define VK_DECODE_MFMA_Q0(KV, G)                                                    \
  extern "C" __global__ void __launch_bounds__(64)                                  \
      vk_decode_mfma_kv##KV##_g##G##_q0(const DecodeParams P) {                     \
    attn_unit_mfma<KV, G, 1, false, DT_F32>(P);                                     \
  }
#define VK_DECODE_MFMA_Q0_G(KV) \
  VK_DECODE_MFMA_Q0(KV, 1) VK_DECODE_MFMA_Q0(KV, 2) VK_DECODE_MFMA_Q0(KV, 4) VK_DECODE_MFMA_Q0(KV, 8)
VK_DECODE_MFMA_Q0_G(0) VK_DECODE_MFMA_Q0_G(1) VK_DECODE_MFMA_Q0_G(2) VK_DECODE_MFMA_Q0_G(3)

// Workgroup-split decode: up to kWgMaxWaves waves of 64 per workgroup.
#define VK_DECODE_WG(KV, G)                                                         \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves)                    \
      vk_decode_wg_kv##KV##_g##G(const DecodeParams P) {                            \
    attn_wg_mfma<KV, G>(P);                                                         \
  }
#define VK_DECODE_WG_G(KV) VK_DECODE_WG(KV, 1) VK_DECODE_WG(KV, 2) VK_DECODE_WG(KV, 4) VK_DECODE_WG(KV, 8)
VK_DECODE_WG_G(0) VK_DECODE_WG_G(2) VK_DECODE_WG_G(3)
#define VK_DECODE_WG_Q0(KV, G)                                                      \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves)                    \
      vk_decode_wg_kv##KV##_g##G##_q0(const DecodeParams P) {                       \
    attn_wg_mfma<KV, G, DT_F32>(P);                                                 \
  }
#define VK_DECODE_WG_Q0_G(KV) VK_DECODE_WG_Q0(KV, 1) VK_DECODE_WG_Q0(KV, 2) VK_DECODE_WG_Q0(KV, 4) VK_DECODE_WG_Q0(KV, 8)
VK_DECODE_WG_Q0_G(0) VK_DECODE_WG_Q0_G(2) VK_DECODE_WG_Q0_G(3)

// Packed workgroup split (ragged batches): up to kWgMaxWaves waves of 64.
#define VK_DECODE_PK(KV, G, QT, SUF)                                                \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves)                    \
      vk_decode_pk_kv##KV##_g##G##SUF(const DecodeParams P) {                       \
    attn_pk_mfma<KV, G, QT>(P);                                                     \
  }
#define VK_DECODE_PK_G(KV, QT, SUF) \
  VK_DECODE_PK(KV, 1, QT, SUF) VK_DECODE_PK(KV, 2, QT, SUF) VK_DECODE_PK(KV, 4, QT, SUF) VK_DECODE_PK(KV, 8, QT, SUF)
VK_DECODE_PK_G(1, DT_F16, ) VK_DECODE_PK_G(2, DT_F16, ) VK_DECODE_PK_G(3, DT_F16, )
VK_DECODE_PK_G(1, DT_F32, _q0) VK_DECODE_PK_G(2, DT_F32, _q0) VK_DECODE_PK_G(3, DT_F32, _q0)

// Two waves per SIMD (at most 256 registers).
#define VK_TWO_WAVES __attribute__((amdgpu_waves_per_eu(2)))
#define VK_DECODE_SK(KV, G)                                                         \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES          \
      vk_decode_sk_kv##KV##_g##G(const DecodeParams P) {                            \
    attn_streamk_mfma<KV, G>(P);                                                    \
  }
#define VK_DECODE_SK_G(KV) VK_DECODE_SK(KV, 1) VK_DECODE_SK(KV, 2) VK_DECODE_SK(KV, 4) VK_DECODE_SK(KV, 8)
VK_DECODE_SK_G(0) VK_DECODE_SK_G(1) VK_DECODE_SK_G(2) VK_DECODE_SK_G(3)
#define VK_DECODE_SK_Q0(KV, G)                                                      \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES          \
      vk_decode_sk_kv##KV##_g##G##_q0(const DecodeParams P) {                       \
    attn_streamk_mfma<KV, G, DT_F32>(P);                                            \
  }
#define VK_DECODE_SK_Q0_G(KV) VK_DECODE_SK_Q0(KV, 1) VK_DECODE_SK_Q0(KV, 2) VK_DECODE_SK_Q0(KV, 4) VK_DECODE_SK_Q0(KV, 8)
VK_DECODE_SK_Q0_G(0) VK_DECODE_SK_Q0_G(1) VK_DECODE_SK_Q0_G(2) VK_DECODE_SK_Q0_G(3)

// Tree verify: RT tiles of 16 (node, head) rows per wave. Over int8 pools the
// kernels are held to 256 registers (two waves per SIMD); the fp16 ones would
// spill, so they keep one wave per SIMD, and so do the int8 two-tile kernels of
// an fp32 q, whose lo parts (32 registers more) would spill at two waves.
#define VK_TREE(KV, G, RT, QT, ATTR)                                                \
  extern "C" __global__ void __launch_bounds__(64) ATTR                             \
      vk_tree_kv##KV##_g##G##_r##RT##_q##QT(const DecodeParams P) {                 \
    attn_unit_mfma<KV, G, RT, true, QT>(P);                                         \
  }
#define VK_TREE_G(KV, RT, QT, ATTR) \
  VK_TREE(KV, 1, RT, QT, ATTR) VK_TREE(KV, 2, RT, QT, ATTR) VK_TREE(KV, 4, RT, QT, ATTR) VK_TREE(KV, 8, RT, QT, ATTR)
#define VK_TREE_KV(KV, ATTR, ATTR_R2Q0) \
  VK_TREE_G(KV, 1, 0, ATTR) VK_TREE_G(KV, 1, 1, ATTR) VK_TREE_G(KV, 2, 0, ATTR_R2Q0) VK_TREE_G(KV, 2, 1, ATTR)
VK_TREE_KV(0, , )
VK_TREE_KV(1, , )
VK_TREE_KV(2, VK_TWO_WAVES, )
VK_TREE_KV(3, VK_TWO_WAVES, )

// Any other GQA group size ("_gx"): the group size is n_heads / n_kv_heads at run
// time, at most 16 rows per tile (decode), two tiles ("_gx2", split-K) up to 32.
#define VK_GX_DECODE(KV)                                                                                        \
  extern "C" __global__ void __launch_bounds__(64) vk_decode_mfma_kv##KV##_gx(const DecodeParams P) {           \
    attn_unit_mfma<KV, 0, 1, false>(P);                                                                        \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64) vk_decode_mfma_kv##KV##_gx_q0(const DecodeParams P) {        \
    attn_unit_mfma<KV, 0, 1, false, DT_F32>(P);                                                                \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64) vk_decode_mfma_kv##KV##_gx2(const DecodeParams P) {          \
    attn_unit_mfma<KV, 0, 2, false>(P);                                                                        \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64) vk_decode_mfma_kv##KV##_gx2_q0(const DecodeParams P) {       \
    attn_unit_mfma<KV, 0, 2, false, DT_F32>(P);                                                                \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES vk_decode_sk_kv##KV##_gx(const DecodeParams P) { \
    attn_streamk_mfma<KV, 0>(P);                                                                               \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES vk_decode_sk_kv##KV##_gx_q0(const DecodeParams P) { \
    attn_streamk_mfma<KV, 0, DT_F32>(P);                                                                       \
  }
VK_GX_DECODE(0) VK_GX_DECODE(1) VK_GX_DECODE(2) VK_GX_DECODE(3)
#define VK_GX_WG(KV)                                                                                            \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves) vk_decode_wg_kv##KV##_gx(const DecodeParams P) { \
    attn_wg_mfma<KV, 0>(P);                                                                                    \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves) vk_decode_wg_kv##KV##_gx_q0(const DecodeParams P) { \
    attn_wg_mfma<KV, 0, DT_F32>(P);                                                                            \
  }
VK_GX_WG(0) VK_GX_WG(2) VK_GX_WG(3)
// head_dim 64 (64-dim pieces, any group size up to 16): split-K, stream-K and
// the workgroup split
#define VK_D64_DECODE(KV)                                                                                       \
  extern "C" __global__ void __launch_bounds__(64) vk_decode_mfma_kv##KV##_gx_d64(const DecodeParams P) {       \
    attn_unit_mfma<KV, 0, 1, false, DT_F16, HD / 2>(P);                                                        \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64) vk_decode_mfma_kv##KV##_gx_d64_q0(const DecodeParams P) {    \
    attn_unit_mfma<KV, 0, 1, false, DT_F32, HD / 2>(P);                                                        \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES vk_decode_sk_kv##KV##_gx_d64(const DecodeParams P) { \
    attn_streamk_mfma<KV, 0, DT_F16, HD / 2>(P);                                                               \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES vk_decode_sk_kv##KV##_gx_d64_q0(const DecodeParams P) { \
    attn_streamk_mfma<KV, 0, DT_F32, HD / 2>(P);                                                               \
  }
VK_D64_DECODE(0) VK_D64_DECODE(1) VK_D64_DECODE(2) VK_D64_DECODE(3)
#define VK_D64_WG(KV)                                                                                           \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves) vk_decode_wg_kv##KV##_gx_d64(const DecodeParams P) { \
    attn_wg_mfma<KV, 0, DT_F16, HD / 2>(P);                                                                    \
  }                                                                                                             \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves) vk_decode_wg_kv##KV##_gx_d64_q0(const DecodeParams P) { \
    attn_wg_mfma<KV, 0, DT_F32, HD / 2>(P);                                                                    \
  }
VK_D64_WG(0) VK_D64_WG(1) VK_D64_WG(2) VK_D64_WG(3)
// vk_append_rope_decode: the kernels that fold the append (stream-K over fp16
// and I8_BLK pools, the workgroup split over I8_BLK pools), with the new K row
// and q rotated in registers; suffix _rope
#define VK_ROPE_SK(KV, TAG, QT, D)                                                  \
  extern "C" __global__ void __launch_bounds__(64 * kSkWaves) VK_TWO_WAVES          \
      vk_decode_sk_kv##KV##TAG##_rope(const DecodeParams P) {                       \
    attn_streamk_mfma<KV, GTAG_##TAG, QT, D, true>(P);                              \
  }
#define VK_ROPE_WG(KV, TAG, QT, D)                                                  \
  extern "C" __global__ void __launch_bounds__(64 * kWgMaxWaves)                    \
      vk_decode_wg_kv##KV##TAG##_rope(const DecodeParams P) {                       \
    attn_wg_mfma<KV, GTAG_##TAG, QT, D, true>(P);                                   \
  }
#define GTAG__g1 1
#define GTAG__g2 2
#define GTAG__g4 4
#define GTAG__g8 8
#define GTAG__gx 0
#define GTAG__gx_d64 0
#define GTAG__g1_q0 1
#define GTAG__g2_q0 2
#define GTAG__g4_q0 4
#define GTAG__g8_q0 8
#define GTAG__gx_q0 0
#define GTAG__gx_d64_q0 0
#define VK_ROPE_ALL(M, KV)                                                                       \
  M(KV, _g1, DT_F16, HD) M(KV, _g2, DT_F16, HD) M(KV, _g4, DT_F16, HD) M(KV, _g8, DT_F16, HD)    \
  M(KV, _gx, DT_F16, HD) M(KV, _gx_d64, DT_F16, HD / 2)                                          \
  M(KV, _g1_q0, DT_F32, HD) M(KV, _g2_q0, DT_F32, HD) M(KV, _g4_q0, DT_F32, HD)                  \
  M(KV, _g8_q0, DT_F32, HD) M(KV, _gx_q0, DT_F32, HD) M(KV, _gx_d64_q0, DT_F32, HD / 2)
VK_ROPE_ALL(VK_ROPE_SK, 1) VK_ROPE_ALL(VK_ROPE_SK, 3) VK_ROPE_ALL(VK_ROPE_WG, 3)
#define VK_GX_TREE(KV, RT, QT, ATTR)                                                                            \
  extern "C" __global__ void __launch_bounds__(64) ATTR vk_tree_kv##KV##_gx_r##RT##_q##QT(const DecodeParams P) { \
    attn_unit_mfma<KV, 0, RT, true, QT>(P);                                                                    \
  }
#define VK_GX_TREE_KV(KV, ATTR, ATTR_R2Q0) \
  VK_GX_TREE(KV, 1, 0, ATTR) VK_GX_TREE(KV, 1, 1, ATTR) VK_GX_TREE(KV, 2, 0, ATTR_R2Q0) VK_GX_TREE(KV, 2, 1, ATTR)
VK_GX_TREE_KV(0, , ) VK_GX_TREE_KV(1, , ) VK_GX_TREE_KV(2, VK_TWO_WAVES, ) VK_GX_TREE_KV(3, VK_TWO_WAVES, )
// head_dim 64 (pools of 64-dim tiles): the tree kernels on 64-dim pieces, any
// group size
#define VK_GX_TREE_D64(KV, RT, QT, ATTR)                                                                        \
  extern "C" __global__ void __launch_bounds__(64) ATTR vk_tree_kv##KV##_gx_d64_r##RT##_q##QT(const DecodeParams P) { \
    attn_unit_mfma<KV, 0, RT, true, QT, HD / 2>(P);                                                            \
  }
#define VK_GX_TREE_D64_KV(KV, ATTR, ATTR_R2Q0) \
  VK_GX_TREE_D64(KV, 1, 0, ATTR) VK_GX_TREE_D64(KV, 1, 1, ATTR) VK_GX_TREE_D64(KV, 2, 0, ATTR_R2Q0) VK_GX_TREE_D64(KV, 2, 1, ATTR)
VK_GX_TREE_D64_KV(0, , ) VK_GX_TREE_D64_KV(1, VK_TWO_WAVES, VK_TWO_WAVES)
VK_GX_TREE_D64_KV(2, VK_TWO_WAVES, VK_TWO_WAVES) VK_GX_TREE_D64_KV(3, VK_TWO_WAVES, VK_TWO_WAVES)

// Shared-prefix pass of tree verify: 8 waves (two per SIMD) per workgroup.
#define VK_TREE_PFX(KV, G, QT)                                                      \
  extern "C" __global__ void __launch_bounds__(64 * kPfxWaves)                      \
      __attribute__((amdgpu_waves_per_eu(kPfxWaves / 4))) vk_tree_pfx_kv##KV##_g##G##_q##QT(const DecodeParams P) { \
    tree_prefix_mfma<KV, G, QT>(P);                                                 \
  }
#define VK_TREE_PFX_G(KV, QT) \
  VK_TREE_PFX(KV, 1, QT) VK_TREE_PFX(KV, 2, QT) VK_TREE_PFX(KV, 4, QT) VK_TREE_PFX(KV, 8, QT)
VK_TREE_PFX_G(1, 0) VK_TREE_PFX_G(1, 1) VK_TREE_PFX_G(3, 0) VK_TREE_PFX_G(3, 1)
#define VK_GX_TREE_PFX(KV, QT)                                                      \
  extern "C" __global__ void __launch_bounds__(64 * kPfxWaves)                      \
      __attribute__((amdgpu_waves_per_eu(kPfxWaves / 4))) vk_tree_pfx_kv##KV##_gx_q##QT(const DecodeParams P) { \
    tree_prefix_mfma<KV, 0, QT>(P);                                                 \
  }
VK_GX_TREE_PFX(1, 0) VK_GX_TREE_PFX(1, 1) VK_GX_TREE_PFX(3, 0) VK_GX_TREE_PFX(3, 1)
// pools of 64-dim tiles: the pass built for 64 dims, any group size
#define VK_GX_TREE_PFX_D64(KV, QT)                                                  \
  extern "C" __global__ void __launch_bounds__(64 * kPfxWaves)                      \
      __attribute__((amdgpu_waves_per_eu(kPfxWaves / 4))) vk_tree_pfx_kv##KV##_gx_d64_q##QT(const DecodeParams P) { \
    tree_prefix_mfma<KV, 0, QT, HD / 2>(P);                                         \
  }
VK_GX_TREE_PFX_D64(1, 0) VK_GX_TREE_PFX_D64(1, 1) VK_GX_TREE_PFX_D64(3, 0) VK_GX_TREE_PFX_D64(3, 1)


#define VK_APPEND(KV) \
  extern "C" __global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(4)))                         \
      vk_append_kv##KV(const AppendParams P) { append_kernel<KV>(P); }
VK_APPEND(0) VK_APPEND(1) VK_APPEND(2) VK_APPEND(3)
extern "C" __global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(4)))
    vk_append_kv3_d64(const AppendParams P) { append_kernel<KV_I8_BLK, HD / 2>(P); }

extern "C" __global__ void __launch_bounds__(256) vk_slot_mapping(const SlotMapParams P) { slot_mapping_kernel(P); }
extern "C" __global__ void __launch_bounds__(256) vk_copy_blocks(const CopyParams P) { copy_blocks_kernel(P); }
extern "C" __global__ void __launch_bounds__(256) vk_fill_normal_f16(const FillParams P) { fill_normal_kernel(P); }
extern "C" __global__ void __launch_bounds__(256) vk_decode_merge(const MergeParams P) { decode_merge(P); }
extern "C" __global__ void __launch_bounds__(256) vk_decode_merge_sk(const MergeParams P) { decode_merge_sk(P); }
extern "C" __global__ void __launch_bounds__(256) vk_nixl_check(const NixlParams P) { nixl_check_kernel(P); }
extern "C" __global__ void __launch_bounds__(256) vk_nixl_copy(const NixlParams P) { nixl_copy_kernel(P); }
#define VK_COMMIT(KV) \
  extern "C" __global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(4)))                         \
      vk_tree_commit_kv##KV(const CommitParams P) { tree_commit<KV>(P); }
VK_COMMIT(0) VK_COMMIT(1) VK_COMMIT(2) VK_COMMIT(3)

