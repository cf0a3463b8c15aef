// velokv_kernels.hip -- hand-written gfx950 (CDNA4) kernels of the KV-cache hot path.
//
// Built with `hipcc --offload-arch=gfx950 --offload-device-only` into a code object
// that the host library loads with hipModuleLoad and launches with
// hipModuleLaunchKernel. Every kernel takes one argument struct (velokv_params.h).
//
// Block size 16 and head_dim 128 are compile-time constants of the attention and
// append kernels; the host rejects other shapes with VK_ERR_UNSUPPORTED.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "velokv_params.h"

using namespace velokv;

#define DEV static __device__ __forceinline__

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int BS = 16;    // tokens per block
constexpr int HD = 128;   // head_dim
constexpr int WAVE = 64;
constexpr int CHUNK_BLOCKS = 16;                 // blocks per two-phase chunk
constexpr int CHUNK_TOKENS = CHUNK_BLOCKS * BS;  // 256
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
DEV uint32_t pack_h2(float a, float b) {
  return (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
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
// part). The partition is walked in chunks of 16 blocks (256 tokens); each chunk
// runs in phases so the softmax max inside a chunk is exact:
//   phase 1  K tiles [tok][D]: lane = (token lane>>2, 32-dim slice lane&3). Dot
//            products with the G query heads of the GQA group are summed over
//            the quad; the lane keeps the score of (its token, head (lane&3)+4k)
//            and stores it in LDS.
//   phase 1b the chunk max joins the running max (online softmax across chunks;
//            accumulators are rescaled when it grows); p = 2^(score - M) and
//            p~ = p * v_scale go to LDS as (token pair, head) pairs.
//   phase 2  V tiles [tok/2][D][2]: lane = (dims 2*lane, 2*lane+1), all 16
//            tokens; acc[g][d] += p~_2j * v_2j[d] + p~_2j+1 * v_2j+1[d].
// FAST (q fp16 and fp16/int8 KV): v_dot2_f32_f16 on exact int8->fp16 codes and
// fp16 p~ pairs. Otherwise fp32 FMA on dequantized values.
// The unit writes unnormalised partials (acc, running max M in log2 units, sum l);
// vk_decode_merge combines the partitions of a sequence.
// Algorithm of kernels.metal:440-501 / 672-732 and llama_cpu.rs:255-284.
// =============================================================================
template <int KV, int G, int QT>
DEV void decode_unit(const DecodeParams& P) {
  constexpr int ESZ = Esz<KV>::v;
  constexpr bool FAST = (QT == DT_F16) && (KV != KV_F32);
  constexpr bool BLK = (KV == KV_I8_BLK);
  constexpr bool REF = (KV == KV_I8_REF);
  constexpr int SPL = (G >= 4) ? G / 4 : 1;   // score slots per lane per block
  constexpr int KDW = 8 * ESZ;                // dwords of K per lane per block
  constexpr int VDW = ESZ;                    // dwords of V per lane per token pair
  constexpr int CH = 4 / ESZ;                 // blocks per load batch
  constexpr int QW = FAST ? 16 : 32;          // q registers per head
  constexpr int PW = FAST ? 1 : 2;            // LDS dwords per (pair, head)

  __shared__ float s_lds[CHUNK_BLOCKS * SPL * WAVE];
  __shared__ uint32_t p_lds[CHUNK_BLOCKS * 8 * G * PW];

  const int lane = lane_id();
  const int t = lane >> 2;   // token of the K tile this lane reads
  const int c = lane & 3;    // 32-dim slice of the K tile

  const int unit = blockIdx.x;
  const int kvh = unit % P.n_kv_heads;
  const int rest = unit / P.n_kv_heads;
  const int part = rest % P.max_parts;
  const int s = rest / P.max_parts;
  if (s >= P.n_seqs) return;

  const int cap = min(P.max_parts * P.part_tokens, P.bt_stride * BS);
  const int ctx = max(0, min(P.context_lens[s], cap));
  const int start = part * P.part_tokens;
  if (start >= ctx) return;
  const int end = min(start + P.part_tokens, ctx);
  int row = P.seq_rows ? P.seq_rows[s] : s;
  if (P.bt_rows > 0) row = min(max(row, 0), P.bt_rows - 1);
  const int32_t* bt = P.block_tables + (int64_t)row * P.bt_stride;
  const int H = P.n_heads;
  const int Hkv = P.n_kv_heads;
  const uint32_t tile = P.tile_bytes;
  const int nb_max = P.n_blocks - 1;

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

  float Mrun[G];   // running max per head (log2 units), wave-uniform
  float lrun[SPL]; // per-lane partial softmax denominators
  float acc[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) { Mrun[g] = kNegInf; acc[g][0] = 0.f; acc[g][1] = 0.f; }
#pragma unroll
  for (int k = 0; k < SPL; ++k) lrun[k] = 0.f;

  for (int cs = start; cs < end; cs += CHUNK_TOKENS) {
    const int ntok = min(CHUNK_TOKENS, end - cs);
    const int nblk = (ntok + BS - 1) / BS;
    const int blk0 = cs / BS;

    // block ids (and per-(block, head) scales) of the chunk, one per lane
    int blkv = 0;
    float ksv = 1.f, vsv = 1.f;
    if (lane < nblk) {
      blkv = min(max(bt[blk0 + lane], 0), nb_max);
      if constexpr (BLK) {
        const uint16_t* ks = reinterpret_cast<const uint16_t*>(P.ks);
        const uint16_t* vs = reinterpret_cast<const uint16_t*>(P.vs);
        ksv = h2f(ks[(int64_t)blkv * Hkv + kvh]);
        vsv = h2f(vs[(int64_t)blkv * Hkv + kvh]);
      }
    }

    // ---------------- phase 1: scores ----------------
    float mloc[SPL];
#pragma unroll
    for (int k = 0; k < SPL; ++k) mloc[k] = kNegInf;
    float vsc_ref[CHUNK_BLOCKS];  // REF: V scale of this lane's token, per block
    (void)vsc_ref;

    for (int i0 = 0; i0 < nblk; i0 += CH) {
      DW<KDW> kw[CH];
      float ksr[CH];
      float vsr[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int bi = min(i0 + u, nblk - 1);
        const int blk = readlane_i(blkv, bi);
        const uint8_t* tp = P.kc + ((uint64_t)blk * Hkv + kvh) * tile;
        kw[u] = load_dw<KDW>(tp + lane * (KDW * 4));
        if constexpr (REF) {
          const float* ks = reinterpret_cast<const float*>(P.ks);
          const float* vs = reinterpret_cast<const float*>(P.vs);
          const int64_t si = ((int64_t)blk * Hkv + kvh) * BS + t;
          ksr[u] = ks[si];
          vsr[u] = vs[si];
        } else {
          ksr[u] = 1.f; vsr[u] = 1.f;
        }
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int i = i0 + u;
        if (i < nblk) {
          float a[G];
#pragma unroll
          for (int g = 0; g < G; ++g) a[g] = 0.f;
          if constexpr (FAST) {
            if constexpr (ESZ == 1) {
#pragma unroll
              for (int w = 0; w < 8; ++w) {
                uint32_t lo, hi;
                i8x4_to_h2x2(kw[u].d[w], lo, hi);
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
                for (int g = 0; g < G; ++g) a[g] = dot2(qh[g][w], kw[u].d[w], a[g]);
            }
          } else {
            float kf[32];
#pragma unroll
            for (int d = 0; d < 32; ++d) {
              if constexpr (ESZ == 1) kf[d] = byte_to_f(kw[u].d[d >> 2], d & 3);
              else if constexpr (ESZ == 2) kf[d] = (d & 1) ? half_hi(kw[u].d[d >> 1]) : half_lo(kw[u].d[d >> 1]);
              else kf[d] = bitcast<float>(kw[u].d[d]);
            }
#pragma unroll
            for (int d = 0; d < 32; ++d)
#pragma unroll
              for (int g = 0; g < G; ++g) a[g] = fmaf(bitcast<float>(qh[g][d]), kf[d], a[g]);
          }
          // sum over the quad (the 4 slices of one token)
#pragma unroll
          for (int g = 0; g < G; ++g) {
            a[g] += dpp<DPP_QUAD_XOR1>(a[g]);
            a[g] += dpp<DPP_QUAD_XOR2>(a[g]);
          }
          float kscale = P.scale_log2;
          if constexpr (BLK) kscale *= readlane_f(ksv, i);
          if constexpr (REF) kscale *= ksr[u];
          const bool valid = (cs + i * BS + t) < end;
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
            v = valid ? v * kscale : kNegInf;
            mloc[k] = fmaxf(mloc[k], v);
            s_lds[(i * SPL + k) * WAVE + lane] = v;
          }
          if constexpr (REF) {
            // kept for phase 1b, indexed by the block of the chunk
#pragma unroll
            for (int b = 0; b < CHUNK_BLOCKS; ++b)
              if (b == i) vsc_ref[b] = vsr[u];
          }
        }
      }
    }

    // ---------------- phase 1b: running max, p, p~ ----------------
    float Mnew[G], alpha[G];
#pragma unroll
    for (int k = 0; k < SPL; ++k) mloc[k] = max_same_quadpos(mloc[k]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mc;
      if constexpr (G >= 4) mc = readlane_f(mloc[g / 4], g % 4);
      else if constexpr (G == 2) mc = readlane_f(mloc[0], g);
      else mc = readlane_f(mloc[0], 0);
      Mnew[g] = fmaxf(Mrun[g], mc);
      alpha[g] = __builtin_amdgcn_exp2f(Mrun[g] - Mnew[g]);  // 0 on the first chunk
      Mrun[g] = Mnew[g];
    }
    bool rescale = false;
#pragma unroll
    for (int g = 0; g < G; ++g) rescale |= (alpha[g] != 1.f);
    if (rescale) {
#pragma unroll
      for (int g = 0; g < G; ++g) { acc[g][0] *= alpha[g]; acc[g][1] *= alpha[g]; }
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        float al = alpha[0];
#pragma unroll
        for (int g = 1; g < G; ++g) al = (slot_head(k) == g) ? alpha[g] : al;
        lrun[k] *= al;
      }
    }
    float Mlane[SPL];
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
      float m = Mnew[0];
#pragma unroll
      for (int g = 1; g < G; ++g) m = (slot_head(k) == g) ? Mnew[g] : m;
      Mlane[k] = m;
    }
    const int jp = t >> 1, e = t & 1;
#pragma unroll 4
    for (int i = 0; i < nblk; ++i) {
      float vscale;
      if constexpr (BLK) vscale = readlane_f(vsv, i);
      else if constexpr (REF) {
        vscale = vsc_ref[0];
#pragma unroll
        for (int b = 1; b < CHUNK_BLOCKS; ++b) vscale = (b == i) ? vsc_ref[b] : vscale;
      } else vscale = 1.f;
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        const float sv = s_lds[(i * SPL + k) * WAVE + lane];
        const float p = __builtin_amdgcn_exp2f(sv - Mlane[k]);
        if (owner) {
          lrun[k] += p;
          const int g = slot_head(k);
          const float pt = p * vscale;
          if constexpr (FAST) {
            reinterpret_cast<uint16_t*>(p_lds)[(((i * 8 + jp) * G + g) << 1) + e] = f2h(pt);
          } else {
            reinterpret_cast<float*>(p_lds)[(((i * 8 + jp) * G + g) << 1) + e] = pt;
          }
        }
      }
    }
    __syncthreads();

    // ---------------- phase 2: V ----------------
    const int last_tok_in_blk = (end - cs) - (nblk - 1) * BS;  // valid tokens of the last block
    for (int i0 = 0; i0 < nblk; i0 += CH) {
      DW<VDW> vw[CH][8];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int bi = min(i0 + u, nblk - 1);
        const int blk = readlane_i(blkv, bi);
        const uint8_t* tp = P.vc + ((uint64_t)blk * Hkv + kvh) * tile;
#pragma unroll
        for (int j = 0; j < 8; ++j) vw[u][j] = load_dw<VDW>(tp + j * (HD * 2 * ESZ) + lane * (VDW * 4));
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int i = i0 + u;
        if (i < nblk) {
          const bool partial = (i == nblk - 1) && (last_tok_in_blk < BS);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            uint32_t pp[G * PW];
            const uint32_t* src = p_lds + (i * 8 + j) * G * PW;
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
            // element order in the lane's V words: [d0: t0, t1][d1: t0, t1]
            const bool z0 = partial && (2 * j >= last_tok_in_blk);
            const bool z1 = partial && (2 * j + 1 >= last_tok_in_blk);
            if constexpr (FAST) {
              uint32_t v0, v1;
              if constexpr (ESZ == 1) i8x4_to_h2x2(vw[u][j].d[0], v0, v1);
              else { v0 = vw[u][j].d[0]; v1 = vw[u][j].d[1]; }
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
                const uint32_t w = vw[u][j].d[0];
                v00 = byte_to_f(w, 0); v01 = byte_to_f(w, 1); v10 = byte_to_f(w, 2); v11 = byte_to_f(w, 3);
              } else if constexpr (ESZ == 2) {
                v00 = half_lo(vw[u][j].d[0]); v01 = half_hi(vw[u][j].d[0]);
                v10 = half_lo(vw[u][j].d[1]); v11 = half_hi(vw[u][j].d[1]);
              } else {
                v00 = bitcast<float>(vw[u][j].d[0]); v01 = bitcast<float>(vw[u][j].d[1]);
                v10 = bitcast<float>(vw[u][j].d[2]); v11 = bitcast<float>(vw[u][j].d[3]);
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
    }
    __syncthreads();
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
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t pr = (hrow0 + g) * P.max_parts + part;
    reinterpret_cast<float2*>(P.part_acc + pr * HD)[lane] = make_float2(acc[g][0], acc[g][1]);
    if (lane == g) reinterpret_cast<float2*>(P.part_ml)[pr] = make_float2(Mrun[g], lsum[g]);
  }
}

// Combine the partitions of one (sequence, head): out = sum_p w_p acc_p / sum_p w_p l_p,
// w_p = 2^(M_p - max_p M_p). One wave per (sequence, head).
__device__ void decode_merge(const MergeParams& P) {
  const int lane = lane_id();
  const int r = blockIdx.x * (blockDim.x / WAVE) + (threadIdx.x / WAVE);
  if (r >= P.n_seqs * P.n_heads) return;
  const int s = r / P.n_heads;
  const int ctx = max(0, min(P.context_lens[s], P.max_parts * P.part_tokens));
  const int np = (ctx + P.part_tokens - 1) / P.part_tokens;
  const float2* ml = reinterpret_cast<const float2*>(P.part_ml) + (int64_t)r * P.max_parts;
  float M = kNegInf;
  for (int p = lane; p < np; p += WAVE) M = fmaxf(M, ml[p].x);
  M = wave_max(M);
  float L = 0.f;
  for (int p = lane; p < np; p += WAVE) L += __builtin_amdgcn_exp2f(ml[p].x - M) * ml[p].y;
  L = wave_sum(L);
  float o0 = 0.f, o1 = 0.f;
  const float2* pa = reinterpret_cast<const float2*>(P.part_acc) + (int64_t)r * P.max_parts * (HD / 2);
  for (int p0 = 0; p0 < np; p0 += WAVE) {
    const float w = (p0 + lane < np) ? __builtin_amdgcn_exp2f(ml[p0 + lane].x - M) : 0.f;
    const int n = min(WAVE, np - p0);
    for (int k = 0; k < n; ++k) {
      const float wk = readlane_f(w, k);
      const float2 a = pa[(int64_t)(p0 + k) * (HD / 2) + lane];
      o0 = fmaf(wk, a.x, o0);
      o1 = fmaf(wk, a.y, o1);
    }
  }
  const float inv = (np > 0 && L > 0.f) ? 1.f / L : 0.f;
  reinterpret_cast<float2*>(P.out)[(int64_t)r * (HD / 2) + lane] = make_float2(o0 * inv, o1 * inv);
}

// =============================================================================
// KV append (kernels.metal:619-645 kv_update, 753-802 kv_update_int8).
// Workgroup (token n, KV head h) with two waves: wave 0 writes K, wave 1 writes V.
// Lane l owns dims 2l and 2l+1.
// =============================================================================
DEV void load_x2(const void* src, int in_dtype, int64_t off, float& x0, float& x1) {
  if (in_dtype == DT_F16) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(src) + off)[0];
    x0 = half_lo(w); x1 = half_hi(w);
  } else {
    const float2 v = reinterpret_cast<const float2*>(reinterpret_cast<const float*>(src) + off)[0];
    x0 = v.x; x1 = v.y;
  }
}

// Byte offset inside a (block, head) tile of element (token, dim).
template <bool IS_V>
DEV uint32_t tile_elem(int tok, int d, int esz) {
  return IS_V ? (uint32_t)(((tok >> 1) * HD + d) * 2 + (tok & 1)) * esz
              : (uint32_t)(tok * HD + d) * esz;
}

DEV int clamp127(float r) { return (int)fminf(fmaxf(r, -127.f), 127.f); }

// VK_KV_I8_BLK: per-(block, head) fp16 scale, round-half-even codes clamped to +-127.
// A run = consecutive tokens of the call that fall in one block; the run's first
// token does the work for all of them, in order, keeping the block's codes in
// registers:
//   s_old = (offset == 0) ? 0 : stored scale
//   s_new = max(s_old, fp16(amax / 127))
//   if s_new > s_old: c' = clamp(rne((c * s_old) / s_new)) for tokens before offset
//   c = s_new > 0 ? clamp(rne(x / s_new)) : 0
template <bool IS_V>
DEV void append_blk(const AppendParams& P, const void* src, uint8_t* codes, uint16_t* scales) {
  const int lane = lane_id();
  const int n = blockIdx.x, h = blockIdx.y;
  const int64_t slot = P.slot_mapping[n];
  if (slot < 0) return;
  const int bs = BS;
  const int64_t b = slot / bs;
  // Not the first token of its run when the previous non-padding token of the
  // call is in the same block (padding slots are negative).
  for (int m = n - 1; m >= 0; --m) {
    const int64_t prev = P.slot_mapping[m];
    if (prev < 0) continue;
    if (prev / bs == b) return;
    break;
  }
  if (b >= P.g.n_blocks) return;
  const int Hkv = P.g.n_kv_heads;
  uint8_t* tile = codes + ((uint64_t)b * Hkv + h) * P.g.tile_bytes;
  uint16_t* sp = scales + (uint64_t)b * Hkv + h;
  const int d0 = 2 * lane;

  int cd[BS][2];
#pragma unroll
  for (int u = 0; u < BS; ++u) {
    cd[u][0] = (int8_t)tile[tile_elem<IS_V>(u, d0, 1)];
    cd[u][1] = (int8_t)tile[tile_elem<IS_V>(u, d0 + 1, 1)];
  }
  int o = (int)(slot % bs);
  float s_old = (o == 0) ? 0.f : h2f(*sp);
  uint16_t s_bits = (o == 0) ? (uint16_t)0 : *sp;
  int hi_written = -1;
  for (int m = n; m < P.n_tok;) {
    float x0, x1;
    load_x2(src, P.in_dtype, ((int64_t)m * Hkv + h) * HD + d0, x0, x1);
    const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
    const uint16_t cand = f2h(amax / 127.0f);
    float s_new = s_old;
    if (h2f(cand) > s_old) { s_new = h2f(cand); s_bits = cand; }
    if (s_new > s_old && o > 0) {
#pragma unroll
      for (int u = 0; u < BS; ++u) {
        if (u < o) {
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const float r = ((float)cd[u][k] * s_old) / s_new;
            cd[u][k] = clamp127(__builtin_rintf(r));
          }
        }
      }
    }
    const int c0 = (s_new > 0.f) ? clamp127(__builtin_rintf(x0 / s_new)) : 0;
    const int c1 = (s_new > 0.f) ? clamp127(__builtin_rintf(x1 / s_new)) : 0;
#pragma unroll
    for (int u = 0; u < BS; ++u)
      if (u == o) { cd[u][0] = c0; cd[u][1] = c1; }
    hi_written = max(hi_written, o);
    s_old = s_new;
    // next token of the run (padding slots in between are skipped)
    ++m;
    while (m < P.n_tok && P.slot_mapping[m] < 0) ++m;
    if (m >= P.n_tok) break;
    const int64_t ns = P.slot_mapping[m];
    if (ns / bs != b) break;
    o = (int)(ns % bs);
    if (o == 0) { s_old = 0.f; s_bits = 0; }
  }
#pragma unroll
  for (int u = 0; u < BS; ++u) {
    if (u <= hi_written) {
      tile[tile_elem<IS_V>(u, d0, 1)] = (uint8_t)(int8_t)cd[u][0];
      tile[tile_elem<IS_V>(u, d0 + 1, 1)] = (uint8_t)(int8_t)cd[u][1];
    }
  }
  if (lane == 0) *sp = s_bits;
}

// VK_KV_I8_REF: per-(token, head) fp32 scale = amax/127, codes = trunc(x * (127/amax)).
template <bool IS_V>
DEV void append_ref(const AppendParams& P, const void* src, uint8_t* codes, float* scales) {
  const int lane = lane_id();
  const int n = blockIdx.x, h = blockIdx.y;
  const int64_t slot = P.slot_mapping[n];
  if (slot < 0) return;
  const int64_t b = slot / BS;
  const int o = (int)(slot % BS);
  if (b >= P.g.n_blocks) return;
  const int Hkv = P.g.n_kv_heads;
  const int d0 = 2 * lane;
  float x0, x1;
  load_x2(src, P.in_dtype, ((int64_t)n * Hkv + h) * HD + d0, x0, x1);
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const float scale = amax / 127.0f;
  const float inv = amax > 0.f ? 127.0f / amax : 0.f;
  uint8_t* tile = codes + ((uint64_t)b * Hkv + h) * P.g.tile_bytes;
  tile[tile_elem<IS_V>(o, d0, 1)] = (uint8_t)(int8_t)(int)(x0 * inv);
  tile[tile_elem<IS_V>(o, d0 + 1, 1)] = (uint8_t)(int8_t)(int)(x1 * inv);
  if (lane == 0) scales[((uint64_t)b * Hkv + h) * BS + o] = scale;
}

// VK_KV_F16 / VK_KV_F32: plain copy (with RNE conversion to fp16 when needed).
template <bool IS_V, int ESZ>
DEV void append_plain(const AppendParams& P, const void* src, uint8_t* codes) {
  const int lane = lane_id();
  const int n = blockIdx.x, h = blockIdx.y;
  const int64_t slot = P.slot_mapping[n];
  if (slot < 0) return;
  const int64_t b = slot / BS;
  const int o = (int)(slot % BS);
  if (b >= P.g.n_blocks) return;
  const int Hkv = P.g.n_kv_heads;
  const int d0 = 2 * lane;
  uint8_t* tile = codes + ((uint64_t)b * Hkv + h) * P.g.tile_bytes;
  if (ESZ == 2 && P.in_dtype == DT_F16) {
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src) + ((int64_t)n * Hkv + h) * HD + d0;
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0, 2)) = s16[0];
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0 + 1, 2)) = s16[1];
    return;
  }
  float x0, x1;
  load_x2(src, P.in_dtype, ((int64_t)n * Hkv + h) * HD + d0, x0, x1);
  if constexpr (ESZ == 2) {
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0, 2)) = f2h(x0);
    *reinterpret_cast<uint16_t*>(tile + tile_elem<IS_V>(o, d0 + 1, 2)) = f2h(x1);
  } else {
    *reinterpret_cast<float*>(tile + tile_elem<IS_V>(o, d0, 4)) = x0;
    *reinterpret_cast<float*>(tile + tile_elem<IS_V>(o, d0 + 1, 4)) = x1;
  }
}

template <int KV>
DEV void append_kernel(const AppendParams& P) {
  const bool is_v = (threadIdx.x >= WAVE);
  uint8_t* L = P.base + (uint64_t)P.layer * P.g.layer_stride;
  const void* src = is_v ? P.v : P.k;
  uint8_t* codes = L + (is_v ? P.g.v_off : P.g.k_off);
  if constexpr (KV == KV_I8_BLK) {
    uint16_t* sc = reinterpret_cast<uint16_t*>(L + (is_v ? P.g.vs_off : P.g.ks_off));
    if (is_v) append_blk<true>(P, src, codes, sc); else append_blk<false>(P, src, codes, sc);
  } else if constexpr (KV == KV_I8_REF) {
    float* sc = reinterpret_cast<float*>(L + (is_v ? P.g.vs_off : P.g.ks_off));
    if (is_v) append_ref<true>(P, src, codes, sc); else append_ref<false>(P, src, codes, sc);
  } else if constexpr (KV == KV_F16) {
    if (is_v) append_plain<true, 2>(P, src, codes); else append_plain<false, 2>(P, src, codes);
  } else {
    if (is_v) append_plain<true, 4>(P, src, codes); else append_plain<false, 4>(P, src, codes);
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
  const uint64_t sb = (uint64_t)P.g.n_kv_heads * P.g.stile_bytes;  // scale bytes per block
  const uint8_t* cs = L + (is_v ? P.g.v_off : P.g.k_off) + (uint64_t)src * cb;
  uint8_t* cdst = L + (is_v ? P.g.v_off : P.g.k_off) + (uint64_t)dst * cb;
  for (uint64_t i = threadIdx.x; i < cb / 16; i += blockDim.x)
    reinterpret_cast<uint4*>(cdst)[i] = reinterpret_cast<const uint4*>(cs)[i];
  if (sb) {
    const uint8_t* ss = L + (is_v ? P.g.vs_off : P.g.ks_off) + (uint64_t)src * sb;
    uint8_t* sd = L + (is_v ? P.g.vs_off : P.g.ks_off) + (uint64_t)dst * sb;
    for (uint64_t i = threadIdx.x; i < sb / 2; i += blockDim.x)
      reinterpret_cast<uint16_t*>(sd)[i] = reinterpret_cast<const uint16_t*>(ss)[i];
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

extern "C" __global__ void __launch_bounds__(256) vk_decode_merge(const MergeParams P) { decode_merge(P); }

#define VK_APPEND(KV) \
  extern "C" __global__ void __launch_bounds__(128) vk_append_kv##KV(const AppendParams P) { append_kernel<KV>(P); }
VK_APPEND(0) VK_APPEND(1) VK_APPEND(2) VK_APPEND(3)

extern "C" __global__ void __launch_bounds__(256) vk_slot_mapping(const SlotMapParams P) { slot_mapping_kernel(P); }
extern "C" __global__ void __launch_bounds__(256) vk_copy_blocks(const CopyParams P) { copy_blocks_kernel(P); }
extern "C" __global__ void __launch_bounds__(256) vk_fill_normal_f16(const FillParams P) { fill_normal_kernel(P); }
