/*
 * velokv_oracle.c -- CPU restatement of the reference's KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker or the timed CPU
 * baseline. The product path (libvelokv.so + the gfx950 code object) never
 * calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, optional OpenMP).
 *
 * Two families of functions:
 *  (1) vko_ref_*: the reference's kernels restated on the REFERENCE layout
 *      ([blk][tok][head][D] fp32, [blk][tok][head][D codes + 4-byte fp32 scale]
 *      int8) with the reference's operation order.
 *  (2) vko_*: the same semantics on the BUILD layout the GPU pool uses
 *      (K [blk][head][tok][D] for fp32 / fp16 and [blk][head][D/16 % 2][tok][D/32][16]
 *      for int8, V [blk][head][tok/2][D][2], scales separate; elem_off),
 *      plus what the reference lacks (fp16 KV, per-block INT8 scales,
 *      tree verify, copy-on-write), so outputs compare byte for byte.
 *
 * Parity pins for every function are in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define VKO_F32 0
#define VKO_F16 1
#define VKO_I8_REF 2
#define VKO_I8_BLK 3

/* ------------------------------------------------------------------------- */
/* fp16 <-> fp32                                                              */
/* ------------------------------------------------------------------------- */

/* quant.rs:18-34 (f16_to_f32): subnormals as mant * 2^-24, exp 31 -> Inf/NaN,
 * normals by re-biasing the exponent (+112) and shifting the mantissa by 13. */
float vko_f16_to_f32(uint16_t bits) {
  const uint32_t sign = ((uint32_t)(bits >> 15)) << 31;
  const uint32_t exp = (bits >> 10) & 0x1Fu;
  const uint32_t mant = bits & 0x3FFu;
  union { uint32_t u; float f; } r;
  if (exp == 0) {
    const float v = (float)mant * (1.0f / (float)(1u << 24));
    return sign ? -v : v;
  } else if (exp == 31) {
    r.u = sign | 0x7F800000u | (mant << 13);
    return r.f;
  }
  r.u = sign | ((exp + 112u) << 23) | (mant << 13);
  return r.f;
}

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even. The reference
 * has no f32->f16 conversion; this one is written from the IEEE definition. */
uint16_t vko_f32_to_f16(float f) {
  union { float f; uint32_t u; } in;
  in.f = f;
  const uint32_t x = in.u;
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t mant = x & 0x7FFFFFu;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
  const int e = (int)exp - 127; /* unbiased */
  if (e > 15) return (uint16_t)(sign | 0x7C00u);
  if (e >= -14) {
    /* normal half: 10 mantissa bits, round the dropped 13 bits */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carries into the exponent correctly */
    return (uint16_t)(sign | h);
  }
  if (e < -25) return sign; /* below half the smallest subnormal */
  /* subnormal half: value = m * 2^-24 with m = full significand >> shift */
  mant |= 0x800000u;
  const int shift = -e - 1; /* 14 .. 24 */
  uint32_t h = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static float load_in(const void* p, int dtype, int64_t i) {
  return dtype == VKO_F16 ? vko_f16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

/* ------------------------------------------------------------------------- */
/* (1) reference layout restatements                                          */
/* ------------------------------------------------------------------------- */

/* kv_update (kernels.metal:619-645): k_cache[((blk*bs + tok)*Hkv + h)*D + d] = k_in[h*D + d],
 * blk = slot_mapping[slot_id*max_pages + pos/bs], tok = pos % bs. */
void vko_ref_kv_update(float* k_cache, float* v_cache, const float* k_in, const float* v_in, uint32_t slot_id,
                       const uint32_t* slot_mapping, uint32_t max_pages, uint32_t block_size, uint32_t n_head,
                       uint32_t head_dim, uint32_t pos) {
  const uint32_t blk = slot_mapping[slot_id * max_pages + pos / block_size];
  const uint32_t tok = pos % block_size;
  for (uint32_t h = 0; h < n_head; ++h)
    for (uint32_t d = 0; d < head_dim; ++d) {
      const uint64_t off = ((uint64_t)blk * block_size * n_head * head_dim) + (uint64_t)tok * n_head * head_dim +
                           (uint64_t)h * head_dim + d;
      k_cache[off] = k_in[h * head_dim + d];
      v_cache[off] = v_in[h * head_dim + d];
    }
}

/* kv_update_int8 (kernels.metal:753-802): per (token, head) amax; scale = amax/127;
 * inv = amax > 0 ? 127/amax : 0; code = (char)(x * inv) (truncation toward zero);
 * the fp32 scale sits in the 4 bytes after the D codes of the head row. */
void vko_ref_kv_update_int8(int8_t* k_cache, int8_t* v_cache, const float* k_in, const float* v_in,
                            uint32_t slot_id, const uint32_t* slot_mapping, uint32_t max_pages,
                            uint32_t block_size, uint32_t n_head, uint32_t head_dim, uint32_t pos) {
  const uint32_t blk = slot_mapping[slot_id * max_pages + pos / block_size];
  const uint32_t tok = pos % block_size;
  const uint32_t hb = head_dim + 4;
  for (uint32_t h = 0; h < n_head; ++h) {
    const uint64_t off = ((uint64_t)blk * block_size * n_head * hb) + (uint64_t)tok * n_head * hb + (uint64_t)h * hb;
    int8_t* kd = k_cache + off;
    int8_t* vd = v_cache + off;
    const float* ks = k_in + h * head_dim;
    const float* vs = v_in + h * head_dim;
    float kmax = 0.0f, vmax = 0.0f;
    for (uint32_t d = 0; d < head_dim; ++d) {
      kmax = fmaxf(kmax, fabsf(ks[d]));
      vmax = fmaxf(vmax, fabsf(vs[d]));
    }
    const float kscale = kmax / 127.0f, vscale = vmax / 127.0f;
    const float kinv = kmax > 0.0f ? 127.0f / kmax : 0.0f;
    const float vinv = vmax > 0.0f ? 127.0f / vmax : 0.0f;
    for (uint32_t d = 0; d < head_dim; ++d) {
      kd[d] = (int8_t)(int)(ks[d] * kinv);
      vd[d] = (int8_t)(int)(vs[d] * vinv);
    }
    memcpy(kd + head_dim, &kscale, 4);
    memcpy(vd + head_dim, &vscale, 4);
  }
}

/* paged_attention_flash / paged_attention_flash_int8 (kernels.metal:440-501,
 * 672-732): one query head at a time, kvh = h / (H / Hkv), online softmax over
 * t = 0..pos with (m, l, acc) and a final acc / l. int8: k = (float)code * scale. */
void vko_ref_paged_attention_flash(float* out, const float* q, const void* k_cache, const void* v_cache,
                                   int int8, uint32_t head_dim, uint32_t pos, uint32_t slot_id,
                                   const uint32_t* slot_mapping, uint32_t max_pages, uint32_t block_size,
                                   uint32_t n_head_kv, uint32_t n_head) {
  const float inv_sqrt = 1.0f / sqrtf((float)head_dim);
  float* acc = (float*)malloc(sizeof(float) * head_dim);
  for (uint32_t h = 0; h < n_head; ++h) {
    const uint32_t kvh = h / (n_head / n_head_kv);
    const float* hq = q + h * head_dim;
    float m = -INFINITY, l = 0.0f;
    for (uint32_t d = 0; d < head_dim; ++d) acc[d] = 0.0f;
    for (uint32_t t = 0; t <= pos; ++t) {
      const uint32_t blk = slot_mapping[slot_id * max_pages + t / block_size];
      const uint32_t tok = t % block_size;
      float score = 0.0f, vscale = 1.0f, kscale = 1.0f;
      const float *kf = NULL, *vf = NULL;
      const int8_t *kc = NULL, *vc = NULL;
      if (int8) {
        const uint32_t hb = head_dim + 4;
        const uint64_t off = (uint64_t)blk * block_size * n_head_kv * hb + (uint64_t)tok * n_head_kv * hb + (uint64_t)kvh * hb;
        kc = (const int8_t*)k_cache + off;
        vc = (const int8_t*)v_cache + off;
        memcpy(&kscale, kc + head_dim, 4);
        memcpy(&vscale, vc + head_dim, 4);
        for (uint32_t d = 0; d < head_dim; ++d) score += hq[d] * ((float)kc[d] * kscale);
      } else {
        const uint64_t off = (uint64_t)blk * block_size * n_head_kv * head_dim + (uint64_t)tok * n_head_kv * head_dim +
                             (uint64_t)kvh * head_dim;
        kf = (const float*)k_cache + off;
        vf = (const float*)v_cache + off;
        for (uint32_t d = 0; d < head_dim; ++d) score += hq[d] * kf[d];
      }
      score *= inv_sqrt;
      const float m_old = m;
      m = fmaxf(m_old, score);
      const float e = expf(score - m);
      const float f = expf(m_old - m);
      l = l * f + e;
      for (uint32_t d = 0; d < head_dim; ++d) {
        const float v = int8 ? (float)vc[d] * vscale : vf[d];
        acc[d] = acc[d] * f + e * v;
      }
    }
    for (uint32_t d = 0; d < head_dim; ++d) out[h * head_dim + d] = acc[d] / l;
  }
  free(acc);
}

/* llama_cpu.rs:22-50 + 251-284 on its contiguous cache k[t*Hkv*D + kvh*D + d]:
 * kv_head = h*Hkv/H, scores = dot/sqrt(D), two-pass softmax (135-146), out += s*v. */
void vko_ref_cpu_attention(float* out, const float* q, const float* k, const float* v, uint32_t n_seq,
                           uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim) {
  const uint32_t stride = n_head_kv * head_dim;
  float* scores = (float*)malloc(sizeof(float) * (n_seq ? n_seq : 1));
  for (uint32_t h = 0; h < n_head; ++h) {
    const uint32_t kvh = h * n_head_kv / n_head;
    const float* qh = q + h * head_dim;
    for (uint32_t t = 0; t < n_seq; ++t) {
      const float* kt = k + t * stride + kvh * head_dim;
      float dot = 0.0f;
      for (uint32_t d = 0; d < head_dim; ++d) dot += qh[d] * kt[d];
      scores[t] = dot / sqrtf((float)head_dim);
    }
    float mx = -INFINITY, sum = 0.0f;
    for (uint32_t t = 0; t < n_seq; ++t) mx = fmaxf(mx, scores[t]);
    for (uint32_t t = 0; t < n_seq; ++t) {
      scores[t] = expf(scores[t] - mx);
      sum += scores[t];
    }
    const float inv = 1.0f / sum;
    for (uint32_t t = 0; t < n_seq; ++t) scores[t] *= inv;
    float* oh = out + h * head_dim;
    for (uint32_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
    for (uint32_t t = 0; t < n_seq; ++t) {
      const float* vt = v + t * stride + kvh * head_dim;
      for (uint32_t d = 0; d < head_dim; ++d) oh[d] += scores[t] * vt[d];
    }
  }
  free(scores);
}

/* ------------------------------------------------------------------------- */
/* (2) build layout                                                           */
/* ------------------------------------------------------------------------- */

typedef struct vko_layer {
  int32_t n_blocks, n_kv_heads, block_size, head_dim, kv_type;
  uint8_t* k;  /* codes */
  uint8_t* v;
  uint8_t* ks; /* scales (I8 types) */
  uint8_t* vs;
} vko_layer;

static int esz_of(int kv) { return kv == VKO_F32 ? 4 : kv == VKO_F16 ? 2 : 1; }

/* byte offset of element (block, head, token, dim) inside K or V codes */
static uint64_t elem_off(const vko_layer* L, int is_v, int64_t blk, int h, int tok, int d) {
  const int esz = esz_of(L->kv_type);
  const uint64_t tile = (uint64_t)L->block_size * L->head_dim * esz;
  const uint64_t base = ((uint64_t)blk * L->n_kv_heads + h) * tile;
  /* int8 K: [h][tok][D/32][16], h = (d/16) % 2 (two 16-byte pieces per 32 dims) */
  if (!is_v && esz == 1)
    return base + (uint64_t)(((d >> 4) & 1) * (tile / 2) + (tok * (L->head_dim / 32) + (d >> 5)) * 16 + (d & 15));
  if (!is_v) return base + ((uint64_t)tok * L->head_dim + d) * esz;
  return base + ((uint64_t)((tok >> 1) * L->head_dim + d) * 2 + (tok & 1)) * esz;
}

/* dequantized element as the reference's kernels read it (fp32) */
static float load_elem(const vko_layer* L, int is_v, int64_t blk, int h, int tok, int d) {
  const uint8_t* base = is_v ? L->v : L->k;
  const uint64_t off = elem_off(L, is_v, blk, h, tok, d);
  switch (L->kv_type) {
    case VKO_F32: { float f; memcpy(&f, base + off, 4); return f; }
    case VKO_F16: { uint16_t b; memcpy(&b, base + off, 2); return vko_f16_to_f32(b); }
    case VKO_I8_REF: {
      float s;
      memcpy(&s, (is_v ? L->vs : L->ks) + (((uint64_t)blk * L->n_kv_heads + h) * L->block_size + tok) * 4, 4);
      return (float)(int8_t)base[off] * s;
    }
    default: {
      uint16_t sb;
      memcpy(&sb, (is_v ? L->vs : L->ks) + ((uint64_t)blk * L->n_kv_heads + h) * 2, 2);
      return (float)(int8_t)base[off] * vko_f16_to_f32(sb);
    }
  }
}

/* byte offset of element (blk, head, tok, d) in the K (is_v = 0) or V codes */
uint64_t vko_elem_offset(const vko_layer* L, int is_v, int64_t blk, int h, int tok, int d) {
  return elem_off(L, is_v, blk, h, tok, d);
}

float vko_load_elem(const vko_layer* L, int is_v, int64_t blk, int h, int tok, int d) {
  return load_elem(L, is_v, blk, h, tok, d);
}

static int clamp127(float r) { return r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r); }

/* One (token, head) of VK_KV_I8_BLK: per-(block, head) fp16 scale, RNE codes:
 *   s_old = offset == 0 ? 0 : stored scale
 *   s_new = max(s_old, fp16(amax / 127))
 *   if s_new > s_old: existing codes c' = clamp(rne((c * s_old) / s_new))
 *   new codes c = s_new > 0 ? clamp(rne(x / s_new)) : 0                      */
static void quant_blk_one(vko_layer* L, int is_v, int64_t blk, int h, int off, const float* x) {
  uint8_t* codes = is_v ? L->v : L->k;
  uint16_t* sp = (uint16_t*)((is_v ? L->vs : L->ks) + ((uint64_t)blk * L->n_kv_heads + h) * 2);
  const int D = L->head_dim;
  float amax = 0.0f;
  for (int d = 0; d < D; ++d) amax = fmaxf(amax, fabsf(x[d]));
  const float s_old = off == 0 ? 0.0f : vko_f16_to_f32(*sp);
  const uint16_t cand = vko_f32_to_f16(amax / 127.0f);
  uint16_t s_bits = off == 0 ? 0 : *sp;
  float s_new = s_old;
  if (vko_f16_to_f32(cand) > s_old) {
    s_new = vko_f16_to_f32(cand);
    s_bits = cand;
  }
  if (off > 0 && s_new > s_old) {
    for (int u = 0; u < off; ++u)
      for (int d = 0; d < D; ++d) {
        uint8_t* cp = codes + elem_off(L, is_v, blk, h, u, d);
        const float r = ((float)(int8_t)*cp * s_old) / s_new;
        *cp = (uint8_t)(int8_t)clamp127(rintf(r));
      }
  }
  for (int d = 0; d < D; ++d) {
    const int c = s_new > 0.0f ? clamp127(rintf(x[d] / s_new)) : 0;
    codes[elem_off(L, is_v, blk, h, off, d)] = (uint8_t)(int8_t)c;
  }
  *sp = s_bits;
}

/* VK_KV_I8_REF on the build layout: kernels.metal:783-801 operation order. */
static void quant_ref_one(vko_layer* L, int is_v, int64_t blk, int h, int off, const float* x) {
  uint8_t* codes = is_v ? L->v : L->k;
  const int D = L->head_dim;
  float amax = 0.0f;
  for (int d = 0; d < D; ++d) amax = fmaxf(amax, fabsf(x[d]));
  const float scale = amax / 127.0f;
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  for (int d = 0; d < D; ++d) codes[elem_off(L, is_v, blk, h, off, d)] = (uint8_t)(int8_t)(int)(x[d] * inv);
  memcpy((is_v ? L->vs : L->ks) + (((uint64_t)blk * L->n_kv_heads + h) * L->block_size + off) * 4, &scale, 4);
}

/* Append n_tok tokens (k, v: [n_tok][Hkv][D] of in_dtype) at flat slots, in
 * index order. A slot that is negative, or at or past n_blocks * block_size, is
 * padding and skipped (the reference's kv_update writes wherever the looked-up
 * block points, kernels.metal:637; the build's append treats both as padding). */
int vko_append(vko_layer* L, const void* k, const void* v, int in_dtype, const int64_t* slot_mapping, int n_tok) {
  const int D = L->head_dim, Hkv = L->n_kv_heads, bs = L->block_size;
  float* x = (float*)malloc(sizeof(float) * D);
  for (int n = 0; n < n_tok; ++n) {
    const int64_t slot = slot_mapping[n];
    if (slot < 0 || slot >= (int64_t)L->n_blocks * bs) continue;
    const int64_t blk = slot / bs;
    const int off = (int)(slot % bs);
    for (int is_v = 0; is_v < 2; ++is_v) {
      const void* src = is_v ? v : k;
      for (int h = 0; h < Hkv; ++h) {
        for (int d = 0; d < D; ++d) x[d] = load_in(src, in_dtype, ((int64_t)n * Hkv + h) * D + d);
        if (L->kv_type == VKO_I8_BLK) {
          quant_blk_one(L, is_v, blk, h, off, x);
        } else if (L->kv_type == VKO_I8_REF) {
          quant_ref_one(L, is_v, blk, h, off, x);
        } else {
          uint8_t* codes = is_v ? L->v : L->k;
          for (int d = 0; d < D; ++d) {
            const uint64_t o = elem_off(L, is_v, blk, h, off, d);
            if (L->kv_type == VKO_F16) {
              uint16_t b = in_dtype == VKO_F16 ? ((const uint16_t*)src)[((int64_t)n * Hkv + h) * D + d]
                                               : vko_f32_to_f16(x[d]);
              memcpy(codes + o, &b, 2);
            } else {
              memcpy(codes + o, &x[d], 4);
            }
          }
        }
      }
    }
  }
  free(x);
  return 0;
}

/* Paged decode attention (llama_cpu.rs:251-284 math on the paged layout):
 * for each sequence s and query head h, kvh = h / (H / Hkv); context
 * t = 0..ctx_lens[s]-1 read through block_tables[s*bt_stride + t/bs];
 * scores = (q . k_t) * scale; two-pass softmax; out = sum_t p_t v_t. fp32. */
void vko_paged_decode(const vko_layer* L, const void* q, int q_dtype, float* out, const int32_t* bt, int bt_stride,
                      const int32_t* ctx_lens, int S, int H, float scale) {
  const int D = L->head_dim, Hkv = L->n_kv_heads, bs = L->block_size;
  const int G = H / Hkv;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < H; ++h) {
      const int n = ctx_lens[s];
      float* o = out + ((int64_t)s * H + h) * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0f;
      if (n <= 0) continue;
      const int kvh = h / G;
      float* qh = (float*)malloc(sizeof(float) * D);
      float* sc = (float*)malloc(sizeof(float) * n);
      for (int d = 0; d < D; ++d) qh[d] = load_in(q, q_dtype, ((int64_t)s * H + h) * D + d);
      float mx = -INFINITY;
      for (int t = 0; t < n; ++t) {
        const int64_t blk = bt[(int64_t)s * bt_stride + t / bs];
        float dot = 0.0f;
        for (int d = 0; d < D; ++d) dot += qh[d] * load_elem(L, 0, blk, kvh, t % bs, d);
        sc[t] = dot * scale;
        mx = fmaxf(mx, sc[t]);
      }
      float sum = 0.0f;
      for (int t = 0; t < n; ++t) {
        sc[t] = expf(sc[t] - mx);
        sum += sc[t];
      }
      const float inv = 1.0f / sum;
      for (int t = 0; t < n; ++t) sc[t] *= inv;
      for (int t = 0; t < n; ++t) {
        const int64_t blk = bt[(int64_t)s * bt_stride + t / bs];
        for (int d = 0; d < D; ++d) o[d] += sc[t] * load_elem(L, 1, blk, kvh, t % bs, d);
      }
      free(qh);
      free(sc);
    }
}

/* Same in fp64 on the same dequantized fp32 values: the brute-force check. */
void vko_paged_decode_f64(const vko_layer* L, const void* q, int q_dtype, double* out, const int32_t* bt,
                          int bt_stride, const int32_t* ctx_lens, int S, int H, double scale) {
  const int D = L->head_dim, Hkv = L->n_kv_heads, bs = L->block_size;
  const int G = H / Hkv;
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < H; ++h) {
      const int n = ctx_lens[s];
      double* o = out + ((int64_t)s * H + h) * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      if (n <= 0) continue;
      const int kvh = h / G;
      double* sc = (double*)malloc(sizeof(double) * n);
      double mx = -INFINITY;
      for (int t = 0; t < n; ++t) {
        const int64_t blk = bt[(int64_t)s * bt_stride + t / bs];
        double dot = 0.0;
        for (int d = 0; d < D; ++d)
          dot += (double)load_in(q, q_dtype, ((int64_t)s * H + h) * D + d) * (double)load_elem(L, 0, blk, kvh, t % bs, d);
        sc[t] = dot * scale;
        if (sc[t] > mx) mx = sc[t];
      }
      double sum = 0.0;
      for (int t = 0; t < n; ++t) { sc[t] = exp(sc[t] - mx); sum += sc[t]; }
      for (int t = 0; t < n; ++t) {
        const int64_t blk = bt[(int64_t)s * bt_stride + t / bs];
        for (int d = 0; d < D; ++d) o[d] += sc[t] / sum * (double)load_elem(L, 1, blk, kvh, t % bs, d);
      }
      free(sc);
    }
}

/* Tree verify: node i of sequence s attends to context tokens 0..ctx-1 and to
 * tree nodes j with bit j of mask[s*N + i] set; node j's K/V sit at position
 * ctx + j. q/out [S][N][H][D]. fp32, two-pass softmax as above. */
void vko_tree_verify(const vko_layer* L, const void* q, int q_dtype, float* out, const int32_t* bt, int bt_stride,
                     const int32_t* ctx_lens, const uint32_t* mask, int S, int N, int H, float scale) {
  const int D = L->head_dim, Hkv = L->n_kv_heads, bs = L->block_size;
  const int G = H / Hkv;
#pragma omp parallel for schedule(dynamic) collapse(3)
  for (int s = 0; s < S; ++s)
    for (int i = 0; i < N; ++i)
      for (int h = 0; h < H; ++h) {
        const int ctx = ctx_lens[s];
        const int kvh = h / G;
        const int64_t qrow = (((int64_t)s * N + i) * H + h) * D;
        float* o = out + qrow;
        const int n_all = ctx + N;
        float* sc = (float*)malloc(sizeof(float) * n_all);
        int* pos = (int*)malloc(sizeof(int) * n_all);
        int n = 0;
        for (int t = 0; t < ctx; ++t) pos[n++] = t;
        for (int j = 0; j < N; ++j)
          if ((mask[(int64_t)s * N + i] >> j) & 1u) pos[n++] = ctx + j;
        for (int d = 0; d < D; ++d) o[d] = 0.0f;
        float mx = -INFINITY;
        for (int k = 0; k < n; ++k) {
          const int t = pos[k];
          const int64_t blk = bt[(int64_t)s * bt_stride + t / bs];
          float dot = 0.0f;
          for (int d = 0; d < D; ++d) dot += load_in(q, q_dtype, qrow + d) * load_elem(L, 0, blk, kvh, t % bs, d);
          sc[k] = dot * scale;
          mx = fmaxf(mx, sc[k]);
        }
        float sum = 0.0f;
        for (int k = 0; k < n; ++k) { sc[k] = expf(sc[k] - mx); sum += sc[k]; }
        if (n > 0) {
          const float inv = 1.0f / sum;
          for (int k = 0; k < n; ++k) {
            const int t = pos[k];
            const int64_t blk = bt[(int64_t)s * bt_stride + t / bs];
            for (int d = 0; d < D; ++d) o[d] += sc[k] * inv * load_elem(L, 1, blk, kvh, t % bs, d);
          }
        }
        free(sc);
        free(pos);
      }
}

/* Copy-on-write: for each (src, dst) pair copy codes and scales of every head. */
void vko_copy_blocks(vko_layer* L, const int32_t* pairs, int n_pairs) {
  const int esz = esz_of(L->kv_type);
  const uint64_t cb = (uint64_t)L->n_kv_heads * L->block_size * L->head_dim * esz;
  const uint64_t sb = L->kv_type == VKO_I8_BLK ? (uint64_t)L->n_kv_heads * 2
                      : L->kv_type == VKO_I8_REF ? (uint64_t)L->n_kv_heads * L->block_size * 4 : 0;
  for (int i = 0; i < n_pairs; ++i) {
    const int64_t s = pairs[2 * i], d = pairs[2 * i + 1];
    memcpy(L->k + d * cb, L->k + s * cb, cb);
    memcpy(L->v + d * cb, L->v + s * cb, cb);
    if (sb) {
      memcpy(L->ks + d * sb, L->ks + s * sb, sb);
      memcpy(L->vs + d * sb, L->vs + s * sb, sb);
    }
  }
}

/* Accepted-path commit of a draft tree, one sequence and one layer (defined
 * here; the reference appends no tree KV). Node accept[d] sits at position
 * ctx + accept[d] and moves to ctx + d. Returns 1 (pool untouched) for a row
 * that is not strictly increasing with d <= accept[d] < 32, n_accept > 32, or
 * positions outside the table row / pool; 0 otherwise. Every moved token is
 * read before anything is written. F32 / F16 / I8_REF rows (with per-token
 * scales) move unchanged; I8_BLK tokens are dequantized (code x block scale)
 * and appended in order with vko_append's rule. */
int vko_tree_commit(vko_layer* L, const int32_t* bt, int bt_stride, int ctx, const int32_t* accept, int n_accept) {
  const int D = L->head_dim, Hkv = L->n_kv_heads, bs = L->block_size;
  if (ctx < 0 || n_accept <= 0) return n_accept == 0 ? 0 : 1;
  if (n_accept > 32) return 1;
  for (int d = 0; d < n_accept; ++d)
    if (accept[d] < d || accept[d] >= 32 || (d > 0 && accept[d] <= accept[d - 1])) return 1;
  int d0 = 0;
  while (d0 < n_accept && accept[d0] == d0) ++d0;
  if (d0 == n_accept) return 0;
  const int last = ctx + accept[n_accept - 1];
  if ((int64_t)last >= (int64_t)bt_stride * bs) return 1;
  for (int b = (ctx + d0) / bs; b <= last / bs; ++b)
    if (bt[b] < 0 || bt[b] >= L->n_blocks) return 1;
  const int n = n_accept - d0;
  if (L->kv_type == VKO_I8_BLK) {
    float* kx = (float*)malloc(sizeof(float) * (size_t)n * Hkv * D);
    float* vx = (float*)malloc(sizeof(float) * (size_t)n * Hkv * D);
    int64_t* slots = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
    for (int i = 0; i < n; ++i) {
      const int q = ctx + accept[d0 + i], p = ctx + d0 + i;
      for (int h = 0; h < Hkv; ++h)
        for (int d = 0; d < D; ++d) {
          kx[((size_t)i * Hkv + h) * D + d] = load_elem(L, 0, bt[q / bs], h, q % bs, d);
          vx[((size_t)i * Hkv + h) * D + d] = load_elem(L, 1, bt[q / bs], h, q % bs, d);
        }
      slots[i] = (int64_t)bt[p / bs] * bs + p % bs;
    }
    vko_append(L, kx, vx, VKO_F32, slots, n);
    free(kx);
    free(vx);
    free(slots);
    return 0;
  }
  const int esz = esz_of(L->kv_type);
  const int ref = L->kv_type == VKO_I8_REF;
  uint8_t* row = (uint8_t*)malloc((size_t)n * 2 * Hkv * D * esz);
  float* sc = (float*)malloc(sizeof(float) * (size_t)n * 2 * Hkv);
  for (int pass = 0; pass < 2; ++pass) /* 0: read every source, 1: write every destination */
    for (int i = 0; i < n; ++i) {
      const int pos = ctx + (pass == 0 ? accept[d0 + i] : d0 + i);
      const int64_t blk = bt[pos / bs];
      const int o = pos % bs;
      for (int is_v = 0; is_v < 2; ++is_v) {
        uint8_t* codes = is_v ? L->v : L->k;
        for (int h = 0; h < Hkv; ++h) {
          uint8_t* r = row + (((size_t)i * 2 + is_v) * Hkv + h) * D * esz;
          for (int d = 0; d < D; ++d) {
            uint8_t* e = codes + elem_off(L, is_v, blk, h, o, d);
            if (pass == 0) memcpy(r + (size_t)d * esz, e, esz); else memcpy(e, r + (size_t)d * esz, esz);
          }
          if (ref) {
            uint8_t* s = (is_v ? L->vs : L->ks) + (((uint64_t)blk * Hkv + h) * bs + o) * 4;
            float* t = &sc[((size_t)i * 2 + is_v) * Hkv + h];
            if (pass == 0) memcpy(t, s, 4); else memcpy(s, t, 4);
          }
        }
      }
    }
  free(row);
  free(sc);
  return 0;
}

/* ---- RoPE -------------------------------------------------------------- */

/* apply_rope of the CPU model (llama_cpu.rs:113-131) on one head row:
 * half-split pairs (i, i + D/2), angle pos / freq_base^(2i/D) in fp32. */
void vko_ref_rope_cpu(float* x, int head_dim, int pos, float freq_base) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float theta = (float)pos / powf(freq_base, 2.0f * (float)i / (float)head_dim);
    const float s = sinf(theta), c = cosf(theta);
    const float x0 = x[i], x1 = x[i + half];
    x[i] = x0 * c - x1 * s;
    x[i + half] = x0 * s + x1 * c;
  }
}

/* The Metal rope kernel (kernels.metal:103-131) on one head row: interleaved
 * pairs (2j, 2j+1), angle pos * freq_base^(-(2j)/D) in fp32. */
void vko_ref_rope_metal(float* x, int head_dim, int pos, float freq_base) {
  for (int i = 0; i < head_dim; i += 2) {
    const float theta = powf(freq_base, -(float)i / (float)head_dim);
    const float m = (float)pos * theta;
    const float c = cosf(m), s = sinf(m);
    const float x0 = x[i], x1 = x[i + 1];
    x[i] = x0 * c - x1 * s;
    x[i + 1] = x0 * s + x1 * c;
  }
}

/* cos / sin table [n_pos][D/2][2] of the angle p * freq_base^(-2i/D), in double
 * precision, rounded to fp32 once (what vk_rope_table computes). */
void vko_rope_table(float* out, int n_pos, int head_dim, float freq_base) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const double inv = pow((double)freq_base, -2.0 * (double)i / (double)head_dim);
    for (int p = 0; p < n_pos; ++p) {
      const double a = (double)p * inv;
      out[((int64_t)p * half + i) * 2] = (float)cos(a);
      out[((int64_t)p * half + i) * 2 + 1] = (float)sin(a);
    }
  }
}

/* Rotate one head row in place with the table: style 1 = interleaved pairs
 * (2i, 2i+1), style 2 = half-split pairs (i, i + D/2); y0 = x0 c - x1 s,
 * y1 = x0 s + x1 c in fp32, no contraction (this file builds with
 * -ffp-contract=off). */
void vko_rope_apply(float* x, int head_dim, int pos, int style, const float* table) {
  const int half = head_dim / 2;
  const float* row = table + (int64_t)pos * head_dim;
  for (int i = 0; i < half; ++i) {
    const float c = row[2 * i], s = row[2 * i + 1];
    const int a = style == 1 ? 2 * i : i, b = style == 1 ? 2 * i + 1 : i + half;
    const float x0 = x[a], x1 = x[b];
    x[a] = x0 * c - x1 * s;
    x[b] = x0 * s + x1 * c;
  }
}

/* ---- NIXL wire format (nixl.rs:24-61) ------------------------------------ */

/* serialize_block (nixl.rs:36-43): block_id.to_le_bytes(), (token_len as
 * u32).to_le_bytes(), (payload.len() as u32).to_le_bytes(), payload. Returns
 * the record length 16 + byte_len. */
uint64_t vko_nixl_serialize(uint64_t block_id, uint32_t token_len, const uint8_t* payload, uint32_t byte_len,
                            uint8_t* out) {
  for (int i = 0; i < 8; ++i) out[i] = (uint8_t)(block_id >> (8 * i));
  for (int i = 0; i < 4; ++i) out[8 + i] = (uint8_t)(token_len >> (8 * i));
  for (int i = 0; i < 4; ++i) out[12 + i] = (uint8_t)(byte_len >> (8 * i));
  if (byte_len) memcpy(out + 16, payload, byte_len);
  return 16u + (uint64_t)byte_len;
}

/* deserialize_block (nixl.rs:49-61): None (0) when the buffer is shorter than
 * the 16-byte header or than header + byte_len; else 1 with the handle and the
 * payload's length (the payload starts at buf + 16). */
int vko_nixl_deserialize(const uint8_t* buf, uint64_t len, uint64_t* block_id, uint32_t* token_len,
                         uint32_t* byte_len) {
  if (len < 16) return 0;
  uint64_t id = 0;
  uint32_t tl = 0, bl = 0;
  for (int i = 0; i < 8; ++i) id |= (uint64_t)buf[i] << (8 * i);
  for (int i = 0; i < 4; ++i) tl |= (uint32_t)buf[8 + i] << (8 * i);
  for (int i = 0; i < 4; ++i) bl |= (uint32_t)buf[12 + i] << (8 * i);
  if (len < 16u + (uint64_t)bl) return 0;
  *block_id = id;
  *token_len = tl;
  *byte_len = bl;
  return 1;
}

static uint64_t scale_bytes_per_head(const vko_layer* L) {
  return L->kv_type == VKO_I8_BLK ? 2u : L->kv_type == VKO_I8_REF ? 4u * (uint64_t)L->block_size : 0u;
}

/* Payload of one KV-cache handle over n_layers layers (velokv.h): tiles of
 * every (page, layer) -- K codes of the page's heads, then V codes -- then the
 * scales of every (page, layer), K then V. */
uint64_t vko_nixl_payload_bytes(const vko_layer* L, int n_layers, uint32_t token_len) {
  const uint64_t pages = ((uint64_t)token_len + L->block_size - 1) / L->block_size;
  const uint64_t cb = (uint64_t)L->n_kv_heads * L->block_size * L->head_dim * esz_of(L->kv_type);
  const uint64_t sb = (uint64_t)L->n_kv_heads * scale_bytes_per_head(L);
  return pages * (uint64_t)n_layers * 2 * (cb + sb);
}

/* pool pages -> payload (dir 0) or payload -> pool pages (dir 1) */
void vko_nixl_move(vko_layer* Ls, int n_layers, const int32_t* pages, int n_pages, uint8_t* payload, int dir) {
  const vko_layer* L0 = &Ls[0];
  const uint64_t cb = (uint64_t)L0->n_kv_heads * L0->block_size * L0->head_dim * esz_of(L0->kv_type);
  const uint64_t sb = (uint64_t)L0->n_kv_heads * scale_bytes_per_head(L0);
  uint8_t* scales = payload + (uint64_t)n_pages * n_layers * 2 * cb;
  for (int i = 0; i < n_pages; ++i)
    for (int l = 0; l < n_layers; ++l) {
      vko_layer* L = &Ls[l];
      const uint64_t r = (uint64_t)i * n_layers + l;
      const uint64_t pg = (uint64_t)pages[i];
      uint8_t* parts[4] = {L->k + pg * cb, L->v + pg * cb, sb ? L->ks + pg * sb : 0, sb ? L->vs + pg * sb : 0};
      uint8_t* wire[4] = {payload + r * 2 * cb, payload + r * 2 * cb + cb, scales + r * 2 * sb, scales + r * 2 * sb + sb};
      const uint64_t len[4] = {cb, cb, sb, sb};
      for (int k = 0; k < 4; ++k) {
        if (!len[k]) continue;
        if (dir == 0) memcpy(wire[k], parts[k], len[k]); else memcpy(parts[k], wire[k], len[k]);
      }
    }
}

/* Layout translation: build layout -> reference layout for the I8_REF and F32
 * types ([blk][tok][head][D] fp32; [blk][tok][head][D codes + fp32 scale]). */
void vko_to_reference_layout(const vko_layer* L, int is_v, uint8_t* dst) {
  const int D = L->head_dim, Hkv = L->n_kv_heads, bs = L->block_size;
  const uint8_t* src = is_v ? L->v : L->k;
  for (int64_t b = 0; b < L->n_blocks; ++b)
    for (int t = 0; t < bs; ++t)
      for (int h = 0; h < Hkv; ++h) {
        if (L->kv_type == VKO_F32) {
          float* row = (float*)dst + ((b * bs + t) * Hkv + h) * D;
          for (int d = 0; d < D; ++d) memcpy(&row[d], src + elem_off(L, is_v, b, h, t, d), 4);
        } else if (L->kv_type == VKO_I8_REF) {
          uint8_t* row = dst + ((b * bs + t) * Hkv + h) * (uint64_t)(D + 4);
          for (int d = 0; d < D; ++d) row[d] = src[elem_off(L, is_v, b, h, t, d)];
          memcpy(row + D, (is_v ? L->vs : L->ks) + ((b * Hkv + h) * bs + t) * 4, 4);
        }
      }
}

/* SplitMix64 (the public-domain mixer of Steele, Lea & Flood) and the
 * counter-based normal generator shared with vk_fill_normal_f16. */
uint64_t vko_splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Thread count of the OpenMP loops (the CPU baseline times 1 and all cores). */
#ifdef _OPENMP
#include <omp.h>
void vko_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int vko_get_threads(void) { return omp_get_max_threads(); }
#else
void vko_set_threads(int n) { (void)n; }
int vko_get_threads(void) { return 1; }
#endif
