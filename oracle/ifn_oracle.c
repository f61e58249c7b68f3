/*
 * CPU oracle for the KV-cache hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline),
 * never as the product path.  The product path is the HIP library under
 * infurnace_amd/ and fails loudly when that library is missing.
 *
 * The reference's own modules for this path are 0-byte placeholders
 * (src/infurnace/kernels/kv_store.py, kernels/paged_attention.py,
 * cache/block_pool.py), so this file restates the documented contract and
 * the contiguous semantics the reference executes today:
 *
 *   - pool layout    docs/architecture.md:225-232
 *                    kv_pool[layer, K_or_V, physical_page, page_offset, kv_head, head_dim]
 *   - slot mapping   docs/architecture.md:234-235
 *                    slot = block_table[seq][pos / page_size] * page_size + pos % page_size
 *   - store_kv       docs/architecture.md:245,249-253 (inactive rows skip stores);
 *                    contiguous precedent src/infurnace/executor/tinygrad/model.py:191-196
 *   - attention      src/infurnace/executor/tinygrad/model.py:196-200 (decode: read
 *                    positions [0, pos], upcast fp16 -> fp32, non-causal SDPA with GQA)
 *                    and model.py:116-132 (chunked prefill: key_pos <= query_pos mask,
 *                    query_pos = start_position + i).  The SDPA itself is tinygrad's
 *                    Tensor.scaled_dot_product_attention (third-party, unpinned per
 *                    reference pyproject.toml:11 / README.md:20-22): softmax(q k^T * scale
 *                    + mask) v with scale 1/sqrt(head_dim) and query head h reading kv
 *                    head h / (Hq / Hkv) under enable_gqa.
 *
 * Arithmetic: fp16 storage, fp32 accumulation in a fixed order (dims ascending,
 * keys ascending), expf from libm, one fp16 round-to-nearest-even at the end.
 * fp16 values are handled as uint16_t bit patterns so the byte path is exact.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_half_to_float / orc_float_to_half: exhaustively against numpy's IEEE
 *     binary16 conversion (all 65536 patterns; 2^20 random floats incl. ties).
 *   orc_slot_mapping: closed form against numpy integer arithmetic and against
 *     brute-force "walk the table" enumeration.
 *   orc_store_kv: numpy dense scatter; sentinel pages bit-identical; paged
 *     gather equals the contiguous cache written at the same positions.
 *   orc_paged_attention: torch.nn.functional.scaled_dot_product_attention
 *     (enable_gqa=True, CPU, float64) on the gathered K/V; float64 brute force;
 *     closed forms (one key -> V row; equal keys -> mean of V; one dominant
 *     logit -> its V row); invariance under physical page permutation; chunked
 *     prefill == unchunked prefill; decode == last row of causal prefill.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------- IEEE binary16 <-> binary32 ---------------- */

float orc_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: renormalise */
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13); /* inf / nan (payload kept) */
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof x);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or nan */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  /* 65520 = largest value that rounds to the finite max 65504 boundary */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  int32_t e = (int32_t)(ax >> 23) - 127;
  uint32_t man = ax & 0x7fffffu;
  if (e >= -14) { /* normal half */
    uint32_t hbits = ((uint32_t)(e + 15) << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (hbits & 1u))) hbits += 1u;
    return (uint16_t)(sign | hbits);
  }
  if (e < -25) return (uint16_t)sign; /* below half the smallest subnormal */
  /* subnormal half: value = m * 2^-24 with m < 1024 */
  man |= 0x800000u;                      /* implicit bit: value = man * 2^(e-23) */
  int shift = -e - 1;                    /* man >> (shift) gives units of 2^-24 ... */
  /* value / 2^-24 = man * 2^(e - 23 + 24) = man * 2^(e+1) = man >> (-e-1) */
  uint32_t q = man >> shift;
  uint32_t rem = man & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1u;
  return (uint16_t)(sign | q);
}

void orc_half_to_float_array(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_half_to_float(src[i]);
}

void orc_float_to_half_array(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_float_to_half(src[i]);
}

/* ---------------- slot mapping (docs/architecture.md:234-235) ---------------- */

/* slot_out[t] = block_tables[seq_idx[t]][positions[t] / bs] * bs + positions[t] % bs.
 * Returns 0, or -1 when a position lies beyond the table row (max_pages * bs). */
int orc_slot_mapping(const int32_t* block_tables, int32_t max_pages, const int32_t* seq_idx,
                     const int32_t* positions, int32_t num_tokens, int32_t block_size,
                     int32_t* slot_out) {
  for (int32_t t = 0; t < num_tokens; ++t) {
    int32_t pos = positions[t];
    if (pos < 0 || pos / block_size >= max_pages) return -1;
    int32_t page = block_tables[(int64_t)seq_idx[t] * max_pages + pos / block_size];
    slot_out[t] = page * block_size + pos % block_size;
  }
  return 0;
}

/* ---------------- store_kv (docs/architecture.md:245,249-253) ---------------- */

/* pool_layer: [2][num_pages][bs][Hkv][D] fp16 bits.  new_k/new_v: [T][Hkv][D].
 * Rows with active_mask[t]==0 (when a mask is given) or a slot outside
 * [0, num_pages*bs) write nothing. */
void orc_store_kv(uint16_t* pool_layer, int64_t num_pages, const int32_t* slot_mapping,
                  const uint8_t* active_mask, const uint16_t* new_k, const uint16_t* new_v,
                  int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim, int32_t block_size) {
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  const int64_t half_pool = num_pages * block_size * row;
  for (int32_t t = 0; t < num_tokens; ++t) {
    if (active_mask && !active_mask[t]) continue;
    int64_t slot = slot_mapping[t];
    if (slot < 0 || slot >= num_pages * block_size) continue;
    memcpy(pool_layer + slot * row, new_k + (int64_t)t * row, (size_t)row * 2);
    memcpy(pool_layer + half_pool + slot * row, new_v + (int64_t)t * row, (size_t)row * 2);
  }
}

/* ---------------- paged attention (model.py:116-132, 196-200) ---------------- */

/* B sequences, each with num_q query rows: q [B][num_q][Hq][D], out likewise.
 * Query row t of sequence b sits at absolute position seq_lens[b] - num_q + t and
 * attends to keys [0, that position] read through block_tables[b] (causal).
 * Decode is num_q == 1 (attend all seq_lens[b] keys, model.py:196-200);
 * chunked prefill is B == 1, num_q == T, start_position = seq_lens[0] - T
 * (model.py:128-132).  Inactive rows leave out untouched.
 * Returns 0, -1 on bad lengths, -2 on a page id outside the pool. */
int orc_paged_attention(uint16_t* out, const uint16_t* q, const uint16_t* pool_layer,
                        int64_t num_pages, const int32_t* block_tables, int32_t max_pages,
                        const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                        int32_t num_q, int32_t num_q_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t block_size, float scale) {
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  const int64_t half_pool = num_pages * block_size * row;
  const int32_t group = num_q_heads / num_kv_heads;
  float* scores = NULL;
  float* acc = (float*)malloc(sizeof(float) * (size_t)head_dim);
  float* qf = (float*)malloc(sizeof(float) * (size_t)head_dim);
  int rc = 0;
  for (int32_t b = 0; b < batch && rc == 0; ++b) {
    if (active_mask && !active_mask[b]) continue;
    int32_t len = seq_lens[b];
    if (len < num_q || (len + block_size - 1) / block_size > max_pages) { rc = -1; break; }
    for (int32_t p = 0; p < (len + block_size - 1) / block_size; ++p) {
      int32_t id = block_tables[(int64_t)b * max_pages + p];
      if (id < 0 || id >= num_pages) { rc = -2; break; }
    }
    if (rc) break;
    free(scores);
    scores = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    for (int32_t t = 0; t < num_q; ++t) {
      int32_t qpos = len - num_q + t;
      int32_t nkeys = qpos + 1;
      for (int32_t h = 0; h < num_q_heads; ++h) {
        int32_t kvh = h / group;
        const uint16_t* qrow = q + (((int64_t)b * num_q + t) * num_q_heads + h) * head_dim;
        for (int32_t d = 0; d < head_dim; ++d) qf[d] = orc_half_to_float(qrow[d]);
        float m = -INFINITY;
        for (int32_t j = 0; j < nkeys; ++j) {
          int64_t page = block_tables[(int64_t)b * max_pages + j / block_size];
          int64_t slot = page * block_size + j % block_size;
          const uint16_t* krow = pool_layer + slot * row + (int64_t)kvh * head_dim;
          float s = 0.f;
          for (int32_t d = 0; d < head_dim; ++d) s += qf[d] * orc_half_to_float(krow[d]);
          s *= scale;
          scores[j] = s;
          if (s > m) m = s;
        }
        float l = 0.f;
        for (int32_t j = 0; j < nkeys; ++j) {
          scores[j] = expf(scores[j] - m);
          l += scores[j];
        }
        for (int32_t d = 0; d < head_dim; ++d) acc[d] = 0.f;
        for (int32_t j = 0; j < nkeys; ++j) {
          int64_t page = block_tables[(int64_t)b * max_pages + j / block_size];
          int64_t slot = page * block_size + j % block_size;
          const uint16_t* vrow = pool_layer + half_pool + slot * row + (int64_t)kvh * head_dim;
          for (int32_t d = 0; d < head_dim; ++d) acc[d] += scores[j] * orc_half_to_float(vrow[d]);
        }
        uint16_t* orow = out + (((int64_t)b * num_q + t) * num_q_heads + h) * head_dim;
        for (int32_t d = 0; d < head_dim; ++d) orow[d] = orc_float_to_half(acc[d] / l);
      }
    }
  }
  free(scores);
  free(acc);
  free(qf);
  return rc;
}

/* ---------------- pre-append step: q/k RMSNorm + rotary, k/v cast + store ----------------
 *
 * Follows src/infurnace/executor/tinygrad/model.py: _rms_norm (:11-13)
 * x * rsqrt(mean(x^2) + eps) then * weight; _apply_rope (:24-27) on the table of
 * _precompute_rope (:19-23), whose row is [cos(pos f_i) | sin(pos f_i)], i < D/2;
 * decode order :183-196 (q/k norm, rope, cast k/v to the cache dtype, store at
 * the slot).  v is only cast.  fp32 arithmetic, sums in ascending dim order,
 * one fp16 round at the end.  A token whose position lies outside
 * [0, max_pos) stores nothing and gets a zero q row; inactive tokens and
 * out-of-range slots store nothing.
 *
 * Pinned by (tests/test_oracle.py): a float64 numpy restatement of the two
 * formulas (within one fp16 rounding), the rotation invariants (each pair's
 * norm is preserved; position 0 is the identity; two rotations compose), and
 * v rows equal to the plain fp16 cast bit for bit.
 */
static void orc_norm_rope_row(const float* x, const float* w, const float* cs, int32_t D, float eps, float* y) {
  float ss = 0.f;
  for (int32_t i = 0; i < D; ++i) ss += x[i] * x[i];
  const float rs = 1.0f / sqrtf(ss / (float)D + eps);
  const int32_t half = D / 2;
  for (int32_t i = 0; i < half; ++i) {
    const float a = x[i] * rs * w[i];
    const float b = x[half + i] * rs * w[half + i];
    y[i] = a * cs[i] - b * cs[half + i];
    y[half + i] = b * cs[i] + a * cs[half + i];
  }
}

int orc_qk_norm_rope_append(uint16_t* q_out, uint16_t* pool_layer, int64_t num_pages, const float* q,
                            const float* k, const float* v, const float* q_norm_w, const float* k_norm_w,
                            const float* rope, int32_t max_pos, const int32_t* positions,
                            const int32_t* slot_mapping, const uint8_t* active, int32_t T, int32_t Hq,
                            int32_t Hkv, int32_t D, int32_t block_size, float eps) {
  if (D < 2 || D % 2 != 0 || Hq % Hkv != 0) return -1;
  float* y = (float*)malloc(sizeof(float) * (size_t)D);
  if (y == NULL) return -3;
  const int64_t num_slots = num_pages * block_size;
  for (int32_t t = 0; t < T; ++t) {
    const int32_t pos = positions[t];
    const int pos_ok = pos >= 0 && pos < max_pos;
    const float* cs = rope + (int64_t)(pos_ok ? pos : 0) * D;
    for (int32_t h = 0; h < Hq; ++h) {
      uint16_t* dst = q_out + ((int64_t)t * Hq + h) * D;
      orc_norm_rope_row(q + ((int64_t)t * Hq + h) * D, q_norm_w, cs, D, eps, y);
      for (int32_t i = 0; i < D; ++i) dst[i] = pos_ok ? orc_float_to_half(y[i]) : 0;
    }
    const int64_t slot = slot_mapping[t];
    if (!pos_ok || (active != NULL && active[t] == 0) || slot < 0 || slot >= num_slots) continue;
    for (int32_t h = 0; h < Hkv; ++h) {
      uint16_t* kd = pool_layer + (slot * Hkv + h) * D;
      uint16_t* vd = pool_layer + ((num_slots + slot) * Hkv + h) * D;
      orc_norm_rope_row(k + ((int64_t)t * Hkv + h) * D, k_norm_w, cs, D, eps, y);
      for (int32_t i = 0; i < D; ++i) kd[i] = orc_float_to_half(y[i]);
      for (int32_t i = 0; i < D; ++i) vd[i] = orc_float_to_half(v[((int64_t)t * Hkv + h) * D + i]);
    }
  }
  free(y);
  return 0;
}
