// Pre-append step and page utilities of the KV-cache path (gfx950).
//
// ifn_qk_norm_rope_append fuses what the reference does between the Q/K/V
// projections and the cache write, per token t and head:
//   q, k: per-head RMSNorm over head_dim (src/infurnace/executor/tinygrad/model.py:11-13,
//         applied at :183-184 / :109-110), then half-split rotary embedding with the
//         [position][cos | sin] table (:19-27, applied at :186-187);
//   k, v: cast to fp16 and stored at slot_mapping[t] (:190-196 decode, :134-137 prefill);
//   q:    written as fp16 for paged attention.
// Head dims 64 and 128 (16-byte aligned arrays) take qk_norm_rope_rows_kernel: 8 rotary pairs per
// lane, rows spread over whole wavefronts.  Other shapes take qk_norm_rope_append_kernel: one
// workgroup per token; a wavefront handles a (token, head) row at a time, lane l owning the
// rotary pairs (i, i + D/2) for i = l, l + 64, ..., so the RMS reduction is one wave sum and the
// rotation never leaves the lane.  The two give the same bits.
//
// ifn_zero_pages / ifn_copy_pages are the paged forms of clear_slot
// (src/infurnace/executor/tinygrad/buffers.py:67-81): zero, or copy, whole pages in every layer.
#include "ifn_common.hpp"

namespace ifn {

constexpr int kPrepWaves = 8;
constexpr int kPrepThreads = kPrepWaves * kWave;
constexpr int kPrepRows = 4;   // rows a wave loads before it computes (loads in flight together)

// One workgroup per token.  The token's rows (Hq q heads, then Hkv k heads, then Hkv v heads)
// go to the 8 waves in batches of kPrepRows; a wave loads its batch, then normalises,
// rotates and stores it.  The rotary row and both norm weights are loaded once per wave.
template <int kMaxPairs>  // rotary pairs per lane: ceil(head_dim / 128)
__global__ __launch_bounds__(kPrepThreads) void qk_norm_rope_append_kernel(
    f16* __restrict__ q_out, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w,
    const float* __restrict__ rope, int32_t max_pos, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ slot_mapping, const uint8_t* __restrict__ active, f16* __restrict__ pool,
    int64_t num_slots, int32_t hq, int32_t hkv, int32_t D, float eps) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int t = blockIdx.x;
  const int rows = hq + 2 * hkv;
  const int half = D / 2;
  const int pos = positions[t];
  const bool pos_ok = pos >= 0 && pos < max_pos;
  const int64_t slot = slot_mapping[t];
  const bool store = pos_ok && (active == nullptr || active[t] != 0) && slot >= 0 && slot < num_slots;
  const float* cs = rope + int64_t(pos_ok ? pos : 0) * D;
  float c[kMaxPairs], sn[kMaxPairs], wq1[kMaxPairs], wq2[kMaxPairs], wk1[kMaxPairs], wk2[kMaxPairs];
#pragma unroll
  for (int j = 0; j < kMaxPairs; ++j) {
    const int i = min(lane + kWave * j, half - 1);
    c[j] = cs[i];
    sn[j] = cs[half + i];
    wq1[j] = q_norm_w[i];
    wq2[j] = q_norm_w[half + i];
    wk1[j] = k_norm_w[i];
    wk2[j] = k_norm_w[half + i];
  }
  for (int r0 = wave * kPrepRows; r0 < rows; r0 += kPrepWaves * kPrepRows) {
    float x1[kPrepRows][kMaxPairs], x2[kPrepRows][kMaxPairs];
#pragma unroll
    for (int rr = 0; rr < kPrepRows; ++rr) {
      const int r = min(r0 + rr, rows - 1);  // a short last batch re-reads a valid row
      const float* src = r < hq ? q + (int64_t(t) * hq + r) * D
                                : (r < hq + hkv ? k + (int64_t(t) * hkv + (r - hq)) * D
                                                : v + (int64_t(t) * hkv + (r - hq - hkv)) * D);
#pragma unroll
      for (int j = 0; j < kMaxPairs; ++j) {
        const int i = min(lane + kWave * j, half - 1);
        x1[rr][j] = src[i];
        x2[rr][j] = src[half + i];
      }
    }
#pragma unroll
    for (int rr = 0; rr < kPrepRows; ++rr) {
      const int r = r0 + rr;
      if (r >= rows) break;
      const int kind = r < hq ? 0 : (r < hq + hkv ? 1 : 2);  // 0 = q, 1 = k, 2 = v
      if (kind != 2) {
        // lane l holds the pairs l, l + 64, ...: their sums, then the butterfly over the lanes
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxPairs; ++j)
          if (lane + kWave * j < half) ss += pair_sq(x1[rr][j], x2[rr][j]);
        ss = wave_sum(ss);
        const float rs = rms_inv(ss, D, eps);
#pragma unroll
        for (int j = 0; j < kMaxPairs; ++j)
          norm_rope_pair(x1[rr][j], x2[rr][j], rs, kind == 0 ? wq1[j] : wk1[j], kind == 0 ? wq2[j] : wk2[j], c[j],
                         sn[j]);
      }
      f16* dst;
      if (kind == 0) {
        dst = q_out + (int64_t(t) * hq + r) * D;
      } else {
        if (!store) continue;
        const int h = kind == 1 ? r - hq : r - hq - hkv;
        // pool layer: [2][slot][hkv][D]; V is num_slots rows after K
        dst = pool + (int64_t(kind - 1) * num_slots + slot) * hkv * D + int64_t(h) * D;
      }
#pragma unroll
      for (int j = 0; j < kMaxPairs; ++j) {
        const int i = lane + kWave * j;
        if (i < half) {
          const bool zero = kind == 0 && !pos_ok;
          dst[i] = zero ? f16(0.f) : f16(x1[rr][j]);
          dst[half + i] = zero ? f16(0.f) : f16(x2[rr][j]);
        }
      }
    }
  }
}

// The same step with rows spread over whole wavefronts, for head_dim 64 or 128 and 16-byte aligned
// arrays: D / 16 lanes per row, each holding 8 rotary pairs (PrepRows), so a wave pass covers
// 64 / (D / 16) rows.  Rows are numbered token-major (token t, then its Hq q heads, Hkv k heads,
// Hkv v heads); wave w takes kPrepPasses consecutive passes and requests all their rows and
// positions, then their rotary rows, before it computes.  q and k equal the
// one-token-per-workgroup kernel's bit for bit (the same sum of squares, see PrepRows; the same
// per-pair arithmetic), v is the same cast.
constexpr int kPrepRowsThreads = 256;
constexpr int kPrepPasses = 2;

template <int D>
__global__ __launch_bounds__(kPrepRowsThreads) void qk_norm_rope_rows_kernel(
    f16* __restrict__ q_out, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w,
    const float* __restrict__ rope, int32_t max_pos, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ slot_mapping, const uint8_t* __restrict__ active, f16* __restrict__ pool,
    int64_t num_slots, int32_t T, int32_t hq, int32_t hkv, float eps) {
  using PR = PrepRows<D>;
  const int lane = threadIdx.x % kWave;
  const int e = lane % PR::kLanes, sub = lane / PR::kLanes;
  const int64_t wave = int64_t(blockIdx.x) * (kPrepRowsThreads / kWave) + threadIdx.x / kWave;
  const int rows_per_token = hq + 2 * hkv;
  const int64_t nrows = int64_t(T) * rows_per_token;
  int64_t row[kPrepPasses];
  int tok[kPrepPasses], head[kPrepPasses], pos[kPrepPasses];
  Pairs8 x[kPrepPasses], cs[kPrepPasses];
#pragma unroll
  for (int p = 0; p < kPrepPasses; ++p) {
    row[p] = (wave * kPrepPasses + p) * PR::kRows + sub;
    const int64_t rc = min(row[p], nrows - 1);  // (past the end: a valid row again, not stored)
    tok[p] = int(rc / rows_per_token);
    head[p] = int(rc - int64_t(tok[p]) * rows_per_token);
    const float* src = head[p] < hq ? q + (int64_t(tok[p]) * hq + head[p]) * D
                       : head[p] < hq + hkv ? k + (int64_t(tok[p]) * hkv + (head[p] - hq)) * D
                                            : v + (int64_t(tok[p]) * hkv + (head[p] - hq - hkv)) * D;
    x[p] = load_pairs8<D>(src, e);
    pos[p] = positions[tok[p]];
  }
  const Pairs8 wq = load_pairs8<D>(q_norm_w, e);
  const Pairs8 wk = load_pairs8<D>(k_norm_w, e);
#pragma unroll
  for (int p = 0; p < kPrepPasses; ++p) {
    const bool pos_ok = pos[p] >= 0 && pos[p] < max_pos;
    cs[p] = load_pairs8<D>(rope + int64_t(pos_ok ? pos[p] : 0) * D, e);
  }
#pragma unroll
  for (int p = 0; p < kPrepPasses; ++p) {
    const int t = tok[p], h = head[p];
    const bool pos_ok = pos[p] >= 0 && pos[p] < max_pos;
    const int kind = h < hq ? 0 : (h < hq + hkv ? 1 : 2);  // 0 = q, 1 = k, 2 = v (uniform per row)
    u32x4 lo, hi;
    // every lane of the wave takes part in the butterfly (rows of any kind), v rows are only cast
    norm_rope_row<D>(x[p], kind == 0 ? wq : wk, cs[p], eps, lo, hi);
    if (kind == 2) {
      lo = pack_f16x8(x[p].a[0], x[p].a[1]);
      hi = pack_f16x8(x[p].b[0], x[p].b[1]);
    }
    if (row[p] >= nrows) continue;
    f16* dst;
    if (kind == 0) {
      dst = q_out + (int64_t(t) * hq + h) * D;
      if (!pos_ok) lo = hi = u32x4{0u, 0u, 0u, 0u};
    } else {
      const int64_t slot = slot_mapping[t];
      if (!(pos_ok && (active == nullptr || active[t] != 0) && slot >= 0 && slot < num_slots)) continue;
      // pool layer: [2][slot][hkv][D]; V is num_slots rows after K
      dst = pool + (int64_t(kind - 1) * num_slots + slot) * hkv * D + int64_t(kind == 1 ? h - hq : h - hq - hkv) * D;
    }
    *reinterpret_cast<u32x4*>(dst + 8 * e) = lo;
    *reinterpret_cast<u32x4*>(dst + D / 2 + 8 * e) = hi;
  }
}

// One thread block per (layer, K|V, listed page): 16-byte stores (and loads) over the page.
template <bool kCopy>
__global__ __launch_bounds__(256) void page_op_kernel(uint8_t* __restrict__ pool, int64_t num_pages,
                                                      int64_t page_bytes, const int32_t* __restrict__ dst_ids,
                                                      const int32_t* __restrict__ src_ids, int32_t n) {
  const int64_t item = blockIdx.x;  // ((layer * 2 + kv) * n + i)
  const int i = int(item % n);
  const int64_t half_index = item / n;  // layer * 2 + kv
  const int dst = dst_ids[i];
  if (dst < 0 || int64_t(dst) >= num_pages) return;
  uint8_t* base = pool + half_index * num_pages * page_bytes;
  u32x4* d = reinterpret_cast<u32x4*>(base + int64_t(dst) * page_bytes);
  const int64_t chunks = page_bytes / 16;
  if constexpr (kCopy) {
    const int src = src_ids[i];
    if (src < 0 || int64_t(src) >= num_pages) return;
    const u32x4* s = reinterpret_cast<const u32x4*>(base + int64_t(src) * page_bytes);
    for (int64_t c = threadIdx.x; c < chunks; c += blockDim.x) d[c] = s[c];
  } else {
    for (int64_t c = threadIdx.x; c < chunks; c += blockDim.x) d[c] = u32x4{0u, 0u, 0u, 0u};
  }
}

static int page_op(bool copy, void* kv_pool, int32_t num_layers, int64_t num_pages, const int32_t* dst_ids,
                   const int32_t* src_ids, int32_t n, int32_t num_kv_heads, int32_t head_dim,
                   int32_t block_size, void* stream) {
  if (kv_pool == nullptr || dst_ids == nullptr || (copy && src_ids == nullptr)) return IFN_ERR_INVALID_ARGUMENT;
  if (num_layers < 1 || num_pages < 1 || n < 0 || num_kv_heads < 1 || head_dim < 1 || block_size < 1)
    return IFN_ERR_INVALID_ARGUMENT;
  const int64_t page_bytes = int64_t(block_size) * num_kv_heads * head_dim * 2;
  if (page_bytes % 16 != 0) return IFN_ERR_UNSUPPORTED;
  IFN_CHECK_ALIGN16(kv_pool);
  if (n == 0) return IFN_OK;
  const int64_t blocks = int64_t(num_layers) * 2 * n;
  if (blocks > int64_t(1) << 31) return IFN_ERR_UNSUPPORTED;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint8_t* pool = static_cast<uint8_t*>(kv_pool);
  if (copy)
    page_op_kernel<true><<<dim3(unsigned(blocks)), dim3(256), 0, s>>>(pool, num_pages, page_bytes, dst_ids, src_ids, n);
  else
    page_op_kernel<false><<<dim3(unsigned(blocks)), dim3(256), 0, s>>>(pool, num_pages, page_bytes, dst_ids, nullptr, n);
  return ifn_launch_status();
}

}  // namespace ifn

extern "C" int ifn_qk_norm_rope_append(void* q_out, const float* q, const float* k, const float* v,
                                       const float* q_norm_weight, const float* k_norm_weight,
                                       const float* rope_table, int32_t max_positions,
                                       const int32_t* positions, const int32_t* slot_mapping,
                                       const uint8_t* active_mask, void* kv_pool_layer, int64_t num_pages,
                                       int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t block_size, float eps, void* stream) {
  using namespace ifn;
  if (q_out == nullptr || q == nullptr || k == nullptr || v == nullptr || q_norm_weight == nullptr ||
      k_norm_weight == nullptr || rope_table == nullptr || positions == nullptr || slot_mapping == nullptr ||
      kv_pool_layer == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (num_tokens < 0 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 2 || head_dim % 2 != 0 ||
      block_size < 1 || num_pages < 1 || max_positions < 1 || num_q_heads % num_kv_heads != 0 || !(eps >= 0.f))
    return IFN_ERR_INVALID_ARGUMENT;
  if (head_dim > 256) return IFN_ERR_UNSUPPORTED;
  if (num_tokens == 0) return IFN_OK;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if ((head_dim == 64 || head_dim == 128) && aligned(q_out) && aligned(q) && aligned(k) && aligned(v) &&
      aligned(q_norm_weight) && aligned(k_norm_weight) && aligned(rope_table) && aligned(kv_pool_layer)) {
    const int64_t rows = int64_t(num_tokens) * (num_q_heads + 2 * num_kv_heads);
    const int per_pass = kWave / (head_dim / 16);
    const int64_t waves = ceil_div(rows, int64_t(per_pass) * kPrepPasses);
    const int64_t blocks = ceil_div(waves, kPrepRowsThreads / kWave);
    if (blocks < (int64_t(1) << 31)) {
      auto rk = head_dim == 128 ? qk_norm_rope_rows_kernel<128> : qk_norm_rope_rows_kernel<64>;
      rk<<<dim3(unsigned(blocks)), dim3(kPrepRowsThreads), 0, s>>>(
          static_cast<f16*>(q_out), q, k, v, q_norm_weight, k_norm_weight, rope_table, max_positions, positions,
          slot_mapping, active_mask, static_cast<f16*>(kv_pool_layer), num_pages * block_size, num_tokens,
          num_q_heads, num_kv_heads, eps);
      return ifn_launch_status();
    }
  }
  auto kernel = head_dim <= 128 ? qk_norm_rope_append_kernel<1> : qk_norm_rope_append_kernel<2>;
  kernel<<<dim3(unsigned(num_tokens)), dim3(kPrepThreads), 0, s>>>(
      static_cast<f16*>(q_out), q, k, v, q_norm_weight, k_norm_weight, rope_table, max_positions, positions,
      slot_mapping, active_mask, static_cast<f16*>(kv_pool_layer), num_pages * block_size, num_q_heads,
      num_kv_heads, head_dim, eps);
  return ifn_launch_status();
}

extern "C" int ifn_zero_pages(void* kv_pool, int32_t num_layers, int64_t num_pages, const int32_t* page_ids,
                              int32_t num_ids, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                              void* stream) {
  return ifn::page_op(false, kv_pool, num_layers, num_pages, page_ids, nullptr, num_ids, num_kv_heads, head_dim,
                      block_size, stream);
}

extern "C" int ifn_copy_pages(void* kv_pool, int32_t num_layers, int64_t num_pages, const int32_t* src_ids,
                              const int32_t* dst_ids, int32_t num_ids, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, void* stream) {
  return ifn::page_op(true, kv_pool, num_layers, num_pages, dst_ids, src_ids, num_ids, num_kv_heads, head_dim,
                      block_size, stream);
}
