// Entry points of causal chunked-prefill paged attention for one sequence (gfx950), and the chunk
// store they fall back to.
//
// Replaces the reference's documented paged_attention for a multi-token query
// (docs/architecture.md:246; placeholder src/infurnace/kernels/paged_attention.py) whose contiguous
// semantics are src/infurnace/executor/tinygrad/model.py:116-132: query row i sits at
// start_position + i and sees keys with key_pos <= query_pos.
//
// The attention itself is prefill_wide_kernel (paged_prefill_wide.hip): MFMA fp16 tiles, K through
// LDS, V through transposing LDS reads.  It compiles head_dim 64 and 128 with GQA groups 1, 2, 4
// and 8; other shapes return IFN_ERR_UNSUPPORTED.  The shared-prefix pass of the shared-prefix
// decode entry point runs on the same kernel (wide_prefix_pass).
//
// ifn_paged_prefill_append fuses the chunk's K/V store into the attention launch when
// query_start % 32 == 0 (a key tile is then wholly before the chunk or wholly in it) and the chunk
// fits one buffer resource; otherwise store_chunk_kernel stores the rows and the plain attention
// follows on the same stream, with the same result.
#include "ifn_common.hpp"

namespace ifn {

constexpr int kPBlock = 16;  // tokens per page compiled in

// The chunk's K and V rows -> the pool at table[pos / 16] * 16 + pos % 16, pos = query_start + t:
// 16-byte chunks, item it of `items` per thread in a grid-stride loop.  Rows whose page id is
// outside the pool are skipped (store_kv skips slots outside the pool).
__device__ __forceinline__ void store_chunk_rows(f16* __restrict__ pool, int64_t num_pages,
                                                 const int32_t* __restrict__ table, int32_t query_start, int32_t T,
                                                 int32_t hkv, int32_t d, const f16* __restrict__ new_k,
                                                 const f16* __restrict__ new_v, int64_t first, int64_t step) {
  const int chunks = hkv * d / 8;
  const int64_t tok_stride = int64_t(hkv) * d;
  const int64_t items = int64_t(T) * 2 * chunks;
  for (int64_t it = first; it < items; it += step) {
    const int t = int(it / (2 * chunks));
    const int rem = int(it % (2 * chunks));
    const int kv = rem / chunks, c = rem % chunks;
    const int pos = query_start + t;
    const int page = table[pos / kPBlock];
    if (page < 0 || int64_t(page) >= num_pages) continue;
    const f16* src = (kv == 0 ? new_k : new_v) + int64_t(t) * tok_stride + c * 8;
    f16* dst = pool + (int64_t(kv) * num_pages * kPBlock + int64_t(page) * kPBlock + pos % kPBlock) * tok_stride + c * 8;
    *reinterpret_cast<u32x4*>(dst) = ld16(src);
  }
}

// The store alone, for chunks the fused kernel does not take (query_start % 32 != 0).
__global__ __launch_bounds__(256) void store_chunk_kernel(f16* __restrict__ pool, int64_t num_pages,
                                                          const int32_t* __restrict__ table, int32_t query_start,
                                                          int32_t T, int32_t hkv, int32_t d,
                                                          const f16* __restrict__ new_k, const f16* __restrict__ new_v) {
  store_chunk_rows(pool, num_pages, table, query_start, T, hkv, d, new_k, new_v,
                   int64_t(blockIdx.x) * blockDim.x + threadIdx.x, int64_t(gridDim.x) * blockDim.x);
}

// The shared-prefix pass (every shape the wide kernel compiles; others are unsupported).
int prefix_pass_splits(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t key_len, int cus) {
  return wide_prefill_supported(hq, hkv, d) ? wide_prefix_splits(batch, hq, hkv, d, key_len, cus) : 0;
}

int prefix_pass(const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages, int32_t key_len,
                int32_t batch, int32_t hq, int32_t hkv, int32_t d, float scale_log2, float* px_ml, float* px_o,
                f16* px_oh, int32_t stride, int cus, hipStream_t stream) {
  if (!wide_prefill_supported(hq, hkv, d)) return IFN_ERR_UNSUPPORTED;
  return wide_prefix_pass(q, pool, num_pages, prefix_pages, key_len, batch, hq, hkv, d, scale_log2, px_ml, px_o,
                          px_oh, stride, cus, stream);
}

}  // namespace ifn

// Workspace for the key split (tickets + partials); 256 bytes when the shapes need no split.
// It depends on the current device's CU count, like the launch itself.
extern "C" size_t ifn_paged_prefill_workspace_bytes(int32_t num_q_tokens, int32_t query_start,
                                                    int32_t num_q_heads, int32_t num_kv_heads,
                                                    int32_t head_dim, int32_t block_size) {
  if (num_q_tokens < 1 || query_start < 0 || num_q_heads < 1 || num_kv_heads < 1 ||
      head_dim < 1 || block_size < 1 || num_q_heads % num_kv_heads != 0)
    return 0;
  int cus = ifn::device_cu_count();
  if (cus < 1) cus = 256;
  if (ifn::wide_prefill_supported(num_q_heads, num_kv_heads, head_dim))
    return ifn::wide_prefill_ws_bytes(num_q_tokens, query_start, num_q_heads, num_kv_heads, head_dim, cus);
  return 256;  // the shape is unsupported; the launch reports it
}

namespace ifn {

static int prefill_entry(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                         const int32_t* block_table, int32_t max_pages, int32_t query_start, int32_t num_q_tokens,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         void* workspace, size_t workspace_bytes, void* stream, PrefillAppend ap) {
  const bool append = ap.pool != nullptr;
  if (out == nullptr || query == nullptr || kv_pool_layer == nullptr || block_table == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (append && (ap.new_k == nullptr || ap.new_v == nullptr)) return IFN_ERR_INVALID_ARGUMENT;
  if (num_pages < 1 || max_pages < 1 || query_start < 0 || num_q_tokens < 0 || num_q_heads < 1 ||
      num_kv_heads < 1 || head_dim < 1 || num_q_heads % num_kv_heads != 0)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size != kPBlock) return IFN_ERR_UNSUPPORTED;
  if (!wide_prefill_supported(num_q_heads, num_kv_heads, head_dim)) return IFN_ERR_UNSUPPORTED;
  IFN_CHECK_ALIGN16(out);
  IFN_CHECK_ALIGN16(query);
  IFN_CHECK_ALIGN16(kv_pool_layer);
  if (append) {
    IFN_CHECK_ALIGN16(ap.new_k);
    IFN_CHECK_ALIGN16(ap.new_v);
  }
  if (num_q_tokens == 0) return IFN_OK;
  if (int64_t(query_start) + num_q_tokens > int64_t(max_pages) * kPBlock)
    return IFN_ERR_INVALID_ARGUMENT;  // keys past the end of the block table
  const int cus = device_cu_count();
  if (cus < 1) return IFN_ERR_HIP;
  if (append && (query_start % 32 != 0 ||
                 int64_t(num_q_tokens) * num_kv_heads * head_dim * 2 >= (int64_t(1) << 31))) {
    // not fusable: the store as its own launch, then the plain attention (same result)
    const int64_t items = int64_t(num_q_tokens) * 2 * num_kv_heads * head_dim / 8;
    const int64_t grid = std::min<int64_t>((items + 255) / 256, int64_t(cus) * 16);
    store_chunk_kernel<<<dim3(unsigned(grid)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        ap.pool, num_pages, block_table, query_start, num_q_tokens, num_kv_heads, head_dim, ap.new_k, ap.new_v);
    const int rc = ifn_launch_status();
    if (rc != IFN_OK) return rc;
    ap = PrefillAppend{nullptr, nullptr, nullptr};
  }
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  return wide_prefill_launch(static_cast<f16*>(out), static_cast<const f16*>(query),
                             static_cast<const f16*>(kv_pool_layer), num_pages, block_table, query_start,
                             num_q_tokens, num_q_heads, num_kv_heads, head_dim, scale * kLog2e, workspace,
                             workspace_bytes, ap, cus, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace ifn

extern "C" int ifn_paged_prefill(void* out, const void* query, const void* kv_pool_layer,
                                 int64_t num_pages, const int32_t* block_table, int32_t max_pages,
                                 int32_t query_start, int32_t num_q_tokens, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 float scale, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  return ifn::prefill_entry(out, query, kv_pool_layer, num_pages, block_table, max_pages, query_start, num_q_tokens,
                            num_q_heads, num_kv_heads, head_dim, block_size, scale, workspace, workspace_bytes, stream,
                            ifn::PrefillAppend{nullptr, nullptr, nullptr});
}

extern "C" int ifn_paged_prefill_append(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                                        const int32_t* block_table, int32_t max_pages, int32_t query_start,
                                        int32_t num_q_tokens, const void* new_k, const void* new_v,
                                        int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t block_size, float scale, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  if (kv_pool_layer == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  return ifn::prefill_entry(out, query, kv_pool_layer, num_pages, block_table, max_pages, query_start, num_q_tokens,
                            num_q_heads, num_kv_heads, head_dim, block_size, scale, workspace, workspace_bytes, stream,
                            ifn::PrefillAppend{static_cast<const ifn::f16*>(new_k), static_cast<const ifn::f16*>(new_v),
                                               static_cast<ifn::f16*>(kv_pool_layer)});
}

extern "C" int ifn_paged_prefill_prep_append(void* out, const float* q, const float* k, const float* v,
                                             const float* q_norm_weight, const float* k_norm_weight,
                                             const float* rope_table, int32_t max_positions, void* kv_pool_layer,
                                             int64_t num_pages, const int32_t* block_table, int32_t max_pages,
                                             int32_t query_start, int32_t num_q_tokens, int32_t num_q_heads,
                                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float eps,
                                             float scale, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace ifn;
  if (out == nullptr || q == nullptr || k == nullptr || v == nullptr || q_norm_weight == nullptr ||
      k_norm_weight == nullptr || rope_table == nullptr || kv_pool_layer == nullptr || block_table == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (num_pages < 1 || max_pages < 1 || query_start < 0 || num_q_tokens < 0 || num_q_heads < 1 ||
      num_kv_heads < 1 || head_dim < 2 || head_dim % 2 != 0 || num_q_heads % num_kv_heads != 0 ||
      max_positions < 1 || !(eps >= 0.f))
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size != kPBlock) return IFN_ERR_UNSUPPORTED;
  if (!wide_prefill_supported(num_q_heads, num_kv_heads, head_dim)) return IFN_ERR_UNSUPPORTED;
  if (query_start % 32 != 0) return IFN_ERR_UNSUPPORTED;  // a key tile must be wholly before or in the chunk
  IFN_CHECK_ALIGN16(out);
  IFN_CHECK_ALIGN16(q);
  IFN_CHECK_ALIGN16(k);
  IFN_CHECK_ALIGN16(v);
  IFN_CHECK_ALIGN16(q_norm_weight);
  IFN_CHECK_ALIGN16(k_norm_weight);
  IFN_CHECK_ALIGN16(rope_table);
  IFN_CHECK_ALIGN16(kv_pool_layer);
  if (num_q_tokens == 0) return IFN_OK;
  if (int64_t(query_start) + num_q_tokens > int64_t(max_pages) * kPBlock)
    return IFN_ERR_INVALID_ARGUMENT;  // keys past the end of the block table
  if (int64_t(query_start) + num_q_tokens > max_positions) return IFN_ERR_INVALID_ARGUMENT;  // past the table
  const int cus = device_cu_count();
  if (cus < 1) return IFN_ERR_HIP;
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  const PrefillPrep prep{q, k, v, q_norm_weight, k_norm_weight, rope_table, static_cast<f16*>(kv_pool_layer), eps};
  return wide_prefill_launch(static_cast<f16*>(out), nullptr, static_cast<const f16*>(kv_pool_layer), num_pages,
                             block_table, query_start, num_q_tokens, num_q_heads, num_kv_heads, head_dim,
                             scale * kLog2e, workspace, workspace_bytes, PrefillAppend{nullptr, nullptr, nullptr}, cus,
                             reinterpret_cast<hipStream_t>(stream), &prep);
}
