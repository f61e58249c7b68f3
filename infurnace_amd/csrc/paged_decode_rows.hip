// Launchers of the whole-row decode kernel and of its step plan (the kernels: decode_rows.hpp).
#include "decode_rows.hpp"

namespace ifn {

typedef void (*RowsKernel)(const int32_t*, const f16*, const int32_t*, const f16*, int32_t, int32_t, int32_t, int32_t,
                           int64_t, f16*, const int32_t*, const uint8_t*, float, DecodeWorkspace, DecodeAppend,
                           DecodePrep, DecodePrefix);

// The fused pre-append variant, compiled where head_dim <= 128: there the pre-append kernel holds
// one rotary pair per lane, and the variant follows that summation order.
template <int D, int G, int HKV>
static RowsKernel prep_rows() {
  if constexpr (D <= 128) return decode_rows_kernel<D, G, HKV, kRowsStages, false, true, true>;
  else return nullptr;
}

static RowsKernel pick_rows(int d, int g, int hkv, bool append, bool stream, bool prep = false,
                            bool cascade = false, int pb = kRowsBlock) {
#define IFN_ROWS_CASE(DD, GG, HH)                                                                  \
  if (d == DD && g == GG && hkv == HH) {                                                           \
    if (prep) return prep_rows<DD, GG, HH>();                                                      \
    if (cascade) return decode_rows_kernel<DD, GG, HH, kRowsStages, false, true, false, true>;     \
    if (append) return decode_rows_kernel<DD, GG, HH, kRowsStages, true, true>;                    \
    return stream ? decode_rows_kernel<DD, GG, HH, kRowsStages, false, true>                       \
                  : decode_rows_kernel<DD, GG, HH, kRowsStages, false, false>;                     \
  }
  // Pages of 32 and 64 tokens (the page-size choice is benchmarked on them): Qwen3 decode shapes,
  // plain (streaming or cached loads) and fused-append variants.
#define IFN_ROWS_PAGES(DD, GG, HH, PP)                                                                           \
  if (d == DD && g == GG && hkv == HH && pb == PP) {                                                             \
    if (prep || cascade) return nullptr;                                                                         \
    if (append) return decode_rows_kernel<DD, GG, HH, kRowsStages, true, true, false, false, PP>;                \
    return stream ? decode_rows_kernel<DD, GG, HH, kRowsStages, false, true, false, false, PP>                   \
                  : decode_rows_kernel<DD, GG, HH, kRowsStages, false, false, false, false, PP>;                 \
  }
  if (pb == kRowsBlock) {
    IFN_ROWS_CASE(128, 1, 8) IFN_ROWS_CASE(128, 2, 8) IFN_ROWS_CASE(128, 4, 8)
    IFN_ROWS_CASE(64, 1, 16) IFN_ROWS_CASE(64, 2, 16)
    IFN_ROWS_CASE(256, 1, 4) IFN_ROWS_CASE(256, 2, 4)
  }
  IFN_ROWS_PAGES(128, 2, 8, 32) IFN_ROWS_PAGES(128, 4, 8, 32)
  IFN_ROWS_PAGES(128, 2, 8, 64) IFN_ROWS_PAGES(128, 4, 8, 64)
#undef IFN_ROWS_PAGES
#undef IFN_ROWS_CASE
  return nullptr;
}

bool rows_prep_supported(int32_t hq, int32_t hkv, int32_t d) {
  return hkv >= 1 && hq % hkv == 0 && pick_rows(d, hq / hkv, hkv, false, true, true) != nullptr;
}

bool rows_decode_supported(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t max_pages, int32_t max_len,
                           int32_t block_size, bool append) {
  // the virtual token list must fit int32: batch * (cap + kRowStartCost) < 2^31
  const int64_t cap = std::min<int64_t>(int64_t(max_pages) * block_size, max_len);
  return batch >= 1 && batch <= kRowsMaxBatch && hq % hkv == 0 && batch <= kMaxTickets &&
         int64_t(batch) * (cap + kRowStartCost) < (int64_t(1) << 31) &&
         pick_rows(d, hq / hkv, hkv, append, true, false, false, block_size) != nullptr;
}

size_t rows_decode_ws_bytes(int32_t batch, int32_t hq, int32_t d, int blocks) {
  size_t off_ml, off_o;
  return rows_ws_layout(batch, hq, d, blocks, &off_ml, &off_o);
}

size_t rows_plan_bytes(int32_t batch, int blocks) { return plan_words(batch, blocks) * sizeof(int32_t); }

int rows_plan_launch(int32_t* plan, const int32_t* block_tables, int32_t max_pages, const int32_t* seq_lens,
                     const uint8_t* active, const int32_t* slots, int64_t num_pages, int32_t batch, int32_t max_len,
                     int blocks, hipStream_t stream, int32_t block_size, int32_t prefix_keys) {
  auto k = block_size == 64 ? decode_plan_kernel<64> : block_size == 32 ? decode_plan_kernel<32>
                                                                         : decode_plan_kernel<kRowsBlock>;
  if (block_size != kRowsBlock && block_size != 32 && block_size != 64) return IFN_ERR_UNSUPPORTED;
  if (prefix_keys < 0 || (prefix_keys > 0 && slots != nullptr)) return IFN_ERR_INVALID_ARGUMENT;
  k<<<dim3(1), dim3(kPlanThreads), 0, stream>>>(plan, block_tables, max_pages, seq_lens, active, slots, num_pages,
                                                batch, max_len, blocks, prefix_keys);
  return ifn_launch_status();
}

int rows_decode_launch(f16* out, const f16* q, const f16* pool, int64_t num_pages, const int32_t* block_tables,
                       int32_t max_pages, const int32_t* seq_lens, const uint8_t* active, int32_t batch, int32_t hq,
                       int32_t hkv, int32_t d, int32_t max_len, float scale_log2, void* workspace, int blocks,
                       const DecodeAppend& ap, bool cached, const int32_t* plan, hipStream_t stream,
                       const DecodePrep* prep, const DecodePrefix* px, int32_t block_size, int32_t* plan_out) {
  if (px != nullptr && (ap.pool != nullptr || prep != nullptr)) return IFN_ERR_UNSUPPORTED;
  RowsKernel k = pick_rows(d, hq / hkv, hkv, ap.pool != nullptr, !cached, prep != nullptr, px != nullptr, block_size);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
  size_t off_ml, off_o;
  rows_ws_layout(batch, hq, d, blocks, &off_ml, &off_o);
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  DecodeWorkspace ws;
  ws.count = reinterpret_cast<uint32_t*>(wsb);
  ws.ml = reinterpret_cast<float*>(wsb + off_ml);
  ws.o = reinterpret_cast<float*>(wsb + off_o);
  ws.plan_out = plan == nullptr ? plan_out : nullptr;
  const DecodePrep pp = prep != nullptr ? *prep : DecodePrep{};
  const DecodePrefix pf = px != nullptr ? *px : DecodePrefix{nullptr, nullptr, 0, 0, nullptr};
  k<<<dim3(unsigned(blocks)), dim3(kRowsThreads), 0, stream>>>(plan, pool, block_tables, q,
                                                                batch, max_pages, max_len, blocks, num_pages, out,
                                                                seq_lens, active, scale_log2, ws, ap, pp, pf);
  return ifn_launch_status();
}

}  // namespace ifn
