// Paged decode without a caller workspace, for callers that cannot allocate device memory (code
// under graph capture, serving loops and harnesses that forbid hipMalloc).  The split-KV tickets
// and partial states live in one file-scope device array per GPU of kNoAllocScratchBytes, which
// the GPU holds until the process ends.
//
// In host code `scratch` only names the array; its device address comes from
// hipGetSymbolAddress, taken once per device (with that device current) at the first call on it,
// and only that address is handed to kernels.  The array has static storage, so it is zero when
// the code object is loaded -- the tickets start at zero without any launch, and set-up puts
// nothing on the caller's stream (a first call made under graph capture records only the
// decode).  Every decode call returns the tickets it used to zero, so the array keeps that
// state between calls.  All calls on one GPU share the array: calls that overlap on one GPU (two
// streams, two host threads, or two replays of graphs holding such calls) race and must be
// serialised by the caller.
#include "ifn_common.hpp"

#include <mutex>

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device (null: not set up)

// The current device's address of `scratch`, looked up on the first call on that device.
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return IFN_ERR_HIP;
  if (dev < 0 || dev >= kMaxDevices) return IFN_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return IFN_ERR_HIP;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return IFN_OK;
}

}  // namespace

extern "C" size_t ifn_paged_decode_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int ifn_paged_decode_noalloc(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                                        const int32_t* block_tables, int32_t max_pages_per_seq,
                                        const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                                        int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t block_size, int32_t max_seq_len, float scale, void* stream) {
  if (batch == 0)  // argument checks only; nothing to launch
    return ifn_paged_decode(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                            active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                            nullptr, 0, stream);
  const size_t need = ifn_paged_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, block_size,
                                                       max_seq_len);
  if (need == 0) return IFN_ERR_INVALID_ARGUMENT;
  if (need > kNoAllocScratchBytes) return IFN_ERR_WORKSPACE;  // more rows than the fixed scratch holds
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != IFN_OK) return rc;
  return ifn_paged_decode(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                          active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                          ws, kNoAllocScratchBytes, stream);
}
