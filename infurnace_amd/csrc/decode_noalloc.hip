// Paged decode without a caller workspace, for callers that cannot allocate device memory (code
// under graph capture, serving loops and harnesses that forbid hipMalloc).  The split-KV tickets
// and partial states live in one file-scope device array per GPU of kNoAllocScratchBytes, which
// the GPU holds until the process ends.
//
// In host code `scratch` only names the array; its device address comes from
// hipGetSymbolAddress, taken once per device (with that device current) at the first call on it,
// and only that address is handed to kernels.  The first call on a device also zeroes the ticket
// area (a fill kernel on the caller's stream, ordered before the decode); every decode call
// returns the tickets it used to zero, so the array keeps that state between calls.  All calls
// on one GPU share the array: calls that overlap on one GPU (two streams, two host threads) race
// and must be serialised by the caller.
#include "ifn_common.hpp"

#include <mutex>

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device (null: not set up)

__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

// The current device's address of `scratch`, set up on the first call on that device.
int scratch_address(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return IFN_ERR_HIP;
  if (dev < 0 || dev >= kMaxDevices) return IFN_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return IFN_ERR_HIP;
    zero_words_kernel<<<dim3(64), dim3(256), 0, stream>>>(static_cast<uint32_t*>(p),
                                                           int64_t(ifn::kTicketBytes / sizeof(uint32_t)));
    if (hipGetLastError() != hipSuccess) return IFN_ERR_HIP;
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
  const int rc = scratch_address(reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc != IFN_OK) return rc;
  return ifn_paged_decode(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                          active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                          ws, kNoAllocScratchBytes, stream);
}
