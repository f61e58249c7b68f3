// Shared device helpers for the gfx950 KV-cache kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stdint.h>

#include "../../include/infurnace_amd.h"

namespace ifn {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;          // CDNA wavefront width
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for running maxima

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-byte global load / store through a plain vector type (global_load_dwordx4).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// The same load with the non-temporal hint (global_load_dwordx4 ... nt), for data read once per
// launch (decode's K/V pages, an append's source rows): the lines are not kept for reuse, and on
// MI355X such streams run measurably faster than with plain loads.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

__device__ __forceinline__ f16x8 as_h8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

// Sum of a*b over 8 fp16 pairs, accumulated in fp32 with v_dot2_f32_f16.
__device__ __forceinline__ float dot8(f16x8 a, f16x8 b, float acc) {
  acc = __builtin_amdgcn_fdot2(f16x2{a[0], a[1]}, f16x2{b[0], b[1]}, acc, false);
  acc = __builtin_amdgcn_fdot2(f16x2{a[2], a[3]}, f16x2{b[2], b[3]}, acc, false);
  acc = __builtin_amdgcn_fdot2(f16x2{a[4], a[5]}, f16x2{b[4], b[5]}, acc, false);
  acc = __builtin_amdgcn_fdot2(f16x2{a[6], a[7]}, f16x2{b[6], b[7]}, acc, false);
  return acc;
}

// DPP lane exchanges inside one 16-lane DPP row.
template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i <-> 7-i within 8 lanes
constexpr int kDppMirror = 0x140;      // row_mirror: lane i <-> 15-i within 16 lanes

// Sum over each aligned group of 8 lanes; every lane of the group gets the total.
__device__ __forceinline__ float sum8(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  return x;
}

// Sum over each aligned group of N lanes (N = 4, 8 or 16); every lane of the group gets the total.
template <int N>
__device__ __forceinline__ float sum_lanes(float x) {
  static_assert(N == 4 || N == 8 || N == 16, "DPP row reductions cover 4, 8 or 16 lanes");
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (N == 16) x += dpp<kDppMirror>(x);
  return x;
}

// Butterfly reductions over the 64 lanes of a wavefront; every lane gets the result.
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- split-KV merge protocol shared by decode and prefill ------------------------------
// Every workspace starts with a fixed ticket area (independent of the call's shapes, so a
// workspace can serve calls of any shape in sequence).  It must be zero when the workspace
// is created; each call returns the tickets it used to zero.  Partial results follow it.
constexpr size_t kTicketBytes = size_t(256) << 10;
constexpr int64_t kTicketWords = int64_t(kTicketBytes / sizeof(uint32_t));
constexpr int64_t kMaxTickets = kTicketWords - 1;  // tickets one call may use (the last word is spare)

// Device-coherent (agent scope) scalar store / load.  They compile to global_store/load
// with the sc1 bit: written through to, and read from, the device coherence point, so
// partials written on one XCD are seen by a workgroup on another without an L2
// write-back or invalidate (which a __threadfence() would issue on every workgroup).
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The same for 8 bytes at an 8-byte aligned address (one instruction each).
__device__ __forceinline__ void st_dev8(void* p, f32x2 v) {
  __hip_atomic_store(static_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x2 ld_dev8(const void* p) {
  return __builtin_bit_cast(f32x2, __hip_atomic_load(static_cast<uint64_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
}

// Device-coherent 8- and 16-byte accesses through a buffer resource: the same sc1 cache policy
// as st_dev / ld_dev (agent scope: written through to, and read from, the device coherence
// point), one instruction per lane instead of one per float.  Offsets are in bytes; an offset
// past the resource reads zero and writes nothing.
constexpr int kCpolDevice = 16;  // cache-policy operand of the buffer builtins: sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ f32x4 ld_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolDevice));
}
__device__ __forceinline__ f32x2 ld_dev2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCpolDevice));
}
__device__ __forceinline__ void st_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kCpolDevice);
}
__device__ __forceinline__ void st_dev2(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, kCpolDevice);
}

// Compiler-only barrier: no memory access is moved across it.  The split-KV handoff relies on
// the order of relaxed device-scope accesses (partial stores, then the ticket, then the merge
// loads); the hardware keeps that order (stores are acknowledged before s_waitcnt returns, and
// the merge loads sit behind a branch on the ticket's value), and these barriers keep the
// compiler from reordering them.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Waits until every memory access this wave issued has completed (stores acknowledged).
__device__ __forceinline__ void wait_all_mem() {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  compiler_fence();
}

// Called by all threads after their st_dev partial stores.  Waits until every store of
// the workgroup is acknowledged, then one thread takes a ticket; returns true in the
// workgroup that arrives last (ticket == last), which then merges with ld_dev.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t last, uint32_t* s_ticket) {
  wait_all_mem();
  __syncthreads();
  if (threadIdx.x == 0)
    *s_ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const bool last_one = *s_ticket == last;
  compiler_fence();
  return last_one;
}

// Wave-level variant: each wavefront publishes and merges on its own (no workgroup barrier).
__device__ __forceinline__ bool wave_arrive_last(uint32_t* counter, uint32_t last, int lane) {
  wait_all_mem();  // this wave's partial stores acknowledged
  uint32_t t = 0;
  if (lane == 0) t = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool last_one = uint32_t(__builtin_amdgcn_readfirstlane(int(t))) == last;
  compiler_fence();
  return last_one;
}

__device__ __forceinline__ void reset_ticket(uint32_t* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A ticket's current count, read at the device coherence point (no increment).
__device__ __forceinline__ uint32_t ld_ticket(const uint32_t* counter) {
  return __hip_atomic_load(const_cast<uint32_t*>(counter), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-KV workspace of the decode kernels: tickets (zero between calls), then the partial
// states (m in log2 units, l) and unnormalised outputs of split segments.
struct DecodeWorkspace {
  uint32_t* count;  // one ticket per segment; every call returns the tickets it used to zero
  float* ml;        // [slot][heads][2]
  float* o;         // [slot][heads][head_dim]: fp32 O (per-segment kernel) or fp16 O / l (whole-row kernel)
  int32_t* plan_out = nullptr;  // whole-row kernel, unplanned: where to write the step's plan (or null)
};

// Shared-prefix (cascade) mode: the first `pages` pages of every row at least pages * block_size
// keys long (a cascade row) hold a prefix attended separately, for all rows at once; its states
// are states 0 .. nstates - 2 of each segment (seg = row * Hkv + kv head):
// ml[((seg * nstates + s) * G + g) * 2 + {0,1}], o[((seg * nstates + s) * G + g) * D + dim].  For a
// cascade row a decode kernel streams only the pages after the prefix.  The per-segment kernel
// leaves the segment's unnormalised state (m, l, O) in state nstates - 1 for
// cascade_combine_kernel; the whole-row kernel merges the prefix states itself and writes fp16.
// Shorter rows are attended in full and written directly.  pages == 0: ordinary decode.
// The whole-row kernel reads the prefix states' outputs from oh instead: O / l in fp16 (a convex
// combination of value rows, so fp16 keeps it to a relative 2^-11), at the same indices.
struct DecodePrefix {
  float* ml;
  float* o;
  int32_t pages;
  int32_t nstates;
  const f16* oh;
};

// Fused append: store new_k / new_v of every active row at slot_mapping[row] (the store_kv
// of the same step) inside the decode launch.  The attention reads the appended token from
// new_k / new_v, not from the pool, so no ordering between the store and the reads is needed.
struct DecodeAppend {
  const f16* new_k;         // [batch][Hkv][D]
  const f16* new_v;
  const int32_t* slots;     // [batch]
  f16* pool;                // the layer's pool (the same memory the kernel reads)
};

// ---- q/k RMSNorm and half-split rotary (model.py:11-13, :24-27) ---------------------------------
// One definition of the arithmetic for the pre-append kernel and the decode kernel that fuses it,
// with every operation rounded on its own (no contraction into fma), so that both produce the same
// bits.  The sum of squares of a head is formed over the rotary pairs (x_i, x_{i + D/2}),
// i < D/2, as the butterfly i ^ 1, i ^ 2, i ^ 4, ... of the pair sums.
__device__ __forceinline__ float pair_sq(float x1, float x2) {
#pragma clang fp contract(off)
  return x1 * x1 + x2 * x2;
}
// 1 / sqrt(sum / D + eps), correctly rounded divide and square root.
__device__ __forceinline__ float rms_inv(float ss, int d, float eps) { return 1.0f / sqrtf(ss / float(d) + eps); }
// Normalise the pair with weights (w1, w2), then rotate it by the angle whose cos / sin are (c, s):
// a = x1 rs w1, b = x2 rs w2 -> (a c - b s, b c + a s).
__device__ __forceinline__ void norm_rope_pair(float& x1, float& x2, float rs, float w1, float w2, float c,
                                               float s) {
#pragma clang fp contract(off)
  const float a = x1 * rs * w1;
  const float b = x2 * rs * w2;
  x1 = a * c - b * s;
  x2 = b * c + a * s;
}

// ---- pre-append rows, 8 rotary pairs per lane ----------------------------------------------
// A row of D fp32 dims is normalised and rotated by D / 16 lanes, lane e of the row's group holding
// the rotary pairs 8 e .. 8 e + 7: dims 8 e .. 8 e + 7 (x1) and D / 2 + 8 e .. (x2).
// ifn_qk_norm_rope_append holds pair p in lane p of a wave and adds the pairs' squares with a
// butterfly over lane offsets 1, 2, 4, ..; here the butterfly's first three levels are this lane's
// own eight pairs, paired the same way, and the remaining levels lane offsets 1, 2, 4 within the
// row's group.  The same additions of the same operands give the same sum, bit for bit (for D = 64
// that kernel's last level adds its idle lanes' zeros to a non-negative sum, which changes
// nothing); the per-pair arithmetic is the shared norm_rope_pair, so q and k are identical to its.
template <int D>
struct PrepRows {
  static constexpr int kLanes = D / 16;         // lanes per row
  static constexpr int kRows = kWave / kLanes;  // rows per wave pass
};
struct Pairs8 {
  f32x4 a[2];  // element 8 e .. 8 e + 7 of the row's first half
  f32x4 b[2];  // element D / 2 + 8 e .. of its second half
};
template <int D>
__device__ __forceinline__ Pairs8 load_pairs8(const float* row, int e) {
  const f32x4* p = reinterpret_cast<const f32x4*>(row + 8 * e);
  const f32x4* s = reinterpret_cast<const f32x4*>(row + D / 2 + 8 * e);
  return Pairs8{{p[0], p[1]}, {s[0], s[1]}};
}
__device__ __forceinline__ u32x4 pack_f16x8(const f32x4& lo, const f32x4& hi) {
  return __builtin_bit_cast(u32x4, f16x8{f16(lo[0]), f16(lo[1]), f16(lo[2]), f16(lo[3]), f16(hi[0]), f16(hi[1]),
                                          f16(hi[2]), f16(hi[3])});
}
// x normalised with the weights w and rotated by the table row cs ([cos | sin]); fp16 results as
// two 16-byte chunks: dims 8 e .. (lo) and D / 2 + 8 e .. (hi).  Every lane of a row's group calls it.
template <int D>
__device__ __forceinline__ void norm_rope_row(const Pairs8& x, const Pairs8& w, const Pairs8& cs, float eps,
                                              u32x4& lo, u32x4& hi) {
  float s[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = pair_sq(x.a[j / 4][j % 4], x.b[j / 4][j % 4]);
  float ss = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
#pragma unroll
  for (int o = 1; o < PrepRows<D>::kLanes; o <<= 1) ss += __shfl_xor(ss, o);
  const float rs = rms_inv(ss, D, eps);
  f32x4 y1[2], y2[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float a = x.a[j / 4][j % 4], b = x.b[j / 4][j % 4];
    norm_rope_pair(a, b, rs, w.a[j / 4][j % 4], w.b[j / 4][j % 4], cs.a[j / 4][j % 4], cs.b[j / 4][j % 4]);
    y1[j / 4][j % 4] = a;
    y2[j / 4][j % 4] = b;
  }
  lo = pack_f16x8(y1[0], y1[1]);
  hi = pack_f16x8(y2[0], y2[1]);
}

// Fused pre-append (decode): the step's fp32 projections are normalised, rotated and cast to fp16
// inside the decode launch, as ifn_qk_norm_rope_append would do before it.  Row b's query heads are
// q[b], its new K/V row k[b] / v[b]; its rotary position positions[b] selects the table row
// [cos | sin] (a position outside [0, max_pos) gives a zero query and stores nothing).
struct DecodePrep {
  const float* q;         // [batch][Hq][D]
  const float* k;         // [batch][Hkv][D]
  const float* v;         // [batch][Hkv][D]
  const float* q_norm_w;  // [D]
  const float* k_norm_w;  // [D]
  const float* rope;      // [max_pos][D]: cos of the D/2 angles, then their sin
  const int32_t* positions;  // [batch]
  int32_t max_pos;
  float eps;
};

// Key-split workspace of the prefill kernels: tickets (zero between calls), then the splits'
// partial states (m in log2 units, l) and unnormalised outputs.
struct PrefillWorkspace {
  uint32_t* count;  // one ticket per (query block, kv head[, head]); every call returns them to zero
  float* ml;
  float* o;
};

// Fused prefill append: the chunk's new_k / new_v [T][Hkv][D] are stored into the pool at the
// table's slots for positions query_start .. query_start + T - 1, and the attention takes the
// chunk's keys and values from new_k / new_v, so the stores need no ordering against the reads.
// Requires query_start % 32 == 0 (a key tile is then wholly before the chunk or wholly in it)
// and T * Hkv * D * 2 < 2^31 bytes (one buffer resource).
struct PrefillAppend {
  const f16* new_k;
  const f16* new_v;
  f16* pool;  // the layer's pool (the memory the kernel reads)
};

// Fused pre-append (prefill chunk): the chunk's fp32 projections are normalised, rotated and cast
// inside the prefill launch, as ifn_qk_norm_rope_append would do before it.  Token t of the chunk has
// position query_start + t, for its rotary angle and for its cache slot (the table's page
// (query_start + t) / 16).  Each wave first writes the K and V rows of the chunk's key tiles it will
// read itself to the pool (workgroups sharing a tile write identical bytes), then reads them back
// like any other page.  Requires query_start % 32 == 0, query_start + T <= max_pos and 16-byte
// aligned q, k, v, weights and table.
struct PrefillPrep {
  const float* q;         // [T][Hq][D]
  const float* k;         // [T][Hkv][D]
  const float* v;         // [T][Hkv][D]
  const float* q_norm_w;  // [D]
  const float* k_norm_w;  // [D]
  const float* rope;      // [max_pos][D]: cos of the D/2 angles, then their sin
  f16* pool;              // the layer's pool (written, then read)
  float eps;
};

// Shared-prefix mode of the prefill kernels: every query row sees keys [0, key_len) (no causal
// mask) and each key split writes its result unnormalised, as the state (m, l, O), for a later
// merge: ml[((seg * stride + split) * G + g) * 2 + {0,1}], o[((seg * stride + split) * G + g) * D + dim]
// with seg = row * Hkv + kv head (stride >= nsplit).  No cross-workgroup merge happens here.
// With oh set, the output goes there instead, normalised (O / l) in fp16, at the same indices.
// key_len == 0 is ordinary causal prefill.
struct PrefixOut {
  float* ml;
  float* o;
  int32_t key_len;
  int32_t stride;
  f16* oh;
};

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Number of CUs of the current device (queried once per device; 0 when there is none).
inline int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Shared-prefix pass (paged_prefill.hip) of the shared-prefix decode entry point: each of
// `batch` query rows attends keys [0, key_len) of the pages prefix_pages[0 ..] with no mask.  The
// keys are split prefix_pass_splits() ways; each split's unnormalised state (m, l, O) goes to
// px_ml[((seg * stride + split) * G + g) * 2 + {0,1}] / px_o[((seg * stride + split) * G + g) * D + dim],
// seg = row * Hkv + kv head, stride >= the split count.
int prefix_pass_splits(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t key_len, int cus);
// With px_oh set the outputs go there as O / l in fp16 (PrefixOut::oh) and px_o is not written.
int prefix_pass(const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages, int32_t key_len,
                int32_t batch, int32_t hq, int32_t hkv, int32_t d, float scale_log2, float* px_ml, float* px_o,
                f16* px_oh, int32_t stride, int cus, hipStream_t stream);

// Chunked prefill with 64 query rows per wavefront (paged_prefill_wide.hip): the entry points'
// kernel for the (head_dim, group) it compiles; the key-split workspace it needs.
bool wide_prefill_supported(int32_t hq, int32_t hkv, int32_t d);
size_t wide_prefill_ws_bytes(int32_t T, int32_t query_start, int32_t hq, int32_t hkv, int32_t d, int cus);
int wide_prefill_launch(f16* out, const f16* q, const f16* pool, int64_t num_pages, const int32_t* table,
                        int32_t query_start, int32_t T, int32_t hq, int32_t hkv, int32_t d, float scale_log2,
                        void* workspace, size_t workspace_bytes, const PrefillAppend& ap, int cus,
                        hipStream_t stream, const PrefillPrep* prep = nullptr);
// The shared-prefix pass on that kernel (same contract as prefix_pass / prefix_pass_splits).
int wide_prefix_splits(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t key_len, int cus);
int wide_prefix_pass(const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages, int32_t key_len,
                     int32_t batch, int32_t hq, int32_t hkv, int32_t d, float scale_log2, float* px_ml, float* px_o,
                     f16* px_oh, int32_t stride, int cus, hipStream_t stream);

// Whole-row decode (paged_decode_rows.hip), used by the decode entry points when the token row
// (num_kv_heads x head_dim fp16) is 2 KiB and its (head_dim, group) is compiled; and its step plan.
// block_size: tokens per page (16 for every compiled shape; 32 and 64 for the Qwen3 decode shapes);
// append: the fused-append variant is needed.
bool rows_decode_supported(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t max_pages, int32_t max_len,
                           int32_t block_size = 16, bool append = false);
size_t rows_decode_ws_bytes(int32_t batch, int32_t hq, int32_t d, int blocks);
size_t rows_plan_bytes(int32_t batch, int blocks);
// prefix_keys > 0: a plan for the shared-prefix mode (rows of at least that many keys stream only
// the keys after them; no appended slots).
int rows_plan_launch(int32_t* plan, const int32_t* block_tables, int32_t max_pages, const int32_t* seq_lens,
                     const uint8_t* active, const int32_t* slots, int64_t num_pages, int32_t batch, int32_t max_len,
                     int blocks, hipStream_t stream, int32_t block_size = 16, int32_t prefix_keys = 0);
// prep (non-null): the fused pre-append variant; ap then carries the slots and the pool, and q is unused.
// px (non-null): shared-prefix mode (DecodePrefix), without append (plan: one built for px.pages).
// plan_out (non-null, with plan null): the call also writes the step's plan there, as
// rows_plan_launch would.
int rows_decode_launch(f16* out, const f16* q, const f16* pool, int64_t num_pages, const int32_t* block_tables,
                       int32_t max_pages, const int32_t* seq_lens, const uint8_t* active, int32_t batch, int32_t hq,
                       int32_t hkv, int32_t d, int32_t max_len, float scale_log2, void* workspace, int blocks,
                       const DecodeAppend& ap, bool cached, const int32_t* plan, hipStream_t stream,
                       const DecodePrep* prep = nullptr, const DecodePrefix* px = nullptr, int32_t block_size = 16,
                       int32_t* plan_out = nullptr);
bool rows_prep_supported(int32_t hq, int32_t hkv, int32_t d);
// The shared-prefix decode as one launch (prefix pass and private-page decode in one grid), for the
// shapes and sizes it is built for; IFN_ERR_UNSUPPORTED otherwise (the caller then runs the two
// launches).  workspace: the whole-row decode's layout for `blocks` workgroups at offset 0; px: the
// prefix states' region, room for max_states states per segment (px.nstates is set here).
int shared_prefix_fused_launch(f16* out, const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages,
                               const int32_t* block_tables, int32_t max_pages, const int32_t* seq_lens,
                               const uint8_t* active, int32_t batch, int32_t hq, int32_t hkv, int32_t d,
                               int32_t max_len, float scale_log2, void* workspace, int blocks, const DecodePrefix& px,
                               int max_states, int cus, hipStream_t stream);

}  // namespace ifn

// Host-side helpers shared by the entry points.
#define IFN_CHECK_ALIGN16(p) \
  do { if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0) return IFN_ERR_ALIGNMENT; } while (0)

static inline int ifn_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? IFN_OK : IFN_ERR_HIP;
}
