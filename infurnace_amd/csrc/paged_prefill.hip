// Causal chunked-prefill paged attention for one sequence, MFMA fp16 (gfx950).
//
// Replaces the reference's documented paged_attention for a multi-token query
// (docs/architecture.md:246; placeholder src/infurnace/kernels/paged_attention.py)
// whose contiguous semantics are src/infurnace/executor/tinygrad/model.py:116-132:
// query row i sits at start_position + i and sees keys with key_pos <= query_pos.
//
// The QK^T and PV contractions are dense, so they run on
// v_mfma_f32_32x32x16_f16 (32x32 output tile, K = 16 per instruction):
//
//  * Workgroup = (key split, block of queries, kv head).  Its waves cover every
//    query head of the GQA group: wave w takes head w % G and the 32-query
//    sub-block w / G, so each K/V tile staged in LDS is shared by all G heads.
//  * Scores are computed transposed, S^T = K . Q^T: the MFMA A operand is a
//    K row (16 B from LDS), the B operand is the lane's query row (held in
//    registers for the whole kernel), and in the 32x32 result each lane owns
//    ONE query column.  The online-softmax max/sum and the rescale of the
//    output accumulator are therefore per-lane scalars, with one lane
//    exchange (lane ^ 32) per tile for the running max.
//  * O^T += V^T . P^T: the probabilities never leave registers -- the lane's
//    16 fp32 scores of a 32-key tile are exactly the B operands of two
//    K = 16 steps once converted to fp16 (the key order inside a step is a
//    permutation shared by both operands, which a contraction allows).  V is
//    stored transposed in LDS (Vt[d][key]) so the A operand is two 8-byte reads.
//  * K/V rows are gathered page by page through the block table with 16-byte
//    loads; keys past the split, past the causal limit or in an invalid page
//    are zero-filled and masked.
//  * Long key ranges are split over workgroups (split-K) so a 512-token chunk
//    still fills the CUs; partial (m, l, O) go to the workspace and the last
//    workgroup of a (query block, kv head) merges them, as in paged decode.
#include "ifn_common.hpp"

namespace ifn {

constexpr int kPBlock = 16;  // tokens per page compiled in
constexpr int kBK = 64;      // keys per LDS tile

template <int D, int G>
struct PrefillCfg {
  static constexpr int kWaves = G > 4 ? G : 4;
  static constexpr int kQB = kWaves / G;  // 32-query sub-blocks per workgroup
  static constexpr int kBQ = 32 * kQB;    // queries per workgroup
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kKS = D + 8;       // K row stride in LDS (halves)
  static constexpr int kVS = kBK + 4;     // Vt row stride in LDS (halves)
};

struct PrefillWorkspace {
  uint32_t* count;  // [num_qblocks][num_kv_heads] tickets, zero between calls
  float* ml;        // [num_q_heads][t_pad][max_splits][2]
  float* o;         // [num_q_heads][t_pad][max_splits][D]
};

static inline size_t p_align256(size_t x) { return (x + 255) & ~size_t(255); }

struct PrefillPlan {
  int bq, n_qb, t_pad, split_keys, max_splits;
  size_t off_ml, off_o, bytes;
};

static inline int prefill_bq(int g) { return 32 * ((g > 4 ? g : 4) / g); }

static PrefillPlan plan_prefill(int32_t T, int32_t query_start, int32_t hq, int32_t hkv, int32_t d) {
  PrefillPlan p;
  const int g = hq / hkv;
  p.bq = prefill_bq(g);
  p.n_qb = int(ceil_div(T, p.bq));
  p.t_pad = p.n_qb * p.bq;
  const int64_t max_keys = int64_t(query_start) + T;
  // enough splits that (query blocks x kv heads x splits) reaches ~512 workgroups
  const int64_t units = int64_t(p.n_qb) * hkv;
  const int64_t want = ceil_div(512, units);
  int64_t sk = ceil_div(ceil_div(max_keys, want), kBK) * kBK;
  if (sk < 2 * kBK) sk = 2 * kBK;
  p.split_keys = int(sk);
  p.max_splits = int(ceil_div(max_keys, sk));
  size_t off = kTicketBytes;  // shape-independent ticket area first
  p.off_ml = off;
  off = p_align256(off + size_t(hq) * p.t_pad * p.max_splits * 2 * sizeof(float));
  p.off_o = off;
  off = p_align256(off + size_t(hq) * p.t_pad * p.max_splits * d * sizeof(float));
  p.bytes = off;
  return p;
}

template <int D, int G>
__global__ __launch_bounds__((PrefillCfg<D, G>::kThreads)) void paged_prefill_kernel(
    f16* __restrict__ out, const f16* __restrict__ q, const f16* __restrict__ pool,
    int64_t num_pages, const int32_t* __restrict__ table, int32_t max_pages, int32_t query_start,
    int32_t T, int32_t num_kv_heads, float scale_log2, int32_t split_keys, int32_t max_splits,
    int32_t t_pad, PrefillWorkspace ws) {
  using C = PrefillCfg<D, G>;
  constexpr int kDT = D / 32;  // 32-row output tiles along head_dim
  constexpr int kKSteps = D / 16;
  const int split = blockIdx.x;
  const int qb = blockIdx.y;
  const int kvh = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int g = wave % G;
  const int qsub = wave / G;
  const int hq = num_kv_heads * G;
  const int head = kvh * G + g;
  const int total = query_start + T;
  const int q0 = qb * C::kBQ;
  const int wg_key_end = min(total, query_start + q0 + C::kBQ);
  const int nsplits = int(ceil_div(wg_key_end, split_keys));
  if (split >= nsplits) return;
  const int k_begin = split * split_keys;
  const int k_end = min(k_begin + split_keys, wg_key_end);

  const int col = lane % 32;  // this lane's query column / K row within a 32-tile
  const int half = lane / 32;
  const int my_q = q0 + qsub * 32 + col;
  const int my_pos = query_start + my_q;
  const bool q_ok = my_q < T;
  const int wave_key_end = min(total, query_start + q0 + qsub * 32 + 32);

  f16x8 qreg[kKSteps];
#pragma unroll
  for (int s = 0; s < kKSteps; ++s) {
    if (q_ok)
      qreg[s] = as_h8(ld16(q + (int64_t(my_q) * hq + head) * D + 16 * s + 8 * half));
    else
      qreg[s] = f16x8{};
  }

  __shared__ __attribute__((aligned(16))) f16 Ks[kBK][C::kKS];
  __shared__ __attribute__((aligned(16))) f16 Vt[D][C::kVS];

  float m = kNegBig, lsum = 0.f;
  f32x16 acc[kDT];
#pragma unroll
  for (int dt = 0; dt < kDT; ++dt) acc[dt] = f32x16{};

  const int64_t tok_stride = int64_t(num_kv_heads) * D;
  const int64_t v_off = num_pages * kPBlock * tok_stride;
  const f16* head_pool = pool + int64_t(kvh) * D;

  for (int kt = k_begin; kt < k_end; kt += kBK) {
    __syncthreads();  // the previous tile has been consumed by every wave
    // K tile: Ks[j][:] = K[kt + j], zero beyond k_end or in an invalid page.
    constexpr int kChunks = D / 8;
    constexpr int kKItems = kBK * kChunks;
#pragma unroll
    for (int it = 0; it < int(ceil_div(kKItems, C::kThreads)); ++it) {
      const int idx = tid + it * C::kThreads;
      if (kKItems % C::kThreads != 0 && idx >= kKItems) break;
      const int j = idx / kChunks;
      const int c = idx % kChunks;
      const int key = kt + j;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (key < k_end) {
        const int page = table[key / kPBlock];
        if (page >= 0 && int64_t(page) < num_pages)
          v = ld16(head_pool + (int64_t(page) * kPBlock + key % kPBlock) * tok_stride + c * 8);
      }
      *reinterpret_cast<u32x4*>(&Ks[j][c * 8]) = v;
    }
    // V tile, transposed: each item is 4 keys x 8 dims -> 8 rows of Vt with 4 keys each.
    constexpr int kVItems = (kBK / 4) * kChunks;
#pragma unroll
    for (int it = 0; it < int(ceil_div(kVItems, C::kThreads)); ++it) {
      const int idx = tid + it * C::kThreads;
      if (kVItems % C::kThreads != 0 && idx >= kVItems) break;
      const int kq = idx / kChunks;
      const int c = idx % kChunks;
      f16x8 rows[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kt + 4 * kq + r;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (key < k_end) {
          const int page = table[key / kPBlock];
          if (page >= 0 && int64_t(page) < num_pages)
            v = ld16(head_pool + v_off + (int64_t(page) * kPBlock + key % kPBlock) * tok_stride + c * 8);
        }
        rows[r] = as_h8(v);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f16x4 col4 = f16x4{rows[0][e], rows[1][e], rows[2][e], rows[3][e]};
        *reinterpret_cast<f16x4*>(&Vt[c * 8 + e][4 * kq]) = col4;
      }
    }
    __syncthreads();
    if (kt >= wave_key_end) continue;  // every key of this tile is after this wave's queries

    // S^T = K . Q^T for keys kt..kt+63 (two 32-key tiles).
    f32x16 st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      st[t] = f32x16{};
#pragma unroll
      for (int s = 0; s < kKSteps; ++s) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(&Ks[32 * t + col][16 * s + 8 * half]);
        st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qreg[s], st[t], 0, 0, 0);
      }
    }
    // scale, causal mask (key_pos <= query_pos), online softmax per query column
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt + 32 * t + 8 * (r / 4) + 4 * half + (r % 4);
        float v = st[t][r] * scale_log2;
        if (key > my_pos || key >= k_end) v = -INFINITY;
        st[t][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx);
    const float alpha = exp2_fast(m - mn);
    m = mn;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) acc[dt] *= alpha;
    f16x8 pb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = exp2_fast(st[u / 2][8 * (u % 2) + e] - mn);
        lsum += p;
        pb[u][e] = f16(p);
      }
    // O^T += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int kb = 32 * (u / 2) + 16 * (u % 2);
        const f16x4 lo = *reinterpret_cast<const f16x4*>(&Vt[32 * dt + col][kb + 4 * half]);
        const f16x4 hi = *reinterpret_cast<const f16x4*>(&Vt[32 * dt + col][kb + 8 + 4 * half]);
        const f16x8 a = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[u], acc[dt], 0, 0, 0);
      }
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
  if (nsplits == 1) {
    if (q_ok) {
      const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
      f16* orow = out + (int64_t(my_q) * hq + head) * D;
#pragma unroll
      for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          const int d0 = 32 * dt + 8 * a4 + 4 * half;
          *reinterpret_cast<f16x4*>(orow + d0) =
              f16x4{f16(acc[dt][4 * a4] * inv), f16(acc[dt][4 * a4 + 1] * inv),
                    f16(acc[dt][4 * a4 + 2] * inv), f16(acc[dt][4 * a4 + 3] * inv)};
        }
    }
    return;
  }

  // split-K partials: unnormalised O plus (m, l), then the last workgroup merges
  {
    const int64_t slot = (int64_t(head) * t_pad + my_q) * max_splits + split;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          st_dev(ws.o + slot * D + 32 * dt + 8 * a4 + 4 * half + c, acc[dt][4 * a4 + c]);
    if (half == 0) {
      st_dev(ws.ml + slot * 2 + 0, m);
      st_dev(ws.ml + slot * 2 + 1, ltot);
    }
  }
  __shared__ uint32_t s_ticket;
  uint32_t* counter = ws.count + int64_t(qb) * num_kv_heads + kvh;
  if (!arrive_last(counter, uint32_t(nsplits - 1), &s_ticket)) return;
  for (int idx = tid; idx < G * C::kBQ * D; idx += C::kThreads) {
    const int gg = idx / (C::kBQ * D);
    const int rem = idx % (C::kBQ * D);
    const int qq = q0 + rem / D;
    const int d = rem % D;
    if (qq >= T) continue;
    const int hh = kvh * G + gg;
    const int64_t base = (int64_t(hh) * t_pad + qq) * max_splits;
    float mx = kNegBig;
    for (int s = 0; s < nsplits; ++s) mx = fmaxf(mx, ld_dev(ws.ml + (base + s) * 2));
    float L = 0.f, O = 0.f;
    for (int s = 0; s < nsplits; ++s) {
      const float wt = exp2_fast(ld_dev(ws.ml + (base + s) * 2) - mx);
      L = fmaf(wt, ld_dev(ws.ml + (base + s) * 2 + 1), L);
      O = fmaf(wt, ld_dev(ws.o + (base + s) * D + d), O);
    }
    out[(int64_t(qq) * hq + hh) * D + d] = f16(L > 0.f ? O / L : 0.f);
  }
  if (tid == 0) reset_ticket(counter);
}

typedef void (*PrefillKernel)(f16*, const f16*, const f16*, int64_t, const int32_t*, int32_t, int32_t,
                              int32_t, int32_t, float, int32_t, int32_t, int32_t, PrefillWorkspace);

static PrefillKernel pick_prefill(int d, int g, int* threads) {
#define IFN_PREFILL_CASE(DD, GG)                          \
  if (d == DD && g == GG) {                               \
    *threads = PrefillCfg<DD, GG>::kThreads;              \
    return paged_prefill_kernel<DD, GG>;                  \
  }
  IFN_PREFILL_CASE(64, 1) IFN_PREFILL_CASE(64, 2) IFN_PREFILL_CASE(64, 4) IFN_PREFILL_CASE(64, 8)
  IFN_PREFILL_CASE(128, 1) IFN_PREFILL_CASE(128, 2) IFN_PREFILL_CASE(128, 4) IFN_PREFILL_CASE(128, 8)
#undef IFN_PREFILL_CASE
  return nullptr;
}

}  // namespace ifn

extern "C" size_t ifn_paged_prefill_workspace_bytes(int32_t num_q_tokens, int32_t query_start,
                                                    int32_t num_q_heads, int32_t num_kv_heads,
                                                    int32_t head_dim, int32_t block_size) {
  if (num_q_tokens < 1 || query_start < 0 || num_q_heads < 1 || num_kv_heads < 1 ||
      head_dim < 1 || block_size < 1 || num_q_heads % num_kv_heads != 0)
    return 0;
  return ifn::plan_prefill(num_q_tokens, query_start, num_q_heads, num_kv_heads, head_dim).bytes;
}

extern "C" int ifn_paged_prefill(void* out, const void* query, const void* kv_pool_layer,
                                 int64_t num_pages, const int32_t* block_table, int32_t max_pages,
                                 int32_t query_start, int32_t num_q_tokens, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 float scale, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  using namespace ifn;
  if (out == nullptr || query == nullptr || kv_pool_layer == nullptr || block_table == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (num_pages < 1 || max_pages < 1 || query_start < 0 || num_q_tokens < 0 || num_q_heads < 1 ||
      num_kv_heads < 1 || head_dim < 1 || num_q_heads % num_kv_heads != 0)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size != kPBlock) return IFN_ERR_UNSUPPORTED;
  int threads = 0;
  PrefillKernel k = pick_prefill(head_dim, num_q_heads / num_kv_heads, &threads);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
  IFN_CHECK_ALIGN16(out);
  IFN_CHECK_ALIGN16(query);
  IFN_CHECK_ALIGN16(kv_pool_layer);
  if (num_q_tokens == 0) return IFN_OK;
  if (int64_t(query_start) + num_q_tokens > int64_t(max_pages) * kPBlock)
    return IFN_ERR_INVALID_ARGUMENT;  // keys past the end of the block table
  const PrefillPlan p = plan_prefill(num_q_tokens, query_start, num_q_heads, num_kv_heads, head_dim);
  if (int64_t(p.n_qb) * num_kv_heads > kMaxTickets) return IFN_ERR_UNSUPPORTED;
  if (p.max_splits > 1) {
    if (workspace == nullptr || workspace_bytes < p.bytes) return IFN_ERR_WORKSPACE;
    IFN_CHECK_ALIGN16(workspace);
  }
  PrefillWorkspace ws;
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  ws.count = reinterpret_cast<uint32_t*>(wsb);
  ws.ml = reinterpret_cast<float*>(wsb + p.off_ml);
  ws.o = reinterpret_cast<float*>(wsb + p.off_o);
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  dim3 grid{unsigned(p.max_splits), unsigned(p.n_qb), unsigned(num_kv_heads)};
  k<<<grid, unsigned(threads), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<f16*>(out), static_cast<const f16*>(query),
      static_cast<const f16*>(kv_pool_layer), num_pages, block_table, max_pages, query_start,
      num_q_tokens, num_kv_heads, scale * kLog2e, p.split_keys, p.max_splits, p.t_pad, ws);
  return ifn_launch_status();
}
