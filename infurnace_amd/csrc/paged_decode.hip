// Paged GQA decode attention (one query token per sequence), split-KV, gfx950.
//
// Replaces the reference's documented paged_attention for decode
// (docs/architecture.md:246; placeholder src/infurnace/kernels/paged_attention.py)
// whose contiguous semantics are src/infurnace/executor/tinygrad/model.py:196-200:
// read positions [0, pos], upcast fp16 K/V to fp32, scaled_dot_product_attention
// with scale 1/sqrt(head_dim) and query head h -> kv head h / group.
//
// Decode is HBM-bound (about 2 FLOP per KV byte), so the design is about
// reading every K/V byte exactly once, in DRAM-friendly order, with enough bytes
// in flight:
//
//  * Workgroup = (partition of pages_per_part pages, sequence, group of 4 kv
//    heads); wavefront w serves one kv head and all G query heads that read it,
//    streaming every page of the partition.  Small workgroups let several share
//    a CU, so one's prologue overlaps another's streaming.  Ragged sequences
//    launch only the partitions they own (the rest exit at once).
//  * Each K/V page is fetched once and reused from registers by every query
//    head of its GQA group.
//  * Inside a page (16 tokens x head_dim), lane = 8*row + col: the 8 lanes of
//    a row read one token's K row as 16 B chunks col, col+8, ..., i.e. every
//    load instruction reads 8 tokens x 128 contiguous bytes.  Each lane holds
//    2 tokens (row, row+8).  Page ids come from lanes via v_readlane; page k+1
//    is in flight while page k is consumed.
//  * q.k uses v_dot2_f32_f16 (fp16 pairs, fp32 accumulation); the 8 partial
//    sums of a token are reduced with three DPP steps inside the row
//    (quad_perm xor1, quad_perm xor2, row_half_mirror) -- no LDS traffic.
//  * Online softmax in base 2 (scores pre-multiplied by scale*log2 e,
//    v_exp_f32), kept per (lane row, head); rows merge once per partition with
//    lane shuffles.  No LDS and no workgroup barrier at all.
//  * Split-KV merge is fused: every partition's wave writes (m, l, o) to the
//    workspace with device-coherent stores, then takes a ticket from a
//    per-(sequence, kv head) counter; the last one merges all partitions
//    (log-sum-exp weights), writes fp16 out and re-zeroes the counter.  No
//    second launch, no wait loop.
#include "ifn_common.hpp"

namespace ifn {

constexpr int kBlock = 16;           // tokens per page compiled in
constexpr int kHeadsPerBlock = 4;    // wavefronts per workgroup, one per kv head
constexpr int kDecodeThreads = kHeadsPerBlock * kWave;
constexpr int kMaxPagesPerPart = 64; // page ids of a partition live in one lane each

// Pages per partition.  Each wave streams all pages of its partition for one kv head, so
// the partition length is the per-wave stream length: long enough to amortise the
// prologue/epilogue, short enough that ragged batches still spread over the CUs.
static inline int decode_pages_per_part(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  const int64_t seq_pages = ceil_div(max_seq_len > 0 ? max_seq_len : 1, kBlock);
  // about 4096 waves over the launch, counting a ragged batch at half its longest row
  int64_t ppp = ceil_div(ceil_div(seq_pages, 2) * int64_t(batch) * num_kv_heads, 4096);
  if (ppp < 8) ppp = 8;
  // the merge holds one partition per lane: at most kWave partitions per sequence
  const int64_t min_ppp = ceil_div(seq_pages, kWave);
  if (ppp < min_ppp) ppp = min_ppp;
  if (ppp > kMaxPagesPerPart) ppp = kMaxPagesPerPart;
  return int(ppp);
}

// Register-ring depth: as deep as the register budget of one 8-wave workgroup per CU allows.
template <int D, int G>
struct DecodeStages {
  static constexpr int kRegsPerLane = G * (D / 64);  // accumulator chunks per lane
  static constexpr int value = kRegsPerLane <= 4 ? 4 : (kRegsPerLane <= 8 ? 3 : 2);
};

struct DecodeWorkspace {
  uint32_t* count;  // [batch][num_kv_heads] tickets, zero between calls
  float* ml;        // [batch][num_q_heads][max_parts][2] (running max in log2 units, sum)
  float* o;         // [batch][num_q_heads][max_parts][head_dim] unnormalised outputs
};

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Workspace: [tickets: kTicketBytes][ml][o]; the ticket area is shape-independent.
static inline size_t decode_ws_layout(int32_t batch, int32_t hq, int32_t d, int32_t max_parts,
                                      size_t* off_ml, size_t* off_o) {
  size_t off = kTicketBytes;
  *off_ml = off;
  off = align256(off + size_t(batch) * hq * max_parts * 2 * sizeof(float));
  *off_o = off;
  off = align256(off + size_t(batch) * hq * max_parts * d * sizeof(float));
  return off;
}

// Grid (partition, sequence, group of 8 kv heads); wave w of a workgroup serves kv head
// 8*blockIdx.z + w and all G query heads that read it.
template <int D, int G>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(
    f16* __restrict__ out, const f16* __restrict__ q, const f16* __restrict__ pool,
    int64_t num_pages, const int32_t* __restrict__ block_tables, int32_t max_pages,
    const int32_t* __restrict__ seq_lens, const uint8_t* __restrict__ active,
    int32_t num_kv_heads, int32_t max_len, float scale_log2, int32_t pages_per_part,
    DecodeWorkspace ws, int32_t max_parts) {
  constexpr int NC = D / 64;  // 16-byte chunks per lane per token row
  const int part = blockIdx.x;
  const int b = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int kvh = blockIdx.z * kHeadsPerBlock + wave;
  if (kvh >= num_kv_heads) return;
  const int lane = threadIdx.x % kWave;
  const int hq = num_kv_heads * G;
  const int64_t bh0 = int64_t(b) * hq + int64_t(kvh) * G;  // first query-head row
  f16* out_bh = out + bh0 * D;

  if (active != nullptr && active[b] == 0) return;
  int len = seq_lens[b];
  len = min(len, max_pages * kBlock);
  len = min(len, max_len);
  if (len <= 0) {
    if (part == 0)
      for (int i = lane; i < G * D; i += kWave) out_bh[i] = f16(0.f);
    return;
  }
  const int seq_pages = int(ceil_div(len, kBlock));
  const int nparts = int(ceil_div(seq_pages, pages_per_part));
  if (part >= nparts) return;
  const int p_begin = part * pages_per_part;
  const int np = min(pages_per_part, seq_pages - p_begin);  // pages of this partition (<= 64)

  const int row = lane / 8;  // lane = 8*row + col: row -> tokens row and row+8 of a page
  const int col = lane % 8;  //                     col -> 16-byte chunks col, col+8, ...

  f16x8 qv[G][NC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int ch = 0; ch < NC; ++ch)
      qv[g][ch] = as_h8(ld16(q + bh0 * D + g * D + (col + 8 * ch) * 8));

  float m[G], l[G], acc[G][NC][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int ch = 0; ch < NC; ++ch)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][ch][e] = 0.f;
  }

  const int64_t tok_stride = int64_t(num_kv_heads) * D;  // elements between token rows
  const int64_t page_elems = kBlock * tok_stride;
  const int64_t v_off = num_pages * page_elems;
  const f16* head_base = pool + int64_t(kvh) * D + int64_t(row) * tok_stride + col * 8;
  // Lane k holds the physical id of the partition's k-th page (one load per partition);
  // the page loop takes ids with v_readlane, so consecutive pages wait on no memory.
  const int my_id = lane < np ? block_tables[int64_t(b) * max_pages + p_begin + lane] : 0;

  // S-stage register ring: page k+S-1 is requested while page k is consumed, so a wave
  // keeps S-1 pages in flight and its iteration time is about latency/(S-1) rather than
  // a full memory round trip.  Loads past the partition clamp to its last page (an L2
  // hit) so the load stream stays unconditional; consume() of those slots is skipped.
  constexpr int S = DecodeStages<D, G>::value;
  u32x4 kb[S][2][NC], vb[S][2][NC];
  bool okb[S];

  auto load_page = [&](int k, u32x4 (&kr)[2][NC], u32x4 (&vr)[2][NC], bool& ok) {
    const int phys = __builtin_amdgcn_readlane(my_id, k < np ? k : np - 1);
    ok = phys >= 0 && int64_t(phys) < num_pages;
    const f16* kbase = head_base + int64_t(ok ? phys : 0) * page_elems;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int ch = 0; ch < NC; ++ch) {
        kr[tt][ch] = ld16(kbase + tt * 8 * tok_stride + ch * 64);
        vr[tt][ch] = ld16(kbase + v_off + tt * 8 * tok_stride + ch * 64);
      }
  };

  auto consume = [&](int k, u32x4 (&kr)[2][NC], u32x4 (&vr)[2][NC], bool ok) {
    const int p = p_begin + k;
    bool valid[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) valid[tt] = ok && (p * kBlock + row + 8 * tt) < len;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
      if (!valid[tt])
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) vr[tt][ch] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        float a = 0.f;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) a = dot8(qv[g][ch], as_h8(kr[tt][ch]), a);
        a = sum8(a);
        s[tt] = valid[tt] ? a * scale_log2 : -INFINITY;
      }
      const float mn = fmaxf(m[g], fmaxf(s[0], s[1]));
      const float alpha = exp2_fast(m[g] - mn);
      const float p0 = exp2_fast(s[0] - mn);
      const float p1 = exp2_fast(s[1] - mn);
      l[g] = l[g] * alpha + p0 + p1;
      m[g] = mn;
#pragma unroll
      for (int ch = 0; ch < NC; ++ch) {
        const f16x8 v0 = as_h8(vr[0][ch]);
        const f16x8 v1 = as_h8(vr[1][ch]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          acc[g][ch][e] = fmaf(p1, float(v1[e]), fmaf(p0, float(v0[e]), acc[g][ch][e] * alpha));
      }
    }
  };

#pragma unroll
  for (int j = 0; j < S - 1; ++j) load_page(j, kb[j], vb[j], okb[j]);
  int k = 0;
  for (; k + S <= np; k += S) {  // steady state: every slot is consumed
#pragma unroll
    for (int j = 0; j < S; ++j) {
      load_page(k + j + S - 1, kb[(j + S - 1) % S], vb[(j + S - 1) % S], okb[(j + S - 1) % S]);
      __builtin_amdgcn_sched_barrier(0);
      consume(k + j, kb[j], vb[j], okb[j]);
    }
  }
  // tail: fewer than S pages left, all already requested (page k + j sits in slot j)
#pragma unroll
  for (int j = 0; j < S - 1; ++j)
    if (k + j < np) consume(k + j, kb[j], vb[j], okb[j]);

  // Merge the 8 lane rows (lanes xor 8, 16, 32 hold the other rows); afterwards every
  // lane holds the wave's state for its column's dims.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mw = m[g];
    mw = fmaxf(mw, __shfl_xor(mw, 8));
    mw = fmaxf(mw, __shfl_xor(mw, 16));
    mw = fmaxf(mw, __shfl_xor(mw, 32));
    const float sc = exp2_fast(m[g] - mw);
    m[g] = mw;
    float lw = l[g] * sc;
    lw += __shfl_xor(lw, 8);
    lw += __shfl_xor(lw, 16);
    lw += __shfl_xor(lw, 32);
    l[g] = lw;
#pragma unroll
    for (int ch = 0; ch < NC; ++ch)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = acc[g][ch][e] * sc;
        a += __shfl_xor(a, 8);
        a += __shfl_xor(a, 16);
        a += __shfl_xor(a, 32);
        acc[g][ch][e] = a;
      }
  }

  if (nparts == 1) {
    if (row == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
          f16x8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = f16(acc[g][ch][e] * inv);
          *reinterpret_cast<f16x8*>(out_bh + g * D + (col + 8 * ch) * 8) = o;
        }
      }
    }
    return;
  }

  // Split-KV: publish this partition's (m, l, O), then the last wave to arrive for
  // (sequence, kv head) merges all partitions with log-sum-exp weights.
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t slot = (bh0 + g) * max_parts + part;
#pragma unroll
      for (int ch = 0; ch < NC; ++ch)
#pragma unroll
        for (int e = 0; e < 8; ++e) st_dev(ws.o + slot * D + (col + 8 * ch) * 8 + e, acc[g][ch][e]);
      if (col == 0) {
        st_dev(ws.ml + slot * 2 + 0, m[g]);
        st_dev(ws.ml + slot * 2 + 1, l[g]);
      }
    }
  }
  uint32_t* counter = ws.count + int64_t(b) * num_kv_heads + kvh;
  if (!wave_arrive_last(counter, uint32_t(nparts - 1), lane)) return;

  // Merge (nparts <= 64).  Lane pp holds partition pp's (m, l) for every head, so the
  // weights cost one batch of loads and two wave reductions; the O partials are then read
  // in unrolled batches of 8 partitions so each batch is one memory round trip.
  float wgt[G], inv[G], mp[G], lp[G];
  const bool have = lane < nparts;
  const int pl = have ? lane : 0;  // loads stay unconditional (in-bounds), values are masked
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mp[g] = ld_dev(ws.ml + ((bh0 + g) * max_parts + pl) * 2);
    lp[g] = ld_dev(ws.ml + ((bh0 + g) * max_parts + pl) * 2 + 1);
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m_l = have ? mp[g] : kNegBig;
    const float mx = wave_max(m_l);
    wgt[g] = have ? exp2_fast(m_l - mx) : 0.f;
    const float L = wave_sum(wgt[g] * (have ? lp[g] : 0.f));
    inv[g] = L > 0.f ? 1.f / L : 0.f;
  }
  constexpr int kDw = D / kWave;  // output dims per lane per head
  float O[G][kDw];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < kDw; ++j) O[g][j] = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += 8) {
    float v[8][G][kDw];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < kDw; ++j)
          v[u][g][j] = ld_dev(ws.o + ((bh0 + g) * max_parts + min(p0 + u, nparts - 1)) * D + lane + kWave * j);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float wu = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt[g]), min(p0 + u, kWave - 1)));
#pragma unroll
        for (int j = 0; j < kDw; ++j) O[g][j] = fmaf(wu, v[u][g][j], O[g][j]);
      }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < kDw; ++j) out_bh[g * D + lane + kWave * j] = f16(O[g][j] * inv[g]);
  if (lane == 0) reset_ticket(counter);
}

typedef void (*DecodeKernel)(f16*, const f16*, const f16*, int64_t, const int32_t*, int32_t,
                             const int32_t*, const uint8_t*, int32_t, int32_t, float, int32_t,
                             DecodeWorkspace, int32_t);

static DecodeKernel pick_decode(int d, int g) {
#define IFN_DECODE_CASE(DD, GG) \
  if (d == DD && g == GG) return paged_decode_kernel<DD, GG>;
  IFN_DECODE_CASE(64, 1) IFN_DECODE_CASE(64, 2) IFN_DECODE_CASE(64, 4) IFN_DECODE_CASE(64, 8)
  IFN_DECODE_CASE(128, 1) IFN_DECODE_CASE(128, 2) IFN_DECODE_CASE(128, 4) IFN_DECODE_CASE(128, 8)
  IFN_DECODE_CASE(256, 1) IFN_DECODE_CASE(256, 2) IFN_DECODE_CASE(256, 4)
#undef IFN_DECODE_CASE
  return nullptr;
}

static int decode_max_parts(int32_t batch, int32_t hkv, int32_t max_seq_len) {
  const int ppp = decode_pages_per_part(batch, hkv, max_seq_len);
  return int(ceil_div(ceil_div(max_seq_len > 0 ? max_seq_len : 1, kBlock), ppp));
}

}  // namespace ifn

extern "C" size_t ifn_paged_decode_workspace_bytes(int32_t batch, int32_t num_q_heads,
                                                   int32_t num_kv_heads, int32_t head_dim,
                                                   int32_t block_size, int32_t max_seq_len) {
  if (batch < 1 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 || block_size < 1 ||
      max_seq_len < 0)
    return 0;
  size_t off_ml, off_o;
  return ifn::decode_ws_layout(batch, num_q_heads, head_dim,
                               ifn::decode_max_parts(batch, num_kv_heads, max_seq_len), &off_ml,
                               &off_o);
}

extern "C" int ifn_paged_decode(void* out, const void* query, const void* kv_pool_layer,
                                int64_t num_pages, const int32_t* block_tables,
                                int32_t max_pages_per_seq, const int32_t* seq_lens,
                                const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t max_seq_len, float scale, void* workspace,
                                size_t workspace_bytes, void* stream) {
  using namespace ifn;
  if (out == nullptr || query == nullptr || kv_pool_layer == nullptr || block_tables == nullptr ||
      seq_lens == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (batch < 0 || num_pages < 1 || max_pages_per_seq < 1 || num_q_heads < 1 ||
      num_kv_heads < 1 || head_dim < 1 || max_seq_len < 0 || num_q_heads % num_kv_heads != 0)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size != kBlock) return IFN_ERR_UNSUPPORTED;
  if (ceil_div(max_seq_len, kBlock) > int64_t(kWave) * kMaxPagesPerPart) return IFN_ERR_UNSUPPORTED;
  DecodeKernel k = pick_decode(head_dim, num_q_heads / num_kv_heads);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
  IFN_CHECK_ALIGN16(out);
  IFN_CHECK_ALIGN16(query);
  IFN_CHECK_ALIGN16(kv_pool_layer);
  if (batch == 0) return IFN_OK;
  const int32_t len_cap = max_seq_len < max_pages_per_seq * kBlock ? max_seq_len
                                                                    : max_pages_per_seq * kBlock;
  const int ppp = decode_pages_per_part(batch, num_kv_heads, len_cap);
  const int max_parts = int(ceil_div(ceil_div(len_cap > 0 ? len_cap : 1, kBlock), ppp));
  size_t off_ml, off_o;
  const size_t need = decode_ws_layout(batch, num_q_heads, head_dim, max_parts, &off_ml, &off_o);
  if (int64_t(batch) * num_kv_heads > kMaxTickets) return IFN_ERR_UNSUPPORTED;
  if (max_parts > 1) {
    if (workspace == nullptr || workspace_bytes < need) return IFN_ERR_WORKSPACE;
    IFN_CHECK_ALIGN16(workspace);
  }
  DecodeWorkspace ws;
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  ws.count = reinterpret_cast<uint32_t*>(wsb);
  ws.ml = reinterpret_cast<float*>(wsb + off_ml);
  ws.o = reinterpret_cast<float*>(wsb + off_o);
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  dim3 grid{unsigned(max_parts), unsigned(batch), unsigned(ceil_div(num_kv_heads, kHeadsPerBlock))};
  k<<<grid, kDecodeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<f16*>(out), static_cast<const f16*>(query),
      static_cast<const f16*>(kv_pool_layer), num_pages, block_tables, max_pages_per_seq,
      seq_lens, active_mask, num_kv_heads, len_cap, scale * kLog2e, ppp, ws, max_parts);
  return ifn_launch_status();
}
