// Paged GQA decode attention (one query token per sequence), split-KV, gfx950.
//
// Replaces the reference's documented paged_attention for decode
// (docs/architecture.md:246; placeholder src/infurnace/kernels/paged_attention.py)
// whose contiguous semantics are src/infurnace/executor/tinygrad/model.py:196-200:
// read positions [0, pos], upcast fp16 K/V to fp32, scaled_dot_product_attention
// with scale 1/sqrt(head_dim) and query head h -> kv head h / group.
//
// Decode is HBM-bound (about 2 FLOP per KV byte), so the design is about
// reading every K/V byte exactly once with enough bytes in flight:
//
//  * Work unit = (sequence b, kv head, partition of pages_per_part pages).  The
//    grid is (max partitions, kv heads, batch); partitions past a sequence's
//    end exit at once, so ragged batches cost only the pages they own.
//  * A workgroup is 4 wavefronts; wave w takes pages w, w+4, ... of the
//    partition.  One wave owns all G query heads of its kv head, so a
//    K/V page tile is fetched once and reused from registers by every query
//    head of the GQA group.
//  * Inside a page (16 tokens x head_dim), lane = 8*row + col: the 8 lanes of
//    a row read one token's 256 B K row as 16 B chunks col and col+8, i.e.
//    each load instruction reads 8 tokens x 128 contiguous bytes.  Each lane
//    holds 2 tokens (row, row+8).  The next page is loaded before the current
//    one is consumed (register double buffering).
//  * q.k uses v_dot2_f32_f16 (fp16 pairs, fp32 accumulation); the 8 partial
//    sums of a token are reduced with three DPP steps inside the row
//    (quad_perm xor1, quad_perm xor2, row_half_mirror) -- no LDS traffic.
//  * Online softmax in base 2 (scores pre-multiplied by scale*log2 e,
//    v_exp_f32), kept per (lane row, head) so no cross-row traffic per page;
//    rows are merged once per wave with lane shuffles, waves once per
//    workgroup through LDS.
//  * Split-KV merge is fused: every partition writes (m, l, o) to the
//    workspace, then takes a ticket from a per-(b, kv head) counter; the last
//    one merges all partitions (log-sum-exp weights), writes fp16 out and
//    re-zeroes the counter.  No second launch, no wait, no spin.
#include "ifn_common.hpp"

namespace ifn {

constexpr int kDecodeThreads = 256;
constexpr int kDecodeWaves = kDecodeThreads / kWave;
constexpr int kBlock = 16;  // tokens per page compiled in

// Pages per partition for a launch: small enough to spread short batches over
// the CUs, at most 16 so ragged sequences balance.
static inline int decode_pages_per_part(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  const int64_t seq_pages = ceil_div(max_seq_len > 0 ? max_seq_len : 1, kBlock);
  const int64_t units = int64_t(batch) * num_kv_heads;
  // aim for >= 2048 workgroups when the batch is long enough to provide them
  int64_t ppp = ceil_div(seq_pages * units, 2048);
  if (ppp < 4) ppp = 4;
  if (ppp > 16) ppp = 16;
  return int(ppp);
}

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

template <int D, int G>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(
    f16* __restrict__ out, const f16* __restrict__ q, const f16* __restrict__ pool,
    int64_t num_pages, const int32_t* __restrict__ block_tables, int32_t max_pages,
    const int32_t* __restrict__ seq_lens, const uint8_t* __restrict__ active,
    int32_t num_kv_heads, int32_t max_len, float scale_log2, int32_t pages_per_part,
    DecodeWorkspace ws, int32_t max_parts) {
  constexpr int NC = D / 64;  // 16-byte chunks per lane per token row
  const int b = blockIdx.z;
  const int kvh = blockIdx.y;
  const int part = blockIdx.x;
  const int tid = threadIdx.x;
  const int hq = num_kv_heads * G;
  f16* out_bh = out + (int64_t(b) * hq + int64_t(kvh) * G) * D;
  const f16* q_bh = q + (int64_t(b) * hq + int64_t(kvh) * G) * D;

  if (active != nullptr && active[b] == 0) return;
  int len = seq_lens[b];
  len = min(len, max_pages * kBlock);
  len = min(len, max_len);
  if (len <= 0) {
    if (part == 0)
      for (int i = tid; i < G * D; i += kDecodeThreads) out_bh[i] = f16(0.f);
    return;
  }
  const int seq_pages = int(ceil_div(len, kBlock));
  const int nparts = int(ceil_div(seq_pages, pages_per_part));
  if (part >= nparts) return;
  const int p_begin = part * pages_per_part;
  const int p_end = min(p_begin + pages_per_part, seq_pages);

  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int row = lane / 8;
  const int col = lane % 8;

  f16x8 qv[G][NC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int ch = 0; ch < NC; ++ch)
      qv[g][ch] = as_h8(ld16(q_bh + g * D + (col + 8 * ch) * 8));

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
  const int32_t* bt = block_tables + int64_t(b) * max_pages;
  const f16* head_base = pool + int64_t(kvh) * D + int64_t(row) * tok_stride + col * 8;

  u32x4 kc[2][NC], vc[2][NC], kn[2][NC], vn[2][NC];
  bool ok_c = false, ok_n = false;

  auto load_page = [&](int p, u32x4 (&kr)[2][NC], u32x4 (&vr)[2][NC], bool& ok) {
    int phys = bt[p];
    ok = phys >= 0 && int64_t(phys) < num_pages;
    const f16* kb = head_base + int64_t(ok ? phys : 0) * page_elems;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int ch = 0; ch < NC; ++ch) {
        kr[tt][ch] = ld16(kb + tt * 8 * tok_stride + ch * 64);
        vr[tt][ch] = ld16(kb + v_off + tt * 8 * tok_stride + ch * 64);
      }
  };

  int p = p_begin + wave;
  if (p < p_end) load_page(p, kc, vc, ok_c);
  for (; p < p_end; p += kDecodeWaves) {
    const int pn = p + kDecodeWaves;
    if (pn < p_end) load_page(pn, kn, vn, ok_n);

    bool valid[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) valid[tt] = ok_c && (p * kBlock + row + 8 * tt) < len;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
      if (!valid[tt])
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) vc[tt][ch] = u32x4{0u, 0u, 0u, 0u};

#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        float a = 0.f;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) a = dot8(qv[g][ch], as_h8(kc[tt][ch]), a);
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
        const f16x8 v0 = as_h8(vc[0][ch]);
        const f16x8 v1 = as_h8(vc[1][ch]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          acc[g][ch][e] = fmaf(p1, float(v1[e]), fmaf(p0, float(v0[e]), acc[g][ch][e] * alpha));
      }
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int ch = 0; ch < NC; ++ch) {
        kc[tt][ch] = kn[tt][ch];
        vc[tt][ch] = vn[tt][ch];
      }
    ok_c = ok_n;
  }

  // Merge the 8 lane rows of this wave (lanes xor 8, 16, 32 hold other rows).
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

  __shared__ float s_o[kDecodeWaves][G][D];
  __shared__ float s_m[kDecodeWaves][G];
  __shared__ float s_l[kDecodeWaves][G];
  __shared__ uint32_t s_ticket;
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int ch = 0; ch < NC; ++ch)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[wave][g][(col + 8 * ch) * 8 + e] = acc[g][ch][e];
      if (col == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  const int64_t bh0 = int64_t(b) * hq + int64_t(kvh) * G;  // first query head row
  for (int i = tid; i < G * D; i += kDecodeThreads) {
    const int g = i / D;
    const int d = i % D;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) mx = fmaxf(mx, s_m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float wt = exp2_fast(s_m[w][g] - mx);
      L = fmaf(wt, s_l[w][g], L);
      O = fmaf(wt, s_o[w][g][d], O);
    }
    if (nparts == 1) {
      out_bh[i] = f16(L > 0.f ? O / L : 0.f);
    } else {
      const int64_t slot = (bh0 + g) * max_parts + part;
      st_dev(ws.o + slot * D + d, O);
      if (d == 0) {
        st_dev(ws.ml + slot * 2 + 0, mx);
        st_dev(ws.ml + slot * 2 + 1, L);
      }
    }
  }
  if (nparts == 1) return;

  // Fused split-KV merge: the last partition to finish merges all of them.
  uint32_t* counter = ws.count + int64_t(b) * num_kv_heads + kvh;
  if (!arrive_last(counter, uint32_t(nparts - 1), &s_ticket)) return;
  for (int i = tid; i < G * D; i += kDecodeThreads) {
    const int g = i / D;
    const int d = i % D;
    const int64_t base = (bh0 + g) * max_parts;
    float mx = kNegBig;
    for (int pp = 0; pp < nparts; ++pp) mx = fmaxf(mx, ld_dev(ws.ml + (base + pp) * 2));
    float L = 0.f, O = 0.f;
    for (int pp = 0; pp < nparts; ++pp) {
      const float wt = exp2_fast(ld_dev(ws.ml + (base + pp) * 2) - mx);
      L = fmaf(wt, ld_dev(ws.ml + (base + pp) * 2 + 1), L);
      O = fmaf(wt, ld_dev(ws.o + (base + pp) * D + d), O);
    }
    out_bh[i] = f16(L > 0.f ? O / L : 0.f);
  }
  if (tid == 0) reset_ticket(counter);
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
  dim3 grid{unsigned(max_parts), unsigned(num_kv_heads), unsigned(batch)};
  k<<<grid, kDecodeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<f16*>(out), static_cast<const f16*>(query),
      static_cast<const f16*>(kv_pool_layer), num_pages, block_tables, max_pages_per_seq,
      seq_lens, active_mask, num_kv_heads, len_cap, scale * kLog2e, ppp, ws, max_parts);
  return ifn_launch_status();
}
