// Paged GQA decode attention (one query token per sequence), gfx950.
//
// Replaces the reference's documented paged_attention for decode
// (docs/architecture.md:246; placeholder src/infurnace/kernels/paged_attention.py)
// whose contiguous semantics are src/infurnace/executor/tinygrad/model.py:196-200:
// read positions [0, pos], upcast fp16 K/V to fp32, scaled_dot_product_attention
// with scale 1/sqrt(head_dim) and query head h -> kv head h / group.
//
// Decode is HBM-bound (about 2 FLOP per KV byte); the kernel is built so every
// CU streams the same number of K/V bytes at a steady rate:
//
//  * Balanced flat split.  The work is the list of (row, kv head, page) units
//    in that order -- Hkv * sum(ceil(len/16)) units of 8 KiB (one kv head's
//    16 K rows + 16 V rows).  The grid is one 8-wave workgroup per CU (two
//    42 KiB LDS tables, page prefix sums and row lengths, keep the dispatcher
//    at one workgroup per CU) and wave w of N takes units [w*U/N, (w+1)*U/N).
//    Ragged batches therefore cost every wave the same bytes.  Workgroups are
//    remapped so that each XCD streams a contiguous eighth of the list.
//  * A wave's range is cut into pieces at (row, kv head) segment boundaries.
//    Inside a piece an S-stage register ring requests page k+S-1 while page k
//    is consumed; page ids sit one per lane (64 per window), read with
//    v_readlane.
//  * Each K/V page is fetched once and reused from registers by every query
//    head of its GQA group.  Inside a page, lane = 8*row + col: every load
//    instruction reads 8 token rows x 128 contiguous bytes; each lane holds 2
//    tokens.  The page loads carry the non-temporal hint (each byte is read
//    once per launch).  q.k uses v_dot2_f32_f16 (fp32 accumulation) and three DPP steps
//    inside the row; the online softmax runs in base 2 per (lane row, head).
//    At the end of a piece the 8 lane rows merge: (m, l) by butterflies, O by
//    a reduce-scatter that leaves lane 8*row + col holding element `row` of
//    its column, so partial and output stores are contiguous across lanes.
//  * A (row, kv head) segment split over several waves (at most the first and
//    last piece of each wave's range) is merged log-sum-exp style by the wave
//    that finishes last: partials go out with device-coherent stores, the
//    tickets are taken once, at the end of the wave, and the merge issues all
//    its loads in one round trip.  No second launch, no wait loop.
#include "ifn_common.hpp"

#include <atomic>

namespace ifn {

constexpr int kBlock = 16;               // tokens per page compiled in
constexpr int kWavesPerBlock = 8;
constexpr int kDecodeThreads = kWavesPerBlock * kWave;
constexpr int kRowInts = 10752;         // per-row LDS tables: 2 x 42 KiB, so one workgroup per CU
constexpr int kMaxBatch = kRowInts - 1;
constexpr int kMaxWaves = 1024 * kWavesPerBlock;  // waves of a launch are capped at this
constexpr int kXcds = 8;            // MI355X: 8 XCDs, workgroups dispatched round-robin over them




// Workspace: [tickets: kTicketBytes][ml][o].  A launch of n waves publishes into at most
// segments + n slots (slot = segment + range index).
static inline size_t decode_ws_layout(int32_t batch, int32_t hkv, int32_t g, int32_t d, int64_t waves,
                                      size_t* off_ml, size_t* off_o) {
  const size_t slots = size_t(waves) + size_t(batch) * hkv;
  size_t off = kTicketBytes;
  *off_ml = off;
  off = align256(off + slots * g * 2 * sizeof(float));
  *off_o = off;
  off = align256(off + slots * g * d * sizeof(float));
  return off;
}

// Workgroups of a decode launch: one per CU (capped so waves <= kMaxWaves).
static int decode_blocks() {
  int cus = device_cu_count();
  if (cus < 1) cus = 256;  // no device visible: size for an MI355X
  return cus < kMaxWaves / kWavesPerBlock ? cus : kMaxWaves / kWavesPerBlock;
}

// Sum over the 8 lane rows (lane = 8*row + col) of x[e], scattered so that the lane of row r
// returns the total of element e = r: three halving steps (xor 32, 16, 8 exchange 4, 2, 1
// values) instead of an all-reduce of all 8.  The selects are two-way on a row bit.
__device__ __forceinline__ float row_reduce_scatter(const float (&x)[8], int row) {
  const bool b2 = (row & 4) != 0, b1 = (row & 2) != 0, b0 = (row & 1) != 0;
  float h[4], q[2];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float keep = b2 ? x[e + 4] : x[e];
    const float send = b2 ? x[e] : x[e + 4];
    h[e] = keep + __shfl_xor(send, 32);
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float keep = b1 ? h[e + 2] : h[e];
    const float send = b1 ? h[e] : h[e + 2];
    q[e] = keep + __shfl_xor(send, 16);
  }
  const float keep = b0 ? q[1] : q[0];
  const float send = b0 ? q[0] : q[1];
  return keep + __shfl_xor(send, 8);
}

// Log-sum-exp merge of the partial states in workspace slots base .. base + npieces - 1 into the
// G output rows at o -- or, with st_ml given, into one unnormalised state at st_ml / st_o (one
// wave).  Pieces are taken 64 at a time, one per lane, with a running
// maximum; the (m, l) loads and the first batch of O loads are issued together so that the
// common case (npieces <= batch) costs a single round trip to device-coherent memory.
template <int D, int G>
__device__ __forceinline__ void merge_pieces(f16* __restrict__ o, const DecodeWorkspace& ws, int64_t base,
                                             int npieces, int lane, float* st_ml = nullptr,
                                             float* st_o = nullptr) {
  auto ml_of = [&](int i) { return ws.ml + (base + i) * G * 2; };
  auto o_of = [&](int i) { return ws.o + (base + i) * G * D; };
  constexpr int NC = D / kWave;
  constexpr int kPB = 64 / (G * NC) < 2 ? 2 : (64 / (G * NC) > 16 ? 16 : 64 / (G * NC));
  float mx[G], L[G], O[G][NC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mx[g] = kNegBig;
    L[g] = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) O[g][j] = 0.f;
  }
  for (int c0 = 0; c0 < npieces; c0 += kWave) {
    const int cnt = min(kWave, npieces - c0);
    const bool have = lane < cnt;
    const float* my_ml = ml_of(c0 + (have ? lane : cnt - 1));
    float mp[G], lp[G], v[kPB][G][NC];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mp[g] = ld_dev(my_ml + g * 2);
      lp[g] = ld_dev(my_ml + g * 2 + 1);
    }
    auto load_batch = [&](int c1) {
#pragma unroll
      for (int uu = 0; uu < kPB; ++uu) {
        const float* po = o_of(c0 + min(c1 + uu, cnt - 1));
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int j = 0; j < NC; ++j) v[uu][g][j] = ld_dev(po + g * D + lane + kWave * j);
      }
    };
    load_batch(0);
    float w[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float nm = fmaxf(mx[g], wave_max(have ? mp[g] : kNegBig));
      const float sc = exp2_fast(mx[g] - nm);
      mx[g] = nm;
      w[g] = have ? exp2_fast(mp[g] - nm) : 0.f;
      L[g] = L[g] * sc + wave_sum(w[g] * lp[g]);
#pragma unroll
      for (int j = 0; j < NC; ++j) O[g][j] *= sc;
    }
    for (int c1 = 0;;) {
#pragma unroll
      for (int uu = 0; uu < kPB; ++uu) {
        const int src = min(c1 + uu, kWave - 1);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w[g]), src));
          const float wz = c1 + uu < cnt ? wu : 0.f;
#pragma unroll
          for (int j = 0; j < NC; ++j) O[g][j] = fmaf(wz, v[uu][g][j], O[g][j]);
        }
      }
      c1 += kPB;
      if (c1 >= cnt) break;
      load_batch(c1);
    }
  }
  if (st_ml != nullptr) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int j = 0; j < NC; ++j) st_o[g * D + lane + kWave * j] = O[g][j];
      if (lane == 0) {
        st_ml[g * 2 + 0] = mx[g];
        st_ml[g * 2 + 1] = L[g];
      }
    }
    return;
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float inv = L[g] > 0.f ? 1.f / L[g] : 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) o[g * D + lane + kWave * j] = f16(O[g][j] * inv);
  }
}

// kCascade: compiled with the shared-prefix (cascade) paths; without it every cascade branch
// folds away and px is ignored.  kAppend: compiled with the fused append (ap); otherwise ap is
// ignored.  kStream: K/V page loads carry the non-temporal hint.  That is right when every page is
// read once per launch (config 2: 60.8 -> 55.2 us per launch on one box) and wrong when rows of the
// batch share pages, which the caches would otherwise serve (config 5 read through this kernel:
// 122.6 -> 149 us); the cached-load variant is kept for batches with shared pages.
template <int D, int G, bool kCascade, bool kAppend, bool kStream = true>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(
    f16* __restrict__ out, const f16* __restrict__ q, const f16* __restrict__ pool,
    int64_t num_pages, const int32_t* __restrict__ block_tables, int32_t max_pages,
    const int32_t* __restrict__ seq_lens, const uint8_t* __restrict__ active, int32_t batch,
    int32_t num_kv_heads, int32_t max_len, float scale_log2, DecodeWorkspace ws, DecodePrefix px,
    DecodeAppend ap) {
  constexpr int NC = D / 64;  // 16-byte chunks per lane per token row
  constexpr int S = 2;  // register-ring stages (measured: deeper rings were no faster)
  __shared__ int s_off[kRowInts];  // s_off[b] = pages of rows < b; s_off[batch] = total
  __shared__ int s_len[kRowInts];  // keys of row b (0 for inactive rows)
  __shared__ int s_slot[kAppend ? kRowInts : 1];  // appended slot of row b, -1 if none
  __shared__ int s_wsum[kWavesPerBlock];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int hq = num_kv_heads * G;
  const int cap = min(max_pages * kBlock, max_len);
  const int prefix_keys = px.pages * kBlock;  // rows with at least this many keys use the prefix
  auto uses_prefix = [&](int len) { return kCascade && px.pages > 0 && len >= prefix_keys; };
  auto fin_state = [&](int64_t seg) { return (seg * px.nstates + px.nstates - 1) * G; };  // cascade state
  auto row_len = [&](int b) -> int {  // keys of row b; inactive rows have none
    const int sl = seq_lens[b];                       // both loads issue before either is used
    const int act = active != nullptr ? int(active[b]) : 1;
    return act != 0 ? min(sl, cap) : 0;
  };
  const int64_t num_slots = num_pages * kBlock;
  auto append_slot = [&](int b) -> int {  // the slot row b appends to, -1 for none (store_kv's rule)
    const int64_t sl = ap.slots[b];
    const bool act = active == nullptr || active[b] != 0;
    return act && sl >= 0 && sl < num_slots ? int(sl) : -1;
  };

  // 0. Fused append: 16-byte chunks of every appended K and V row, spread over the grid.  No
  // wave of this launch reads these slots (the attention takes the token from new_k / new_v).
  // A thread's first chunk is loaded here and stored once its attention work is done
  // (flush_append), so the copy adds no round trip to the start of the launch.
  const int app_chunks = num_kv_heads * D / 8;  // per row of K (and of V)
  const int64_t app_items = kAppend ? int64_t(batch) * 2 * app_chunks : 0;
  // item it: row b = it / (2 chunks), K or V, 16-byte chunk c; the slot comes from the LDS table
  // (filled below)
  auto app_src = [&](int64_t it) __attribute__((always_inline)) {
    const int b = int(it / (2 * app_chunks)), rem = int(it % (2 * app_chunks));
    return (rem / app_chunks == 0 ? ap.new_k : ap.new_v) + int64_t(b) * num_kv_heads * D + (rem % app_chunks) * 8;
  };
  auto app_dst = [&](int64_t it) __attribute__((always_inline)) -> f16* {  // null: nothing to store
    const int b = int(it / (2 * app_chunks)), rem = int(it % (2 * app_chunks));
    const int slot = s_slot[b];
    return slot < 0 ? nullptr
                    : ap.pool + (int64_t(rem / app_chunks) * num_slots + slot) * num_kv_heads * D + (rem % app_chunks) * 8;
  };
  const int64_t app_first = int64_t(blockIdx.x) * kDecodeThreads + tid;
  u32x4 app_data = u32x4{0u, 0u, 0u, 0u};
  if constexpr (kAppend)
    if (app_first < app_items) app_data = ld16(app_src(app_first));
  auto flush_append = [&]() __attribute__((always_inline)) {
    if constexpr (kAppend) {
      if (app_first < app_items) {
        f16* d0 = app_dst(app_first);
        if (d0 != nullptr) *reinterpret_cast<u32x4*>(d0) = app_data;
      }
      for (int64_t it = app_first + int64_t(gridDim.x) * kDecodeThreads; it < app_items;
           it += int64_t(gridDim.x) * kDecodeThreads) {  // more rows than one chunk per thread
        f16* d = app_dst(it);
        if (d != nullptr) *reinterpret_cast<u32x4*>(d) = ld16(app_src(it));
      }
    }
  };

  // 1. Exclusive prefix of pages per row, in LDS (every workgroup builds its own copy).
  int running = 0;
  for (int base = 0; base < batch; base += kDecodeThreads) {
    const int i = base + tid;
    int pages = 0;
    if (i < batch) {
      const int len = row_len(i);
      s_len[i] = len;
      if constexpr (kAppend) s_slot[i] = append_slot(i);
      pages = len > 0 ? (len + kBlock - 1) / kBlock : 0;
      if (uses_prefix(len)) pages -= px.pages;  // cascade: only the pages after the prefix
    }
    int x = pages;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == kWave - 1) s_wsum[wave] = x;
    __syncthreads();
    int wpre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const int v = s_wsum[w];
      wpre += w < wave ? v : 0;
      tot += v;
    }
    if (i < batch) s_off[i] = running + wpre + x - pages;
    running += tot;
    __syncthreads();
  }
  if (tid == 0) s_off[batch] = running;
  __syncthreads();

  // Active rows with no keys get zeros (workgroup 0, one wave per row).
  if (blockIdx.x == 0) {
    for (int b = wave; b < batch; b += kWavesPerBlock) {
      const bool live = active == nullptr || active[b] != 0;
      if (live && s_off[b + 1] == s_off[b]) {  // no pages to stream
        if (uses_prefix(s_len[b])) {  // everything it sees is the prefix: an empty own state
          for (int h = 0; h < num_kv_heads; ++h) {
            const int64_t st = fin_state(int64_t(b) * num_kv_heads + h);
            for (int i = lane; i < G * D; i += kWave) px.o[st * D + i] = 0.f;
            if (lane < 2 * G) px.ml[st * 2 + lane] = (lane & 1) ? 0.f : kNegBig;
          }
        } else {
          for (int i = lane; i < hq * D; i += kWave) out[int64_t(b) * hq * D + i] = f16(0.f);
        }
      }
    }
  }

  const int64_t total_units = int64_t(running) * num_kv_heads;
  if (total_units == 0) {
    flush_append();
    return;
  }
  const int64_t nw = min(int64_t(gridDim.x) * kWavesPerBlock, total_units);
  // Static balanced split: range r covers units [T*r/nw, (T*(r+1))/nw), one per wave, so
  // every wave streams the same number of 8 KiB units.  Workgroup i runs on XCD i % 8
  // (round-robin dispatch); workgroups are remapped so that XCD x takes a contiguous
  // eighth of the unit order.  Without the remap, consecutive workgroups -- and so each
  // XCD -- would serve a fixed kv head, i.e. the same 256-byte column of every 2 KiB token
  // row, and camp on a few of its L2 channels.  Range r publishes split-segment partials in
  // slot segment + r (unique because ranges are ordered); the ranges covering a segment
  // are [range_of(first unit), range_of(last unit)].
  const int64_t nblk = gridDim.x;
  const int64_t blk = nblk % kXcds == 0 ? (blockIdx.x % kXcds) * (nblk / kXcds) + blockIdx.x / kXcds
                                        : int64_t(blockIdx.x);
  const int64_t r_wave = blk * kWavesPerBlock + wave;
  if (r_wave >= nw) {
    flush_append();
    return;
  }
  auto range_of = [&](int64_t u) -> int64_t { return ((u + 1) * nw - 1) / total_units; };

  const int row = lane / 8;  // tokens row and row+8 of a page
  const int col = lane % 8;  // 16-byte chunks col, col+8, ...
  const int64_t tok_stride = int64_t(num_kv_heads) * D;
  const int64_t page_elems = kBlock * tok_stride;
  const int64_t v_off = num_pages * page_elems;

  f16x8 qv[G][NC];
  float m[G], l[G], acc[G][NC][8];
  u32x4 kb[S][2][NC], vb[S][2][NC];
  bool okb[S];

  auto run_range = [&](int64_t r, int64_t u_lo, int64_t u_hi) {
    int pend_n = 0, pend_seg0 = 0, pend_seg1 = 0, pend_first0 = 0, pend_first1 = 0, pend_np0 = 0, pend_np1 = 0;
    struct Piece {
      int b, kvh, seg, page0, np, len, poff;  // poff: table entries skipped (shared prefix)
      int slot;  // fused append: the row's appended slot (-1: none)
      int64_t seg_start, seg_end;
    };
    auto locate = [&](int64_t u) -> Piece {  // unit u -> the piece of this range that starts at u
      int lo = 0, hi = batch - 1;              // last row whose first unit is <= u
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (int64_t(s_off[mid]) * num_kv_heads <= u) lo = mid; else hi = mid - 1;
      }
      Piece P;
      P.b = __builtin_amdgcn_readfirstlane(lo);
      const int pages_b = s_off[P.b + 1] - s_off[P.b];
      const int64_t row_start = int64_t(s_off[P.b]) * num_kv_heads;
      P.kvh = int((u - row_start) / pages_b);
      P.seg_start = row_start + int64_t(P.kvh) * pages_b;
      P.seg_end = P.seg_start + pages_b;
      P.page0 = int(u - P.seg_start);
      P.np = int(min(u_hi, P.seg_end) - u);
      P.seg = P.b * num_kv_heads + P.kvh;
      P.len = s_len[P.b];
      P.poff = uses_prefix(P.len) ? px.pages : 0;
      P.slot = kAppend ? s_slot[P.b] : -1;
      return P;
    };
    // Query rows of a piece and its first two 64-page windows of ids.  The loads are
    // unconditional (indices clamped into the piece): a fixed number of outstanding loads
    // lets every later wait count exactly.
    auto fetch_q = [&](const Piece& P, f16x8 (&qr)[G][NC]) {
      const f16* qs = q + int64_t(P.seg) * G * D;  // rows (b, kvh*G + g)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) qr[g][ch] = as_h8(ld16(qs + g * D + (col + 8 * ch) * 8));
    };
    auto fetch_ids = [&](const Piece& P, int& i0, int& i1) {
      const int32_t* bt = block_tables + int64_t(P.b) * max_pages + P.poff + P.page0;
      i0 = bt[min(lane, P.np - 1)];
      i1 = bt[min(lane + kWave, P.np - 1)];
    };
    auto head_of = [&](const Piece& P) {
      return pool + int64_t(P.kvh) * D + int64_t(row) * tok_stride + col * 8;
    };
    auto issue = [&](const Piece& P, const f16* hb, int phys, u32x4 (&kr)[2][NC], u32x4 (&vr)[2][NC], bool& ok) {
      ok = phys >= 0 && int64_t(phys) < num_pages;
      const f16* base = hb + int64_t(ok ? phys : 0) * page_elems;
      if constexpr (kAppend) {
        if (P.slot >= 0 && phys == P.slot / kBlock) {  // the page of the appended token (uniform)
          const int tok = P.slot % kBlock;
          const int64_t src = (int64_t(P.b) * num_kv_heads + P.kvh) * D + col * 8;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const bool mine = row + 8 * tt == tok;  // this lane's token is the appended one
#pragma unroll
            for (int ch = 0; ch < NC; ++ch) {
              const f16* ks_ = mine ? ap.new_k + src + ch * 64 : base + tt * 8 * tok_stride + ch * 64;
              const f16* vs_ = mine ? ap.new_v + src + ch * 64 : base + v_off + tt * 8 * tok_stride + ch * 64;
              kr[tt][ch] = kStream ? ld16_stream(ks_) : ld16(ks_);
              vr[tt][ch] = kStream ? ld16_stream(vs_) : ld16(vs_);
            }
          }
          return;
        }
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
          const f16* ks_ = base + tt * 8 * tok_stride + ch * 64;
          const f16* vs_ = base + v_off + tt * 8 * tok_stride + ch * 64;
          kr[tt][ch] = kStream ? ld16_stream(ks_) : ld16(ks_);
          vr[tt][ch] = kStream ? ld16_stream(vs_) : ld16(vs_);
        }
    };

    // The next piece is located, and its query and page ids requested, when the current
    // piece starts; its first page is requested before the current piece's row merge and
    // stores.  A piece therefore starts with its data in flight instead of paying a chain of
    // dependent loads.
    // With few accumulator chunks the next query goes to a second register set while the
    // current piece streams; otherwise (register budget) it is loaded into the live set once the
    // last page has been consumed, and arrives during the row merge.
    constexpr bool kPrefetchQ = G * NC <= 4;
    Piece cur = locate(u_lo);
    int ids0, ids1, nid0, nid1;
    f16x8 qn[kPrefetchQ ? G : 1][NC];
    fetch_q(cur, qv);
    fetch_ids(cur, ids0, ids1);
    issue(cur, head_of(cur), __builtin_amdgcn_readlane(ids0, 0), kb[0], vb[0], okb[0]);
    for (int64_t u = u_lo;;) {  // one piece per iteration (uniform loop)
      const int np = cur.np, page0 = cur.page0, len = cur.len, seg = cur.seg, poff = cur.poff;
      const int64_t seg_start = cur.seg_start, seg_end = cur.seg_end;
      const bool has_next = u + np < u_hi;
      const Piece nxt = has_next ? locate(u + np) : cur;
      if constexpr (kPrefetchQ) fetch_q(nxt, qn);
      fetch_ids(nxt, nid0, nid1);
      const int32_t* bt = block_tables + int64_t(cur.b) * max_pages + poff + page0;
      const f16* head_base = head_of(cur);
      const f16* head_next = head_of(nxt);
      int cur_w = 0;
      auto page_id = [&](int k) -> int {
        const int j = k & (kWave - 1);
        return (k >> 6) == cur_w ? __builtin_amdgcn_readlane(ids0, j) : __builtin_amdgcn_readlane(ids1, j);
      };
      auto shift = [&](int k) {  // consume enters the next 64-page window of the piece
        if ((k >> 6) != cur_w) {
          ids0 = ids1;
          cur_w = k >> 6;
          ids1 = bt[min(kWave * (cur_w + 1) + lane, np - 1)];
        }
      };
      // page k of the piece; k == np is the next piece's first page
      auto load_page = [&](int k, u32x4 (&kr)[2][NC], u32x4 (&vr)[2][NC], bool& ok) {
        if (k < np)
          issue(cur, head_base, page_id(k), kr, vr, ok);
        else if (has_next)
          issue(nxt, head_next, __builtin_amdgcn_readlane(nid0, 0), kr, vr, ok);
      };
      auto consume = [&](int k, u32x4 (&kr)[2][NC], u32x4 (&vr)[2][NC], bool ok) {
        const int p = poff + page0 + k;  // page of the row
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
          float sc[2];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            float a = 0.f;
#pragma unroll
            for (int ch = 0; ch < NC; ++ch) a = dot8(qv[g][ch], as_h8(kr[tt][ch]), a);
            a = sum8(a);
            sc[tt] = valid[tt] ? a * scale_log2 : -INFINITY;
          }
          const float mn = fmaxf(m[g], fmaxf(sc[0], sc[1]));
          const float alpha = exp2_fast(m[g] - mn);
          const float p0 = exp2_fast(sc[0] - mn);
          const float p1 = exp2_fast(sc[1] - mn);
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
      for (int g = 0; g < G; ++g) {
        m[g] = kNegBig;
        l[g] = 0.f;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][ch][e] = 0.f;
      }
      // Two-stage register ring: page k+1 is requested while page k is consumed (page k lives
      // in slot k & 1; page 0 is already in flight).  The scheduling barriers keep the loads
      // ahead of the arithmetic.
      int k = 0;
      for (; k + 2 <= np; k += 2) {
        shift(k);
        load_page(k + 1, kb[1], vb[1], okb[1]);
        __builtin_amdgcn_sched_barrier(0);
        consume(k, kb[0], vb[0], okb[0]);
        shift(k + 1);
        load_page(k + 2, kb[0], vb[0], okb[0]);  // k + 2 == np: the next piece's first page
        __builtin_amdgcn_sched_barrier(0);
        consume(k + 1, kb[1], vb[1], okb[1]);
      }
      if (k < np) {  // odd page count: the last page sits in slot 0
        shift(k);
        consume(k, kb[0], vb[0], okb[0]);
        if (has_next) issue(nxt, head_next, __builtin_amdgcn_readlane(nid0, 0), kb[0], vb[0], okb[0]);
      }
      if constexpr (!kPrefetchQ) {
        if (has_next) fetch_q(nxt, qv);
      }

      // Merge the 8 lane rows: (m, l) by butterflies; O by a reduce-scatter after which lane
      // 8*row + col holds element e = row of its column, i.e. output dim (col + 8*ch)*8 + row.
      float o_red[G][NC];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mw = m[g];
        mw = fmaxf(mw, __shfl_xor(mw, 8));
        mw = fmaxf(mw, __shfl_xor(mw, 16));
        mw = fmaxf(mw, __shfl_xor(mw, 32));
        const float scl = exp2_fast(m[g] - mw);
        m[g] = mw;
        float lw = l[g] * scl;
        lw += __shfl_xor(lw, 8);
        lw += __shfl_xor(lw, 16);
        lw += __shfl_xor(lw, 32);
        l[g] = lw;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][ch][e] *= scl;
          o_red[g][ch] = row_reduce_scatter(acc[g][ch], row);
        }
      }
      const int64_t w_first = range_of(seg_start);
      const int np_seg = int(range_of(seg_end - 1) - w_first + 1);
      if (np_seg == 1 && poff == 0) {  // this wave held the whole segment: write the output
        f16* o = out + int64_t(seg) * G * D;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
#pragma unroll
          for (int ch = 0; ch < NC; ++ch) o[g * D + (col + 8 * ch) * 8 + row] = f16(o_red[g][ch] * inv);
        }
      } else {
        // publish (m, l, O): one of several pieces to slot = segment + range; a whole segment of
        // a cascade row to its final state (merged with the prefix's by the combine kernel)
        const bool whole = np_seg == 1;
        const int64_t so = whole ? fin_state(seg) : (int64_t(seg) + r) * G;
        float* dml = (whole ? px.ml : ws.ml) + so * 2;
        float* dout = (whole ? px.o : ws.o) + so * D;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int ch = 0; ch < NC; ++ch)  // 64 lanes cover 64 consecutive floats
            st_dev(dout + g * D + (col + 8 * ch) * 8 + row, o_red[g][ch]);
        if (lane == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            st_dev(dml + g * 2 + 0, m[g]);
            st_dev(dml + g * 2 + 1, l[g]);
          }
        }
        // only the first and the last piece of a wave's range can be a split segment
        if (!whole) {
          if (pend_n == 0) {
            pend_seg0 = seg; pend_first0 = int(w_first); pend_np0 = np_seg;
          } else {
            pend_seg1 = seg; pend_first1 = int(w_first); pend_np1 = np_seg;
          }
          pend_n = pend_n + 1;
        }
      }
      if (!has_next) break;
      u += np;
      cur = nxt;
      ids0 = nid0;
      ids1 = nid1;
      if constexpr (kPrefetchQ) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int ch = 0; ch < NC; ++ch) qv[g][ch] = qn[g][ch];
      }
    }
    if (pend_n == 0) return;
    // Tickets for the range's split segments (at most its first and last piece).
    wait_all_mem();  // every partial store of this wave acknowledged
    uint32_t t = 0;
    if (lane < pend_n)
      t = __hip_atomic_fetch_add(ws.count + (lane == 0 ? pend_seg0 : pend_seg1), 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    compiler_fence();  // the merge loads below stay behind the ticket
    for (int i = 0; i < pend_n; ++i) {
      const uint32_t ti = uint32_t(__builtin_amdgcn_readlane(int(t), i));
      const int seg = i == 0 ? pend_seg0 : pend_seg1;
      const int npieces = i == 0 ? pend_np0 : pend_np1;
      if (ti != uint32_t(npieces - 1)) continue;
      // Merge pieces slot = seg + w for w = first .. first + npieces - 1 (log-sum-exp weights).
      const bool cascade = uses_prefix(s_len[seg / num_kv_heads]);  // leave a state for the combine
      merge_pieces<D, G>(out + int64_t(seg) * G * D, ws, int64_t(seg) + (i == 0 ? pend_first0 : pend_first1),
                         npieces, lane, cascade ? px.ml + fin_state(seg) * 2 : nullptr,
                         cascade ? px.o + fin_state(seg) * D : nullptr);
      if (lane == 0) reset_ticket(ws.count + seg);
    }
  };

  run_range(r_wave, total_units * r_wave / nw, total_units * (r_wave + 1) / nw);
  flush_append();
}

// Cascade rows: merge each (segment, head)'s prefix states (one per key split) and the state the
// decode kernel left for its own pages into the fp16 output.  One single-wave workgroup per
// (row, kv head, head); rows that are inactive or shorter than the prefix were finished by the
// decode kernel.  Lane s holds state s's (m, l); every state's O slice is requested before any is
// used (indices clamped, weights zero past the last state), so the merge is two round trips.
constexpr int kMaxStates = 17;  // prefix key splits (at most 16) + the decode state

template <int D>
__global__ __launch_bounds__(kWave) void cascade_combine_kernel(
    f16* __restrict__ out, const int32_t* __restrict__ seq_lens, const uint8_t* __restrict__ active,
    int32_t batch, int32_t num_kv_heads, int32_t G, int32_t cap, DecodePrefix px) {
  constexpr int NC = D / kWave;
  const int lane = threadIdx.x;
  const int64_t sg = blockIdx.x;  // (row * Hkv + kv head) * G + head
  if (sg >= int64_t(batch) * num_kv_heads * G) return;
  const int64_t seg = sg / G;
  const int g = int(sg % G);
  const int b = int(seg / num_kv_heads);
  const int len = (active == nullptr || active[b] != 0) ? min(seq_lens[b], cap) : 0;
  if (px.pages <= 0 || len < px.pages * kBlock) return;  // the decode kernel's rule for cascade rows
  const int ns = px.nstates;
  auto state = [&](int s) { return (seg * ns + min(s, ns - 1)) * G + g; };
  const float mv = px.ml[state(lane) * 2 + 0];
  const float lv = px.ml[state(lane) * 2 + 1];
  float o[kMaxStates][NC];
#pragma unroll
  for (int s = 0; s < kMaxStates; ++s)
#pragma unroll
    for (int j = 0; j < NC; ++j) o[s][j] = px.o[state(s) * D + lane + kWave * j];
  const float mx = wave_max(lane < ns ? mv : kNegBig);
  const float w = lane < ns ? exp2_fast(mv - mx) : 0.f;
  const float L = wave_sum(w * lv);
  float acc[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) acc[j] = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxStates; ++s) {
    const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s));
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = fmaf(ws, o[s][j], acc[j]);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  f16* dst = out + sg * D;
#pragma unroll
  for (int j = 0; j < NC; ++j) dst[lane + kWave * j] = f16(acc[j] * inv);
}

typedef void (*DecodeKernel)(f16*, const f16*, const f16*, int64_t, const int32_t*, int32_t,
                             const int32_t*, const uint8_t*, int32_t, int32_t, int32_t, float,
                             DecodeWorkspace, DecodePrefix, DecodeAppend);
typedef void (*CombineKernel)(f16*, const int32_t*, const uint8_t*, int32_t, int32_t, int32_t, int32_t,
                              DecodePrefix);

static CombineKernel pick_combine(int d) {
  if (d == 64) return cascade_combine_kernel<64>;
  if (d == 128) return cascade_combine_kernel<128>;
  return nullptr;
}

// kPlain streams its pages; kPlainCached is the same kernel with cached page loads, for batches whose
// rows share pages outside a common leading run.
enum class DecodeMode { kPlain, kPlainCached, kCascade, kAppend };

static DecodeKernel pick_decode(int d, int g, DecodeMode mode = DecodeMode::kPlain) {
#define IFN_DECODE_CASE(DD, GG) \
  if (d == DD && g == GG && mode == DecodeMode::kPlain) return paged_decode_kernel<DD, GG, false, false>;
#define IFN_CASCADE_CASE(DD, GG) \
  if (d == DD && g == GG && mode == DecodeMode::kCascade) return paged_decode_kernel<DD, GG, true, false>;
#define IFN_APPEND_CASE(DD, GG) \
  if (d == DD && g == GG && mode == DecodeMode::kAppend) return paged_decode_kernel<DD, GG, false, true>;
#define IFN_CACHED_CASE(DD, GG) \
  if (d == DD && g == GG && mode == DecodeMode::kPlainCached) return paged_decode_kernel<DD, GG, false, false, false>;
  IFN_DECODE_CASE(64, 1) IFN_DECODE_CASE(64, 2) IFN_DECODE_CASE(64, 4) IFN_DECODE_CASE(64, 8)
  IFN_DECODE_CASE(128, 1) IFN_DECODE_CASE(128, 2) IFN_DECODE_CASE(128, 4) IFN_DECODE_CASE(128, 8)
  IFN_DECODE_CASE(256, 1) IFN_DECODE_CASE(256, 2) IFN_DECODE_CASE(256, 4)
  IFN_CASCADE_CASE(64, 1) IFN_CASCADE_CASE(64, 2) IFN_CASCADE_CASE(64, 4) IFN_CASCADE_CASE(64, 8)
  IFN_CASCADE_CASE(128, 1) IFN_CASCADE_CASE(128, 2) IFN_CASCADE_CASE(128, 4) IFN_CASCADE_CASE(128, 8)
  IFN_APPEND_CASE(64, 1) IFN_APPEND_CASE(64, 2) IFN_APPEND_CASE(64, 4) IFN_APPEND_CASE(64, 8)
  IFN_APPEND_CASE(128, 1) IFN_APPEND_CASE(128, 2) IFN_APPEND_CASE(128, 4) IFN_APPEND_CASE(128, 8)
  IFN_APPEND_CASE(256, 1) IFN_APPEND_CASE(256, 2) IFN_APPEND_CASE(256, 4)
  IFN_CACHED_CASE(64, 1) IFN_CACHED_CASE(64, 2) IFN_CACHED_CASE(64, 4) IFN_CACHED_CASE(64, 8)
  IFN_CACHED_CASE(128, 1) IFN_CACHED_CASE(128, 2) IFN_CACHED_CASE(128, 4) IFN_CACHED_CASE(128, 8)
  IFN_CACHED_CASE(256, 1) IFN_CACHED_CASE(256, 2) IFN_CACHED_CASE(256, 4)
#undef IFN_DECODE_CASE
#undef IFN_CASCADE_CASE
#undef IFN_APPEND_CASE
#undef IFN_CACHED_CASE
  return nullptr;
}

}  // namespace ifn

extern "C" size_t ifn_paged_decode_workspace_bytes(int32_t batch, int32_t num_q_heads,
                                                   int32_t num_kv_heads, int32_t head_dim,
                                                   int32_t block_size, int32_t max_seq_len) {
  if (batch < 1 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 || block_size < 1 ||
      max_seq_len < 0 || num_q_heads % num_kv_heads != 0)
    return 0;
  size_t off_ml, off_o;
  const int blocks = ifn::decode_blocks();
  const size_t per_head = ifn::decode_ws_layout(batch, num_kv_heads, num_q_heads / num_kv_heads, head_dim,
                                                int64_t(blocks) * ifn::kWavesPerBlock, &off_ml, &off_o);
  const size_t rows = ifn::rows_decode_ws_bytes(batch, num_q_heads, head_dim, blocks);
  return per_head > rows ? per_head : rows;
}

namespace ifn {

// ifn_paged_decode, ifn_paged_decode_append and ifn_paged_decode_shared_prefix with no shared
// pages: the same checks and launch; `ap` carries the fused append (kAppend variant) when its
// pointers are given; `cached` selects the cached-load plain variant.
static int decode_entry(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                        const int32_t* block_tables, int32_t max_pages_per_seq, const int32_t* seq_lens,
                        const uint8_t* active_mask, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t block_size, int32_t max_seq_len, float scale, void* workspace,
                        size_t workspace_bytes, void* stream, const DecodeAppend& ap, bool cached = false,
                        const void* plan = nullptr, size_t plan_bytes = 0, const DecodePrep* prep = nullptr,
                        bool build_plan = false) {
  const bool append = ap.pool != nullptr;
  if (out == nullptr || query == nullptr || kv_pool_layer == nullptr || block_tables == nullptr ||
      seq_lens == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (append && (ap.slots == nullptr || (prep == nullptr && (ap.new_k == nullptr || ap.new_v == nullptr))))
    return IFN_ERR_INVALID_ARGUMENT;
  if (batch < 0 || num_pages < 1 || max_pages_per_seq < 1 || num_q_heads < 1 ||
      num_kv_heads < 1 || head_dim < 1 || max_seq_len < 0 || num_q_heads % num_kv_heads != 0)
    return IFN_ERR_INVALID_ARGUMENT;
  if (batch > kMaxBatch || int64_t(batch) * num_kv_heads > kMaxTickets) return IFN_ERR_UNSUPPORTED;
  // (an empty batch is checked as one row: it returns IFN_OK below, whichever kernel the shape has)
  const bool rows = rows_decode_supported(std::max(batch, 1), num_q_heads, num_kv_heads, head_dim, max_pages_per_seq,
                                          max_seq_len, block_size, append && prep == nullptr);
  // pages of other sizes than 16 tokens: the whole-row kernel, where it compiles them, only
  if (block_size != kBlock && (!rows || prep != nullptr)) return IFN_ERR_UNSUPPORTED;
  DecodeKernel k = rows ? nullptr
                        : pick_decode(head_dim, num_q_heads / num_kv_heads,
                                      append ? DecodeMode::kAppend
                                             : (cached ? DecodeMode::kPlainCached : DecodeMode::kPlain));
  if (!rows && k == nullptr) return IFN_ERR_UNSUPPORTED;
  if (prep != nullptr && (!rows || !rows_prep_supported(num_q_heads, num_kv_heads, head_dim)))
    return IFN_ERR_UNSUPPORTED;
  // (a call that builds the step's plan needs somewhere to write it, where the shape has a plan)
  if (build_plan && rows && batch > 0 && plan == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  IFN_CHECK_ALIGN16(out);
  IFN_CHECK_ALIGN16(query);
  IFN_CHECK_ALIGN16(kv_pool_layer);
  if (append && prep == nullptr) {
    IFN_CHECK_ALIGN16(ap.new_k);
    IFN_CHECK_ALIGN16(ap.new_v);
  }
  if (batch == 0) return IFN_OK;
  const int blocks = decode_blocks();
  // the size ifn_paged_decode_workspace_bytes reports is the requirement, whichever kernel runs
  const size_t need = ifn_paged_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, block_size,
                                                       max_seq_len);
  if (workspace == nullptr || workspace_bytes < need) return IFN_ERR_WORKSPACE;
  IFN_CHECK_ALIGN16(workspace);
  if (device_cu_count() < 1) return IFN_ERR_HIP;
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  if (rows) {
    // planned: the kernel reads this workgroup's record before checking the header; build_plan: every
    // workgroup writes its record
    if (plan != nullptr) {
      if (plan_bytes < rows_plan_bytes(batch, blocks)) return IFN_ERR_WORKSPACE;
      IFN_CHECK_ALIGN16(plan);
    }
    return rows_decode_launch(static_cast<f16*>(out), static_cast<const f16*>(query),
                              static_cast<const f16*>(kv_pool_layer), num_pages, block_tables, max_pages_per_seq,
                              seq_lens, active_mask, batch, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                              scale * kLog2e, workspace, blocks, ap, cached,
                              build_plan ? nullptr : static_cast<const int32_t*>(plan),
                              reinterpret_cast<hipStream_t>(stream), prep, nullptr, block_size,
                              build_plan ? static_cast<int32_t*>(const_cast<void*>(plan)) : nullptr);
  }
  size_t off_ml, off_o;
  decode_ws_layout(batch, num_kv_heads, num_q_heads / num_kv_heads, head_dim, int64_t(blocks) * kWavesPerBlock,
                   &off_ml, &off_o);
  DecodeWorkspace ws;
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  ws.count = reinterpret_cast<uint32_t*>(wsb);
  ws.ml = reinterpret_cast<float*>(wsb + off_ml);
  ws.o = reinterpret_cast<float*>(wsb + off_o);
  k<<<dim3(unsigned(blocks)), dim3(kDecodeThreads), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<f16*>(out), static_cast<const f16*>(query),
      static_cast<const f16*>(kv_pool_layer), num_pages, block_tables, max_pages_per_seq,
      seq_lens, active_mask, batch, num_kv_heads, max_seq_len, scale * kLog2e, ws, DecodePrefix{nullptr, nullptr, 0, 0, nullptr},
      ap);
  return ifn_launch_status();
}

}  // namespace ifn

extern "C" int ifn_paged_decode(void* out, const void* query, const void* kv_pool_layer,
                                int64_t num_pages, const int32_t* block_tables,
                                int32_t max_pages_per_seq, const int32_t* seq_lens,
                                const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t max_seq_len, float scale, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return ifn::decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                           active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                           workspace, workspace_bytes, stream, ifn::DecodeAppend{nullptr, nullptr, nullptr, nullptr});
}

extern "C" int ifn_paged_decode_append(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                                       const int32_t* block_tables, int32_t max_pages_per_seq,
                                       const int32_t* seq_lens, const uint8_t* active_mask,
                                       const int32_t* slot_mapping, const void* new_k, const void* new_v,
                                       int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                       int32_t block_size, int32_t max_seq_len, float scale, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  if (kv_pool_layer == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  return ifn::decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                           active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                           workspace, workspace_bytes, stream,
                           ifn::DecodeAppend{static_cast<const ifn::f16*>(new_k), static_cast<const ifn::f16*>(new_v),
                                             slot_mapping, static_cast<ifn::f16*>(kv_pool_layer)});
}

extern "C" size_t ifn_paged_decode_plan_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                              int32_t head_dim, int32_t block_size, int32_t max_pages_per_seq,
                                              int32_t max_seq_len) {
  if (batch < 1 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 || block_size < 1 ||
      num_q_heads % num_kv_heads != 0 || max_pages_per_seq < 1 || max_seq_len < 0)
    return 0;
  if (!ifn::rows_decode_supported(batch, num_q_heads, num_kv_heads, head_dim, max_pages_per_seq, max_seq_len,
                                  block_size))
    return 0;
  return ifn::rows_plan_bytes(batch, ifn::decode_blocks());
}

extern "C" int ifn_paged_decode_plan(void* plan, size_t plan_bytes, const int32_t* block_tables,
                                     int32_t max_pages_per_seq, const int32_t* seq_lens, const uint8_t* active_mask,
                                     const int32_t* slot_mapping, int64_t num_pages, int32_t batch,
                                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                     int32_t max_seq_len, void* stream) {
  using namespace ifn;
  if (block_tables == nullptr || seq_lens == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  if (batch < 0 || num_pages < 1 || max_pages_per_seq < 1 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 ||
      max_seq_len < 0 || num_q_heads % num_kv_heads != 0)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size < 1) return IFN_ERR_INVALID_ARGUMENT;
  if (batch == 0) return IFN_OK;
  if (!rows_decode_supported(batch, num_q_heads, num_kv_heads, head_dim, max_pages_per_seq, max_seq_len, block_size))
    return block_size == kBlock ? IFN_OK : IFN_ERR_UNSUPPORTED;  // 16: these shapes decode without a plan
  const int blocks = decode_blocks();
  if (plan == nullptr || plan_bytes < rows_plan_bytes(batch, blocks)) return IFN_ERR_WORKSPACE;
  IFN_CHECK_ALIGN16(plan);
  if (device_cu_count() < 1) return IFN_ERR_HIP;
  return rows_plan_launch(static_cast<int32_t*>(plan), block_tables, max_pages_per_seq, seq_lens, active_mask,
                          slot_mapping, num_pages, batch, max_seq_len, blocks, reinterpret_cast<hipStream_t>(stream),
                          block_size);
}

extern "C" int ifn_paged_decode_planned(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                                        const int32_t* block_tables, int32_t max_pages_per_seq,
                                        const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                                        int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t block_size, int32_t max_seq_len, float scale, const void* plan,
                                        size_t plan_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  return ifn::decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                           active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                           workspace, workspace_bytes, stream, ifn::DecodeAppend{nullptr, nullptr, nullptr, nullptr},
                           false, plan, plan_bytes);
}

extern "C" int ifn_paged_decode_append_planned(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                                               const int32_t* block_tables, int32_t max_pages_per_seq,
                                               const int32_t* seq_lens, const uint8_t* active_mask,
                                               const int32_t* slot_mapping, const void* new_k, const void* new_v,
                                               int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                               int32_t head_dim, int32_t block_size, int32_t max_seq_len, float scale,
                                               const void* plan, size_t plan_bytes, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  if (kv_pool_layer == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  return ifn::decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                           active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                           workspace, workspace_bytes, stream,
                           ifn::DecodeAppend{static_cast<const ifn::f16*>(new_k), static_cast<const ifn::f16*>(new_v),
                                             slot_mapping, static_cast<ifn::f16*>(kv_pool_layer)},
                           false, plan, plan_bytes);
}

extern "C" int ifn_paged_decode_planning(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                                         const int32_t* block_tables, int32_t max_pages_per_seq,
                                         const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                         int32_t block_size, int32_t max_seq_len, float scale, void* plan,
                                         size_t plan_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  return ifn::decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                           active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                           workspace, workspace_bytes, stream, ifn::DecodeAppend{nullptr, nullptr, nullptr, nullptr},
                           false, plan, plan_bytes, nullptr, true);
}

extern "C" int ifn_paged_decode_append_planning(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                                                const int32_t* block_tables, int32_t max_pages_per_seq,
                                                const int32_t* seq_lens, const uint8_t* active_mask,
                                                const int32_t* slot_mapping, const void* new_k, const void* new_v,
                                                int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t block_size, int32_t max_seq_len,
                                                float scale, void* plan, size_t plan_bytes, void* workspace,
                                                size_t workspace_bytes, void* stream) {
  if (kv_pool_layer == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  return ifn::decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                           active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                           workspace, workspace_bytes, stream,
                           ifn::DecodeAppend{static_cast<const ifn::f16*>(new_k), static_cast<const ifn::f16*>(new_v),
                                             slot_mapping, static_cast<ifn::f16*>(kv_pool_layer)},
                           false, plan, plan_bytes, nullptr, true);
}

namespace ifn {

static int prep_append_entry(void* out, const float* q, const float* k, const float* v, const float* q_norm_weight,
                             const float* k_norm_weight, const float* rope_table, int32_t max_positions,
                             const int32_t* positions, const int32_t* slot_mapping, void* kv_pool_layer,
                             int64_t num_pages, const int32_t* block_tables, int32_t max_pages_per_seq,
                             const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t max_seq_len,
                             float scale, float eps, const void* plan, size_t plan_bytes, void* workspace,
                             size_t workspace_bytes, void* stream, bool build_plan) {
  if (q == nullptr || k == nullptr || v == nullptr || q_norm_weight == nullptr || k_norm_weight == nullptr ||
      rope_table == nullptr || positions == nullptr || slot_mapping == nullptr || kv_pool_layer == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (max_positions < 1 || !(eps >= 0.f) || head_dim % 8 != 0) return IFN_ERR_INVALID_ARGUMENT;
  IFN_CHECK_ALIGN16(k);
  IFN_CHECK_ALIGN16(v);
  IFN_CHECK_ALIGN16(q_norm_weight);
  IFN_CHECK_ALIGN16(k_norm_weight);
  IFN_CHECK_ALIGN16(rope_table);
  const DecodePrep pp{q, k, v, q_norm_weight, k_norm_weight, rope_table, positions, max_positions, eps};
  // the fp32 query stands in for the fp16 one, which this variant does not read
  return decode_entry(out, q, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens, active_mask,
                      batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale, workspace,
                      workspace_bytes, stream, DecodeAppend{nullptr, nullptr, slot_mapping, static_cast<f16*>(kv_pool_layer)},
                      false, plan, plan_bytes, &pp, build_plan);
}

}  // namespace ifn

extern "C" int ifn_paged_decode_prep_append(void* out, const float* q, const float* k, const float* v,
                                            const float* q_norm_weight, const float* k_norm_weight,
                                            const float* rope_table, int32_t max_positions,
                                            const int32_t* positions, const int32_t* slot_mapping,
                                            void* kv_pool_layer, int64_t num_pages, const int32_t* block_tables,
                                            int32_t max_pages_per_seq, const int32_t* seq_lens,
                                            const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                                            int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                            int32_t max_seq_len, float scale, float eps, const void* plan,
                                            size_t plan_bytes, void* workspace, size_t workspace_bytes,
                                            void* stream) {
  return ifn::prep_append_entry(out, q, k, v, q_norm_weight, k_norm_weight, rope_table, max_positions, positions,
                                slot_mapping, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                                active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len,
                                scale, eps, plan, plan_bytes, workspace, workspace_bytes, stream, false);
}

extern "C" int ifn_paged_decode_prep_append_planning(void* out, const float* q, const float* k, const float* v,
                                                     const float* q_norm_weight, const float* k_norm_weight,
                                                     const float* rope_table, int32_t max_positions,
                                                     const int32_t* positions, const int32_t* slot_mapping,
                                                     void* kv_pool_layer, int64_t num_pages,
                                                     const int32_t* block_tables, int32_t max_pages_per_seq,
                                                     const int32_t* seq_lens, const uint8_t* active_mask,
                                                     int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                                     int32_t head_dim, int32_t block_size, int32_t max_seq_len,
                                                     float scale, float eps, void* plan, size_t plan_bytes,
                                                     void* workspace, size_t workspace_bytes, void* stream) {
  return ifn::prep_append_entry(out, q, k, v, q_norm_weight, k_norm_weight, rope_table, max_positions, positions,
                                slot_mapping, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                                active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len,
                                scale, eps, plan, plan_bytes, workspace, workspace_bytes, stream, true);
}

namespace ifn {

// Workspace of the shared-prefix entry: [tickets][decode partials][states].  The partials region
// fits either decode kernel's (the per-segment kernel's, or the whole-row kernel's with one
// workgroup per `waves / kWavesPerBlock`).  The states are
// nstates = (prefix key splits + 1) per (segment, head): the prefix pass writes the first
// nstates - 1, the decode kernel the last.  The tickets are the same kTicketBytes at offset 0 as in
// every other entry point (the prefix pass and the combine take none), so one workspace zeroed
// once serves all entry points in any order.
struct SharedLayout {
  int nstates;
  size_t dec_ml, dec_o, st_ml, st_o, bytes;
};

static SharedLayout shared_layout(int32_t batch, int32_t hkv, int32_t g, int32_t d, int64_t waves,
                                  int32_t key_len, int cus) {
  SharedLayout L;
  size_t off_ml, off_o;
  const size_t dec = std::max(decode_ws_layout(batch, hkv, g, d, waves, &off_ml, &off_o),
                              rows_decode_ws_bytes(batch, hkv * g, d, int(waves / kWavesPerBlock)));
  L.nstates = prefix_pass_splits(batch, hkv * g, hkv, d, key_len, cus) + 1;  // <= kMaxStates
  const size_t states = size_t(batch) * hkv * L.nstates * g;
  L.dec_ml = off_ml;
  L.dec_o = off_o;
  L.st_ml = dec;
  L.st_o = align256(L.st_ml + states * 2 * sizeof(float));
  L.bytes = align256(L.st_o + states * d * sizeof(float));
  return L;
}

}  // namespace ifn

extern "C" size_t ifn_paged_decode_shared_prefix_workspace_bytes(int32_t batch, int32_t num_q_heads,
                                                                 int32_t num_kv_heads, int32_t head_dim,
                                                                 int32_t block_size, int32_t shared_pages) {
  if (batch < 1 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 || block_size < 1 || shared_pages < 0 ||
      num_q_heads % num_kv_heads != 0)
    return 0;
  int cus = ifn::device_cu_count();
  if (cus < 1) cus = 256;
  const int blocks = ifn::decode_blocks();
  const size_t shared = ifn::shared_layout(batch, num_kv_heads, num_q_heads / num_kv_heads, head_dim,
                                           int64_t(blocks) * ifn::kWavesPerBlock, shared_pages * block_size, cus)
                            .bytes;
  // shared_pages == 0 runs the plain decode (whole-row kernel where compiled)
  const size_t rows = ifn::rows_decode_ws_bytes(batch, num_q_heads, head_dim, blocks);
  return shared > rows ? shared : rows;
}

namespace ifn {

static int shared_prefix_entry(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                               const int32_t* prefix_pages, int32_t shared_pages, const int32_t* block_tables,
                               int32_t max_pages_per_seq, const int32_t* seq_lens, const uint8_t* active_mask,
                               int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t block_size, int32_t max_seq_len, float scale, const void* plan,
                               size_t plan_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  if (shared_pages == 0)  // no common leading run: plain decode with cached page loads
    return decode_entry(out, query, kv_pool_layer, num_pages, block_tables, max_pages_per_seq, seq_lens,
                        active_mask, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, scale,
                        workspace, workspace_bytes, stream, DecodeAppend{nullptr, nullptr, nullptr, nullptr}, true,
                        plan, plan_bytes);
  if (out == nullptr || query == nullptr || kv_pool_layer == nullptr || block_tables == nullptr ||
      seq_lens == nullptr || prefix_pages == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (batch < 0 || num_pages < 1 || max_pages_per_seq < 1 || num_q_heads < 1 || num_kv_heads < 1 ||
      head_dim < 1 || max_seq_len < 0 || num_q_heads % num_kv_heads != 0 || shared_pages < 0 ||
      shared_pages > max_pages_per_seq)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size != kBlock) return IFN_ERR_UNSUPPORTED;
  if (batch > kMaxBatch || int64_t(batch) * num_kv_heads > kMaxTickets) return IFN_ERR_UNSUPPORTED;
  const int g = num_q_heads / num_kv_heads;
  // the private pages on the whole-row kernel where it compiles the shape, else per segment
  const bool rows = rows_decode_supported(batch, num_q_heads, num_kv_heads, head_dim, max_pages_per_seq, max_seq_len);
  DecodeKernel k = rows ? nullptr : pick_decode(head_dim, g, DecodeMode::kCascade);
  CombineKernel kc = pick_combine(head_dim);
  if ((!rows && k == nullptr) || kc == nullptr) return IFN_ERR_UNSUPPORTED;
  if (!wide_prefill_supported(num_q_heads, num_kv_heads, head_dim)) return IFN_ERR_UNSUPPORTED;  // prefix pass
  IFN_CHECK_ALIGN16(out);
  IFN_CHECK_ALIGN16(query);
  IFN_CHECK_ALIGN16(kv_pool_layer);
  if (batch == 0) return IFN_OK;
  const int cus = device_cu_count();
  if (cus < 1) return IFN_ERR_HIP;
  const int blocks = decode_blocks();
  const int32_t key_len = shared_pages * kBlock;
  const SharedLayout L = shared_layout(batch, num_kv_heads, g, head_dim, int64_t(blocks) * kWavesPerBlock,
                                      key_len, cus);
  if (L.nstates > kMaxStates) return IFN_ERR_UNSUPPORTED;  // the combine merges at most kMaxStates
  if (workspace == nullptr || workspace_bytes < L.bytes) return IFN_ERR_WORKSPACE;
  IFN_CHECK_ALIGN16(workspace);
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  // (the whole-row kernel takes the prefix outputs as O / l in fp16, in the same region)
  const DecodePrefix px{reinterpret_cast<float*>(wsb + L.st_ml), reinterpret_cast<float*>(wsb + L.st_o),
                        shared_pages, L.nstates, rows ? reinterpret_cast<const f16*>(wsb + L.st_o) : nullptr};
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (rows) {  // one launch where it is built for the shape (the step plan is then not used)
    const int rc = shared_prefix_fused_launch(
        static_cast<f16*>(out), static_cast<const f16*>(query), static_cast<const f16*>(kv_pool_layer), num_pages,
        prefix_pages, block_tables, max_pages_per_seq, seq_lens, active_mask, batch, num_q_heads, num_kv_heads,
        head_dim, max_seq_len, scale * kLog2e, workspace, blocks, px, L.nstates, cus, s);
    if (rc != IFN_ERR_UNSUPPORTED) return rc;
  }
  // 1. every row's queries against the shared pages, once (states 0 .. nstates - 2)
  int rc = prefix_pass(static_cast<const f16*>(query), static_cast<const f16*>(kv_pool_layer), num_pages,
                       prefix_pages, key_len, batch, num_q_heads, num_kv_heads, head_dim, scale * kLog2e, px.ml,
                       px.o, const_cast<f16*>(px.oh), L.nstates, cus, s);
  if (rc != IFN_OK) return rc;
  // 2. the private pages.  Whole-row kernel: each cascade row's own keys merged with its prefix
  // states, to fp16.  Per-segment kernel: its state goes to state nstates - 1 (other rows are
  // written directly), merged by the combine below.
  if (rows) {
    if (plan != nullptr) {  // the kernel reads this workgroup's record before checking the header
      if (plan_bytes < rows_plan_bytes(batch, blocks)) return IFN_ERR_WORKSPACE;
      IFN_CHECK_ALIGN16(plan);
    }
    rc = rows_decode_launch(static_cast<f16*>(out), static_cast<const f16*>(query),
                            static_cast<const f16*>(kv_pool_layer), num_pages, block_tables, max_pages_per_seq,
                            seq_lens, active_mask, batch, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                            scale * kLog2e, workspace, blocks, DecodeAppend{nullptr, nullptr, nullptr, nullptr}, false,
                            static_cast<const int32_t*>(plan), s, nullptr, &px);
  } else {
    DecodeWorkspace ws;
    ws.count = reinterpret_cast<uint32_t*>(wsb);
    ws.ml = reinterpret_cast<float*>(wsb + L.dec_ml);
    ws.o = reinterpret_cast<float*>(wsb + L.dec_o);
    k<<<dim3(unsigned(blocks)), dim3(kDecodeThreads), 0, s>>>(
        static_cast<f16*>(out), static_cast<const f16*>(query), static_cast<const f16*>(kv_pool_layer), num_pages,
        block_tables, max_pages_per_seq, seq_lens, active_mask, batch, num_kv_heads, max_seq_len, scale * kLog2e, ws,
        px, DecodeAppend{nullptr, nullptr, nullptr, nullptr});
    rc = ifn_launch_status();
  }
  if (rc != IFN_OK) return rc;
  if (rows) return IFN_OK;  // the whole-row kernel merged the prefix states itself
  // 3. merge the states of every cascade segment into the output
  const int64_t segs = int64_t(batch) * num_kv_heads;
  const int32_t cap = int32_t(std::min<int64_t>(int64_t(max_pages_per_seq) * kBlock, max_seq_len));
  kc<<<dim3(unsigned(segs * g)), dim3(kWave), 0, s>>>(
      static_cast<f16*>(out), seq_lens, active_mask, batch, num_kv_heads, g, cap, px);
  return ifn_launch_status();
}

}  // namespace ifn

extern "C" int ifn_paged_decode_shared_prefix(void* out, const void* query, const void* kv_pool_layer,
                                              int64_t num_pages, const int32_t* prefix_pages, int32_t shared_pages,
                                              const int32_t* block_tables, int32_t max_pages_per_seq,
                                              const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                                              int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                              int32_t block_size, int32_t max_seq_len, float scale, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  return ifn::shared_prefix_entry(out, query, kv_pool_layer, num_pages, prefix_pages, shared_pages, block_tables,
                                  max_pages_per_seq, seq_lens, active_mask, batch, num_q_heads, num_kv_heads,
                                  head_dim, block_size, max_seq_len, scale, nullptr, 0, workspace, workspace_bytes,
                                  stream);
}

extern "C" int ifn_paged_decode_shared_prefix_planned(void* out, const void* query, const void* kv_pool_layer,
                                                      int64_t num_pages, const int32_t* prefix_pages,
                                                      int32_t shared_pages, const int32_t* block_tables,
                                                      int32_t max_pages_per_seq, const int32_t* seq_lens,
                                                      const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                                                      int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                                      int32_t max_seq_len, float scale, const void* plan,
                                                      size_t plan_bytes, void* workspace, size_t workspace_bytes,
                                                      void* stream) {
  return ifn::shared_prefix_entry(out, query, kv_pool_layer, num_pages, prefix_pages, shared_pages, block_tables,
                                  max_pages_per_seq, seq_lens, active_mask, batch, num_q_heads, num_kv_heads,
                                  head_dim, block_size, max_seq_len, scale, plan, plan_bytes, workspace,
                                  workspace_bytes, stream);
}

extern "C" int ifn_paged_decode_shared_prefix_plan(void* plan, size_t plan_bytes, const int32_t* block_tables,
                                                   int32_t max_pages_per_seq, const int32_t* seq_lens,
                                                   const uint8_t* active_mask, int32_t shared_pages,
                                                   int64_t num_pages, int32_t batch, int32_t num_q_heads,
                                                   int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                                   int32_t max_seq_len, void* stream) {
  using namespace ifn;
  if (block_tables == nullptr || seq_lens == nullptr) return IFN_ERR_INVALID_ARGUMENT;
  if (batch < 0 || num_pages < 1 || max_pages_per_seq < 1 || num_q_heads < 1 || num_kv_heads < 1 || head_dim < 1 ||
      max_seq_len < 0 || num_q_heads % num_kv_heads != 0 || shared_pages < 0 || shared_pages > max_pages_per_seq)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size < 1) return IFN_ERR_INVALID_ARGUMENT;
  if (batch == 0) return IFN_OK;
  if (block_size != kBlock) return IFN_ERR_UNSUPPORTED;
  if (!rows_decode_supported(batch, num_q_heads, num_kv_heads, head_dim, max_pages_per_seq, max_seq_len, block_size))
    return IFN_OK;  // these shapes decode without a plan
  const int blocks = decode_blocks();
  if (plan == nullptr || plan_bytes < rows_plan_bytes(batch, blocks)) return IFN_ERR_WORKSPACE;
  IFN_CHECK_ALIGN16(plan);
  if (device_cu_count() < 1) return IFN_ERR_HIP;
  return rows_plan_launch(static_cast<int32_t*>(plan), block_tables, max_pages_per_seq, seq_lens, active_mask, nullptr,
                          num_pages, batch, max_seq_len, blocks, reinterpret_cast<hipStream_t>(stream), block_size,
                          shared_pages * block_size);
}
