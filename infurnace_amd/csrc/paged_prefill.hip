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
//  * Workgroup = (block of 32 queries, kv head), over every key the block can
//    see; when those pairs cannot cover the CUs, up to kMaxSplit workgroups
//    share a pair's key tiles (interleaved) and the last to finish merges
//    their partials through the workspace.  The waves are G query heads x
//    kGroups key groups: group k takes the 32-key tiles t = k, k + kGroups,
//    ... of its workgroup (interleaved, so the causal diagonal costs every
//    group the same), and the G waves of a group share each K/V tile staged
//    in LDS.  At the end the groups merge log-sum-exp style through LDS, each
//    wave finishing its own share of the head dims.
//  * Tiles are double-buffered in LDS with one register stage: step i first
//    moves tile i+1 from registers to the other LDS buffer and issues tile
//    i+2's 16-byte global loads, then multiplies tile i.  A tile's K and V^T
//    fragments are read from LDS in one batch each, ahead of the MFMAs that
//    use them.  Page ids come from a lane window (two per tile), so no load
//    waits on a table load.
//    Only the G waves of a key group share its tiles, so they synchronise
//    through a per-group count in LDS instead of a workgroup barrier.
//  * Workgroup i runs on XCD i % 8; the kv head is i % Hkv, so for Hkv = 8
//    each XCD serves one head and its K/V stay in that XCD's L2.
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
//    stored as it is in the pool, [key][d], and the A operand (4 keys x 1 dim per
//    lane, twice) comes from two transposing LDS reads (ds_read_b64_tr_b16).
//  * K/V rows are gathered page by page through the block table; keys at or
//    past the end of the sequence or in an invalid page are zero-filled and
//    masked.
#include "ifn_common.hpp"

namespace ifn {

constexpr int kPBlock = 16;  // tokens per page compiled in
constexpr int kMaxSplit = 16;  // workgroups per (query block, kv head) at most




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

struct PrefillPlan {
  int64_t n_qb;
  int nsplit;
  size_t ml_bytes, o_bytes;  // key-split partial arrays
  size_t off_ml, off_o, bytes;
};

// Key split: enough workgroups to cover the CUs when (query blocks x kv heads) alone does not,
// provided every split still gets at least two tiles per key group.
static PrefillPlan plan_prefill(int32_t T, int32_t query_start, int32_t hq, int32_t hkv, int32_t d, int cus,
                                int32_t key_len = 0) {
  PrefillPlan p;
  const int g = hq / hkv;
  const int groups = g >= 8 ? 1 : (g >= 4 ? 2 : 4);
  p.n_qb = (int64_t(T) + 31) / 32;
  const int64_t units = p.n_qb * hkv;
  const int64_t max_tiles = ((key_len > 0 ? int64_t(key_len) : int64_t(query_start) + T) + 31) / 32;
  int ns = 1;
  while (ns < kMaxSplit && units * ns * 2 <= cus && max_tiles >= int64_t(2 * ns) * 2 * groups) ns *= 2;
  if (units * g > kMaxTickets) ns = 1;
  p.nsplit = ns;
  const size_t slots = size_t(units) * g * ns;
  p.ml_bytes = (slots * 64 * 2 * sizeof(float) + 255) & ~size_t(255);
  p.o_bytes = (slots * size_t(d) / 32 * 16 * 64 * sizeof(float) + 255) & ~size_t(255);
  p.off_ml = kTicketBytes;
  p.off_o = p.off_ml + p.ml_bytes;
  p.bytes = ns > 1 ? p.off_o + p.o_bytes : 256;
  return p;
}
constexpr int kPT = 32;      // keys per tile (one 32x32 MFMA tile)

template <int D, int G>
struct PrefillCfg {
  static constexpr int kGroups = G >= 8 ? 1 : (G >= 4 ? 2 : 4);  // key groups per workgroup
  static constexpr int kWaves = G * kGroups;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kGroupThreads = G * kWave;
  static constexpr int kKS = D + 8;    // K tile row stride (halves)
  // V row stride (halves): 32 bytes past a multiple of 128 bytes, so the 4 rows one 16-lane group
  // reads in a transposing load sit on disjoint banks
  static constexpr int kVS = D + 16;
  static constexpr int kBufHalves = kPT * kKS + kPT * kVS;  // one (group, buffer): K tile + V tile
  static constexpr int kTileBytes = 2 * kGroups * kBufHalves * 2;
  static constexpr int kDT = D / 32;
  // merge area: (m, l) of every wave, then the accumulators of groups 1.. (lane-contiguous)
  static constexpr int kMergeBytes = kWaves * 32 * 2 * 4 + (kGroups - 1) * G * kDT * 16 * kWave * 4;
  static constexpr int kLdsBytes = kTileBytes > kMergeBytes ? kTileBytes : kMergeBytes;
  static constexpr int kKItems = kPT * (D / 8);        // 16-byte K chunks per tile
  static constexpr int kKPer = (kKItems + kGroupThreads - 1) / kGroupThreads;
};

template <int D, int G, bool kAppend>
__global__ __launch_bounds__((PrefillCfg<D, G>::kThreads)) void paged_prefill_kernel(
    f16* __restrict__ out, const f16* __restrict__ q, const f16* __restrict__ pool,
    int64_t num_pages, const int32_t* __restrict__ table, int32_t query_start, int32_t T,
    int32_t num_kv_heads, int32_t n_qb, int32_t nsplit, float scale_log2, PrefillWorkspace ws, PrefixOut px,
    PrefillAppend ap) {
  using C = PrefillCfg<D, G>;
  constexpr int kDT = C::kDT;
  constexpr int kKSteps = D / 16;
  constexpr int kChunks = D / 8;
  // Workgroup i runs on XCD i % 8: kv head = i % Hkv keeps each head's K/V in one XCD's L2
  // (for Hkv = 8), and query blocks go longest key range first.
  // The nsplit workgroups of one (query block, kv head) take interleaved key tiles and merge
  // through the workspace at the end.
  const int kvh = int(blockIdx.x) % num_kv_heads;
  const int split = (int(blockIdx.x) / num_kv_heads) % nsplit;
  const int qb = n_qb - 1 - int(blockIdx.x) / (num_kv_heads * nsplit);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  // Waves w and w + 4 share a SIMD, whose issue arbitration favours the older one: with key group k
  // made of waves G*k .. G*k + G - 1, groups 0 and 1 (waves 0-3) finished their tiles about 2 us
  // before groups 2 and 3 at config 3.  So every key group takes as many older as younger waves
  // (G = 2: waves w and 7 - w; G = 4: waves {0, 2, 5, 7} and {1, 3, 4, 6}), each SIMD still
  // hosting two different groups; the groups then keep the same pace (config 3: 1-3% faster,
  // same output).
  const int hw = wave & 3, young = wave >> 2;
  constexpr bool kMix = C::kWaves == 8 && C::kGroups > 1;
  const int grp = !kMix ? wave / G : (G == 2 ? (young ? 3 - hw : hw) : ((hw + young) & 1));
  const int g = !kMix ? wave % G : (G == 2 ? young : 2 * young + (hw >> 1));
  const int gt = g * kWave + lane;  // thread index inside the key group
  const int hq = num_kv_heads * G;
  const int head = kvh * G + g;
  const bool prefix_mode = px.key_len > 0;
  const int total = prefix_mode ? px.key_len : query_start + T;  // keys that exist
  const int q0 = qb * 32;
  // keys some query of the block sees, and the position of the block's first query
  const int key_end = prefix_mode ? total : min(total, query_start + q0 + 32);
  const int min_pos = prefix_mode ? total - 1 : query_start + q0;
  const int n_tiles = int(ceil_div(key_end, kPT));
  // tile of iteration i for this wave's key group: (i * nsplit + split) * kGroups + grp
  auto tile_of = [&](int i) { return (i * nsplit + split) * C::kGroups + grp; };
  const int first = split * C::kGroups;  // first tile of this workgroup (group 0)
  const int iters = n_tiles > first ? int(ceil_div(n_tiles - first, C::kGroups * nsplit)) : 0;

  const int col = lane % 32;  // this lane's query column / K row within a tile
  const int half = lane / 32;
  const int my_q = q0 + col;
  const int my_pos = prefix_mode ? total - 1 : query_start + my_q;
  const bool q_ok = my_q < T;

  f16x8 qreg[kKSteps];
#pragma unroll
  for (int s = 0; s < kKSteps; ++s) {
    if (q_ok)
      qreg[s] = as_h8(ld16(q + (int64_t(my_q) * hq + head) * D + 16 * s + 8 * half));
    else
      qreg[s] = f16x8{};
  }

  __shared__ __attribute__((aligned(16))) unsigned char smem[C::kLdsBytes];
  auto k_tile = [&](int buf) {
    return reinterpret_cast<f16*>(smem) + (buf * C::kGroups + grp) * C::kBufHalves;
  };
  auto v_tile = [&](int buf) { return k_tile(buf) + kPT * C::kKS; };

  const int64_t tok_stride = int64_t(num_kv_heads) * D;
  const int64_t v_off = num_pages * kPBlock * tok_stride;
  const f16* head_pool = pool + int64_t(kvh) * D;

  // Fused append: 16-byte chunks of the chunk's K and V rows, spread over the grid, stored at
  // table[pos / 16] * 16 + pos % 16 (skipped when that page id is outside the pool).
  if constexpr (kAppend)
    store_chunk_rows(ap.pool, num_pages, table, query_start, T, num_kv_heads, D, ap.new_k, ap.new_v,
                     int64_t(blockIdx.x) * C::kThreads + tid, int64_t(gridDim.x) * C::kThreads);
  // Page ids: a tile of 32 keys spans exactly two pages.  Lane l of every wave of the group
  // holds page 2*tile + (l & 1) of the group's (l / 2)-th upcoming tile, 32 tiles per window,
  // so a tile's two ids are uniform v_readlane reads -- no dependent table load per tile.
  const int seq_pages = int(ceil_div(total, kPBlock));
  int pid = -1, pid_w = -1;
  auto tile_pages = [&](int i, int& pa, int& pb) __attribute__((always_inline)) {  // pages of the group's tile of iteration i
    if ((i >> 5) != pid_w) {
      pid_w = i >> 5;
      const int pg = 2 * tile_of(32 * pid_w + lane / 2) + (lane & 1);
      const int id = table[min(pg, seq_pages - 1)];
      pid = pg < seq_pages ? id : -1;
      // Complete the window load here: otherwise the wait for it lands on the v_readlane
      // below, on every iteration, and drains the tile prefetch each time.
      asm volatile("" ::"v"(pid));
    }
    pa = __builtin_amdgcn_readlane(pid, 2 * (i & 31));
    pb = __builtin_amdgcn_readlane(pid, 2 * (i & 31) + 1);
  };

  // Per-thread constants of the tile copy: which page half, the element offset inside the page
  // and the LDS offset of each item (the same for every tile).
  // K and V items: 16 bytes (8 dims) of one key row; V uses the K item's row and chunk
  int k_goff[C::kKPer], k_loff[C::kKPer], v_loff[C::kKPer], k_key[C::kKPer];
  bool k_hi[C::kKPer];
#pragma unroll
  for (int it = 0; it < C::kKPer; ++it) {
    const int idx = min(gt + it * C::kGroupThreads, C::kKItems - 1);
    const int j = idx / kChunks, c = idx % kChunks;
    k_hi[it] = j >= kPBlock;
    k_key[it] = j;
    k_goff[it] = (j % kPBlock) * int(tok_stride) + c * 8;
    k_loff[it] = j * C::kKS + c * 8;
    v_loff[it] = j * C::kVS + c * 8;
  }
  const int64_t page_elems = int64_t(kPBlock) * tok_stride;

  // Tile flags (uniform): bit 0/1 = first/second page valid, bit 2 = every key of the tile is
  // visible to every query of the block (no mask, no zero fill).
  auto tile_flags = [&](int i, int pa, int pb) __attribute__((always_inline)) -> int {
    const int kt = tile_of(i) * kPT;
    const int oka = pa >= 0 && int64_t(pa) < num_pages, okb = pb >= 0 && int64_t(pb) < num_pages;
    const int full = oka && okb && kt + kPT <= total && kt + kPT - 1 <= min_pos;
    return oka | (okb << 1) | (full << 2);
  };

  // Fused append: buffer resources over the chunk's rows (num_records = T rows; gfx9 format word).
  const int rsrc_bytes = kAppend ? T * int(tok_stride) * 2 : 0;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(ap.new_k), 0, rsrc_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(ap.new_v), 0, rsrc_bytes, 0x00020000);

  struct Stage {
    u32x4 k[C::kKPer];
    u32x4 v[C::kKPer];
    int flags;
  };
  // Global -> registers: this thread's share of the tile.  Every address is a real row (an
  // invalid page reads page 0); masked keys are dealt with in store_tile / compute_tile.
  auto load_tile = [&](int i, Stage& st) __attribute__((always_inline)) {
    int pa, pb;
    tile_pages(i, pa, pb);
    st.flags = tile_flags(i, pa, pb);
    const f16* base_a = head_pool + int64_t((st.flags & 1) ? pa : 0) * page_elems;
    const f16* base_b = head_pool + int64_t((st.flags & 2) ? pb : 0) * page_elems;
    if constexpr (kAppend) {
      const int kt = tile_of(i) * kPT;
      if (kt >= query_start) {  // (uniform; query_start % 32 == 0) every key of the tile is a chunk key
        // Buffer loads from new_k / new_v: rows past the chunk's end fall outside the resource and
        // read as zero (their keys are masked), so no address is ever out of bounds.  The whole
        // byte offset goes in the per-lane operand, which is the one the range check covers.
        const int so = (int(kt - query_start) * int(tok_stride) + kvh * D) * 2;  // bytes, uniform
#pragma unroll
        for (int it = 0; it < C::kKPer; ++it) {
          const int vo = (k_goff[it] + (k_hi[it] ? kPBlock * int(tok_stride) : 0)) * 2;
          st.k[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, so + vo, 0, 0));
          st.v[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, so + vo, 0, 0));
        }
        return;
      }
    }
#pragma unroll
    for (int it = 0; it < C::kKPer; ++it) {
      const f16* src = (k_hi[it] ? base_b : base_a) + k_goff[it];
      st.k[it] = ld16(src);
      st.v[it] = ld16(src + v_off);
    }
  };
  auto store_tile = [&](int i, int buf, Stage& st) __attribute__((always_inline)) {  // registers -> LDS
    f16* ks = k_tile(buf);
    f16* vs = v_tile(buf);
    if (!(st.flags & 4)) {  // zero V rows of keys past the end or in an invalid page (K is masked)
      const int kt = tile_of(i) * kPT;
#pragma unroll
      for (int it = 0; it < C::kKPer; ++it) {
        const int key = k_key[it];
        const bool ok = ((st.flags >> (key >= kPBlock ? 1 : 0)) & 1) && kt + key < total;
        st.v[it] = ok ? st.v[it] : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int it = 0; it < C::kKPer; ++it)
      if (gt + it * C::kGroupThreads < C::kKItems) {
        *reinterpret_cast<u32x4*>(ks + k_loff[it]) = st.k[it];
        *reinterpret_cast<u32x4*>(vs + v_loff[it]) = st.v[it];
      }
  };

  // transposing V reads: lane = 16 g + 4 r + q reads key row 4 (lane / 32) + r, dims 16 (g % 2) + 4 q
  const int tr_off = (4 * half + (lane % 16) / 4) * C::kVS + 16 * ((lane / 16) % 2) + 4 * (lane % 4);

  float m = kNegBig, lsum = 0.f;
  f32x16 acc[kDT];
#pragma unroll
  for (int dt = 0; dt < kDT; ++dt) acc[dt] = f32x16{};

  auto compute_tile = [&](int i, int buf, int flags) __attribute__((always_inline)) {
    const int kt = tile_of(i) * kPT;
    const f16* ks = k_tile(buf);
    const f16* vt = v_tile(buf);
    // All K fragments, then the S MFMAs; the V^T fragments are requested right behind them, so
    // their LDS latency runs under the softmax.  (The scheduling barriers keep that order.)
    f32x16 st = f32x16{};
    f16x8 kf[kKSteps];
#pragma unroll
    for (int s = 0; s < kKSteps; ++s) kf[s] = *reinterpret_cast<const f16x8*>(ks + col * C::kKS + 16 * s + 8 * half);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kKSteps; ++s) st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[s], qreg[s], st, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    // A = V^T for dims 32 dt + col, keys 16 u + 4 half + 0..3 (lo) and 16 u + 8 + 4 half + 0..3 (hi):
    // in each 16-lane group, lane 4r + q reads 4 dims of key row r and the read hands lane i dim i
    // of the 4 rows
    f16x4 vlo[kDT][2], vhi[kDT][2];
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f16* vp = vt + tr_off + 16 * u * C::kVS + 32 * dt;
        vlo[dt][u] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                   (__attribute__((address_space(3))) v4i16*)(vp)));
        vhi[dt][u] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                   (__attribute__((address_space(3))) v4i16*)(vp + 8 * C::kVS)));
      }
    __builtin_amdgcn_sched_barrier(0);
    // causal mask (key_pos <= query_pos), end of sequence and invalid pages -- only on tiles
    // that are not entirely visible; raw scores, the scale is folded into the exponent below
    if (!(flags & 4)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = 8 * (r / 4) + 4 * half + (r % 4);
        const bool ok = ((flags >> (kk >= kPBlock ? 1 : 0)) & 1) && kt + kk <= my_pos && kt + kk < total;
        st[r] = ok ? st[r] : -INFINITY;
      }
    }
    float mx = st[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, st[r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // Lazy rescale: the reference m moves only when a score exceeds it by more than kSlack
    // (log2 units), so P = 2^(s - m) stays below 2^kSlack and the 16-per-lane accumulator
    // rescale runs on a few tiles instead of most of them.  acc and lsum stay relative to m, so
    // the normalised result is unchanged.
    constexpr float kSlack = 8.f;
    const float cand = mx * scale_log2;
    const bool grow = cand > m + kSlack;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float mn = grow ? cand : m;
      const float alpha = exp2_fast(m - mn);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < kDT; ++dt) acc[dt] *= alpha;
      m = mn;
    }
    float pv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pv[r] = exp2_fast(fmaf(st[r], scale_log2, -m));
      lsum += pv[r];
    }
    // built by value: element-wise writes into a local vector array end up in scratch
    const f16x8 pb[2] = {
        f16x8{f16(pv[0]), f16(pv[1]), f16(pv[2]), f16(pv[3]), f16(pv[4]), f16(pv[5]), f16(pv[6]), f16(pv[7])},
        f16x8{f16(pv[8]), f16(pv[9]), f16(pv[10]), f16(pv[11]), f16(pv[12]), f16(pv[13]), f16(pv[14]),
              f16(pv[15])}};
    // O^T += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f16x4 lo = vlo[dt][u], hi = vhi[dt][u];
        const f16x8 a = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[u], acc[dt], 0, 0, 0);
      }
  };

  // Sweep: step i multiplies the group's tile i*kGroups + grp from LDS buffer i&1.  It first
  // stores tile i+1 (in registers since step i-1) into buffer (i+1)&1 and issues tile i+2's
  // loads into the same register stage, so a tile's loads have one step to arrive.  Against two
  // register stages (tile i+1 stored after the multiply) this measured the same at config 3
  // (81.6 us per layer) and 1.5% faster fused (86.9 against 88.3 us), with 9 fewer registers.
  auto has = [&](int i) __attribute__((always_inline)) { return i < iters && tile_of(i) < n_tiles; };
  Stage s0;
  s0.flags = 0;
  // Loads are unconditional (tiles past the end read page 0 and are never used), so every
  // iteration waits for a fixed number of loads.
  load_tile(0, s0);
#pragma unroll
  for (int st = 0; st < kKSteps; ++st) asm volatile("" ::"v"(qreg[st]));  // query loads done before the loop
  // Per key group synchronisation: a group's G waves share its tiles and nothing else, so instead of
  // a workgroup barrier per iteration each wave counts its finished steps in LDS (release) and
  // waits for its group's count before the next step (acquire).  After the wait, every wave of the
  // group has stored tile i and finished multiplying tile i-1, whose buffer tile i+1 reuses; no
  // wave runs more than one step ahead of its group.  The wait is bounded (a safety net: the
  // waves of a group run the same number of steps, so the count always arrives).  The
  // config-3 prefill measured 82.6 us per layer this way against 85.5 us with a workgroup
  // barrier per iteration.
  __shared__ int s_grp_cnt[C::kGroups];
  if (tid < C::kGroups) s_grp_cnt[tid] = 0;
  if (has(0)) store_tile(0, 0, s0);
  int cur_flags = s0.flags;
  load_tile(1, s0);
  __syncthreads();
  // Returns false when the count did not arrive within the bound (never expected): the wave
  // then skips that tile's arithmetic -- it does not multiply a tile that may not be stored --
  // keeps counting its steps so that the rest of its group is not held up, and raises the
  // workspace's error flag, which the caller's validate mode reports.
  auto group_wait = [&](int target) __attribute__((always_inline)) -> bool {
    for (int spins = 0; spins < (1 << 20); ++spins) {
      if (__hip_atomic_load(&s_grp_cnt[grp], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return true;
      __builtin_amdgcn_s_sleep(1);
    }
    return false;
  };
  bool wait_failed = false;
  for (int i = 0; i < iters; ++i) {
    const int fl = cur_flags;
    const bool ready = i == 0 || group_wait(G * i);  // every wave of the group has finished step i - 1
    wait_failed |= !ready;
    if (has(i + 1)) store_tile(i + 1, (i + 1) & 1, s0);
    cur_flags = s0.flags;
    load_tile(i + 2, s0);
    if (has(i) && ready) compute_tile(i, i & 1, fl);
    if (lane == 0) __hip_atomic_fetch_add(&s_grp_cnt[grp], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (wait_failed && lane == 0 && ws.count != nullptr) raise_error_flag(ws.count);

  __syncthreads();  // every group is done with the tile buffers, which the merge area reuses
  const float ltot = lsum + __shfl_xor(lsum, 32);
  // From here on the work is spread over all waves: wave (grp, g) finishes the dims blocks dt of
  // head g with dt % kGroups == grp -- the key groups' log-sum-exp merge, the key-split merge and
  // the output stores.  (With group 0 doing all of it, the epilogue of a config-3 chunk took
  // about 5.5 us.)  The arithmetic and its order are the same as one wave doing everything.
  auto owns = [&](int dt) __attribute__((always_inline)) { return dt % C::kGroups == grp; };
  float mfin = m, lfin = ltot;
  if constexpr (C::kGroups > 1) {
    // Every wave publishes (m, l) and the blocks it does not own; LDS rows are 16 bytes per lane
    // (4 consecutive accumulator entries), 1 KB per instruction.
    float* mlb = reinterpret_cast<float*>(smem);  // [grp][g][32][2]
    f32x4* accb = reinterpret_cast<f32x4*>(mlb + C::kWaves * 32 * 2);  // [g][dt][group other than dt's owner][4][lane]
    auto blk = [&](int gg, int dt, int k, int r4) __attribute__((always_inline)) {
      const int ko = k - (k > dt % C::kGroups ? 1 : 0);
      return accb + (((gg * kDT + dt) * (C::kGroups - 1) + ko) * 4 + r4) * kWave + lane;
    };
    if (half == 0) {
      mlb[((grp * G + g) * 32 + col) * 2 + 0] = m;
      mlb[((grp * G + g) * 32 + col) * 2 + 1] = ltot;
    }
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
      if (!owns(dt))
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *blk(g, dt, grp, r4) = f32x4{acc[dt][4 * r4], acc[dt][4 * r4 + 1], acc[dt][4 * r4 + 2], acc[dt][4 * r4 + 3]};
    __syncthreads();
    float mk[C::kGroups], lk[C::kGroups];
#pragma unroll
    for (int k = 0; k < C::kGroups; ++k) {
      mk[k] = mlb[((k * G + g) * 32 + col) * 2];
      lk[k] = mlb[((k * G + g) * 32 + col) * 2 + 1];
    }
    float mxg = mk[0];
#pragma unroll
    for (int k = 1; k < C::kGroups; ++k) mxg = fmaxf(mxg, mk[k]);
    float wk[C::kGroups];
#pragma unroll
    for (int k = 0; k < C::kGroups; ++k) wk[k] = exp2_fast(mk[k] - mxg);
    float L = wk[0] * lk[0];
#pragma unroll
    for (int k = 1; k < C::kGroups; ++k) L = fmaf(wk[k], lk[k], L);
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) {
      if (!owns(dt)) continue;
      f32x16 o;
#pragma unroll
      for (int k = 0; k < C::kGroups; ++k) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          f32x4 x;
          if (k == grp)
            x = f32x4{acc[dt][4 * r4], acc[dt][4 * r4 + 1], acc[dt][4 * r4 + 2], acc[dt][4 * r4 + 3]};
          else
            x = *blk(g, dt, k, r4);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[4 * r4 + e] = k == 0 ? x[e] * wk[0] : fmaf(wk[k], x[e], o[4 * r4 + e]);
        }
      }
      acc[dt] = o;
    }
    mfin = mxg;
    lfin = L;
  }

  if (nsplit > 1 && !prefix_mode) {
    // Cross-workgroup merge: every wave publishes its blocks of this split's (m, l, O) for head g
    // with device-coherent stores (lane-contiguous); once all are acknowledged, one thread per
    // head takes the (query block, head) ticket.  The last of the nsplit arrivals combines the
    // partials of every split, its own included (read back from memory), in split order, so the
    // result does not depend on which workgroup arrived last.
    __shared__ uint32_t s_ticket[G];
    constexpr int kSlotO = kDT * 16 * kWave;  // floats of O per (pair, split)
    const int64_t pair = (int64_t(qb) * num_kv_heads + kvh) * G + g;
    const int64_t slot = pair * nsplit + split;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
      if (owns(dt))
#pragma unroll
        for (int r = 0; r < 16; ++r) st_dev(ws.o + slot * kSlotO + (dt * 16 + r) * kWave + lane, acc[dt][r]);
    if (grp == 0) {
      st_dev(ws.ml + (slot * kWave + lane) * 2 + 0, mfin);
      st_dev(ws.ml + (slot * kWave + lane) * 2 + 1, lfin);
    }
    wait_all_mem();   // this wave's stores are acknowledged
    __syncthreads();  // ... and every other wave's
    if (grp == 0 && lane == 0)
      s_ticket[g] = __hip_atomic_fetch_add(ws.count + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_ticket[g] != uint32_t(nsplit - 1)) return;
    compiler_fence();  // the merge loads below stay behind the ticket
    float mo[kMaxSplit], lo[kMaxSplit];
    float mx = kNegBig;
#pragma unroll
    for (int s2 = 0; s2 < kMaxSplit; ++s2) {
      if (s2 < nsplit) {
        mo[s2] = ld_dev(ws.ml + ((pair * nsplit + s2) * kWave + lane) * 2 + 0);
        lo[s2] = ld_dev(ws.ml + ((pair * nsplit + s2) * kWave + lane) * 2 + 1);
        mx = fmaxf(mx, mo[s2]);
      }
    }
    lfin = 0.f;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
      if (owns(dt)) acc[dt] = f32x16{};
#pragma unroll
    for (int s2 = 0; s2 < kMaxSplit; ++s2) {
      if (s2 < nsplit) {
        const float wsp = exp2_fast(mo[s2] - mx);
        lfin = fmaf(wsp, lo[s2], lfin);
        const float* so = ws.o + (pair * nsplit + s2) * kSlotO;
#pragma unroll
        for (int dt = 0; dt < kDT; ++dt)
          if (owns(dt))
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[dt][r] = fmaf(wsp, ld_dev(so + (dt * 16 + r) * kWave + lane), acc[dt][r]);
      }
    }
    mfin = mx;  // acc and lfin are now relative to the maximum over all splits
    if (grp == 0 && lane == 0) reset_ticket(ws.count + pair);
  }

  if (!q_ok) return;
  if (prefix_mode) {  // this split's unnormalised partial (row my_q, kv head kvh, head g)
    const int64_t pslot = ((int64_t(my_q) * num_kv_heads + kvh) * px.stride + split) * G + g;
    if (half == 0 && grp == 0) *reinterpret_cast<f32x2*>(px.ml + pslot * 2) = f32x2{mfin, lfin};
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
      if (owns(dt))
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)  // 4 consecutive dims per 16-byte store
          *reinterpret_cast<f32x4*>(px.o + pslot * D + 32 * dt + 8 * a4 + 4 * half) =
              f32x4{acc[dt][4 * a4], acc[dt][4 * a4 + 1], acc[dt][4 * a4 + 2], acc[dt][4 * a4 + 3]};
    return;
  }
  const float inv = lfin > 0.f ? 1.f / lfin : 0.f;
  f16* orow = out + (int64_t(my_q) * hq + head) * D;
#pragma unroll
  for (int dt = 0; dt < kDT; ++dt)
    if (owns(dt))
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int d0 = 32 * dt + 8 * a4 + 4 * half;
        *reinterpret_cast<f16x4*>(orow + d0) =
            f16x4{f16(acc[dt][4 * a4] * inv), f16(acc[dt][4 * a4 + 1] * inv),
                  f16(acc[dt][4 * a4 + 2] * inv), f16(acc[dt][4 * a4 + 3] * inv)};
      }
}

typedef void (*PrefillKernel)(f16*, const f16*, const f16*, int64_t, const int32_t*, int32_t, int32_t,
                              int32_t, int32_t, int32_t, float, PrefillWorkspace, PrefixOut, PrefillAppend);

static PrefillKernel pick_prefill(int d, int g, int* threads, bool append = false) {
#define IFN_PREFILL_CASE(DD, GG)                                                               \
  if (d == DD && g == GG) {                                                                    \
    *threads = PrefillCfg<DD, GG>::kThreads;                                                   \
    return append ? paged_prefill_kernel<DD, GG, true> : paged_prefill_kernel<DD, GG, false>;  \
  }
  IFN_PREFILL_CASE(64, 1) IFN_PREFILL_CASE(64, 2) IFN_PREFILL_CASE(64, 4) IFN_PREFILL_CASE(64, 8)
  IFN_PREFILL_CASE(128, 1) IFN_PREFILL_CASE(128, 2) IFN_PREFILL_CASE(128, 4) IFN_PREFILL_CASE(128, 8)
#undef IFN_PREFILL_CASE
  return nullptr;
}

// (the shapes the wide kernel compiles take it: wide_prefix_splits / wide_prefix_pass)
int prefix_pass_splits(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t key_len, int cus) {
  if (wide_prefill_supported(hq, hkv, d)) return wide_prefix_splits(batch, hq, hkv, d, key_len, cus);
  return plan_prefill(batch, 0, hq, hkv, d, cus, key_len).nsplit;
}

int prefix_pass(const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages, int32_t key_len,
                int32_t batch, int32_t hq, int32_t hkv, int32_t d, float scale_log2, float* px_ml, float* px_o,
                int32_t stride, int cus, hipStream_t stream) {
  if (wide_prefill_supported(hq, hkv, d))
    return wide_prefix_pass(q, pool, num_pages, prefix_pages, key_len, batch, hq, hkv, d, scale_log2, px_ml, px_o,
                            stride, cus, stream);
  int threads = 0;
  PrefillKernel k = pick_prefill(d, hq / hkv, &threads);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
  const PrefillPlan p = plan_prefill(batch, 0, hq, hkv, d, cus, key_len);
  if (p.n_qb * hkv * p.nsplit > int64_t(1) << 31 || stride < p.nsplit) return IFN_ERR_UNSUPPORTED;
  k<<<dim3(unsigned(p.n_qb * hkv * p.nsplit)), unsigned(threads), 0, stream>>>(
      nullptr, q, pool, num_pages, prefix_pages, 0, batch, hkv, int(p.n_qb), p.nsplit, scale_log2,
      PrefillWorkspace{nullptr, nullptr, nullptr}, PrefixOut{px_ml, px_o, key_len, stride},
      PrefillAppend{nullptr, nullptr, nullptr});
  return ifn_launch_status();
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
  return ifn::plan_prefill(num_q_tokens, query_start, num_q_heads, num_kv_heads, head_dim, cus).bytes;
}

namespace ifn {

static int prefill_entry(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                         const int32_t* block_table, int32_t max_pages, int32_t query_start, int32_t num_q_tokens,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         void* workspace, size_t workspace_bytes, void* stream, PrefillAppend ap) {
  bool append = ap.pool != nullptr;
  if (out == nullptr || query == nullptr || kv_pool_layer == nullptr || block_table == nullptr)
    return IFN_ERR_INVALID_ARGUMENT;
  if (append && (ap.new_k == nullptr || ap.new_v == nullptr)) return IFN_ERR_INVALID_ARGUMENT;
  if (num_pages < 1 || max_pages < 1 || query_start < 0 || num_q_tokens < 0 || num_q_heads < 1 ||
      num_kv_heads < 1 || head_dim < 1 || num_q_heads % num_kv_heads != 0)
    return IFN_ERR_INVALID_ARGUMENT;
  if (block_size != kPBlock) return IFN_ERR_UNSUPPORTED;
  int threads = 0;
  PrefillKernel k = pick_prefill(head_dim, num_q_heads / num_kv_heads, &threads, append);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
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
    append = false;
    ap = PrefillAppend{nullptr, nullptr, nullptr};
    k = pick_prefill(head_dim, num_q_heads / num_kv_heads, &threads, false);
  }
  if (scale <= 0.f) scale = 1.0f / sqrtf(float(head_dim));
  if (wide_prefill_supported(num_q_heads, num_kv_heads, head_dim))
    return wide_prefill_launch(static_cast<f16*>(out), static_cast<const f16*>(query),
                               static_cast<const f16*>(kv_pool_layer), num_pages, block_table, query_start,
                               num_q_tokens, num_q_heads, num_kv_heads, head_dim, scale * kLog2e, workspace,
                               workspace_bytes, ap, cus, reinterpret_cast<hipStream_t>(stream));
  const PrefillPlan p = plan_prefill(num_q_tokens, query_start, num_q_heads, num_kv_heads, head_dim, cus);
  if (p.n_qb * num_kv_heads * p.nsplit > int64_t(1) << 31) return IFN_ERR_UNSUPPORTED;
  PrefillWorkspace ws{nullptr, nullptr, nullptr};
  if (p.nsplit > 1) {
    if (workspace == nullptr || workspace_bytes < p.bytes) return IFN_ERR_WORKSPACE;
    IFN_CHECK_ALIGN16(workspace);
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    ws.count = reinterpret_cast<uint32_t*>(wsb);
    ws.ml = reinterpret_cast<float*>(wsb + p.off_ml);
    ws.o = reinterpret_cast<float*>(wsb + p.off_o);
  } else if (workspace != nullptr && workspace_bytes >= kTicketBytes) {
    IFN_CHECK_ALIGN16(workspace);
    ws.count = static_cast<uint32_t*>(workspace);  // no split: only the error flag is used
  }
  k<<<dim3(unsigned(p.n_qb * num_kv_heads * p.nsplit)), unsigned(threads), 0,
      reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<f16*>(out), static_cast<const f16*>(query),
      static_cast<const f16*>(kv_pool_layer), num_pages, block_table, query_start, num_q_tokens,
      num_kv_heads, int(p.n_qb), p.nsplit, scale * kLog2e, ws, PrefixOut{nullptr, nullptr, 0, 0}, ap);
  return ifn_launch_status();
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
