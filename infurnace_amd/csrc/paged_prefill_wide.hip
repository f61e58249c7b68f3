// Causal chunked-prefill paged attention with 32 or 64 query rows per wavefront (gfx950 MFMA fp16).
//
// Same operation and entry points as paged_prefill.hip (docs/architecture.md:246; contiguous
// semantics src/infurnace/executor/tinygrad/model.py:116-132: query row i sits at
// start_position + i and sees keys with key_pos <= query_pos):
//
//  * Rows.  A workgroup serves one (query block, kv head): 32 RT rows = 32 RT / G queries x the G
//    query heads of the kv head, held by every wave as RT 32-row MFMA tiles.  Its W waves are W key
//    groups: wave k takes the 32-key tiles t = k, k + W, ... (interleaved, so the causal diagonal
//    costs every group the same).  RT = 2 with W = 4 (one wave per SIMD, up to 512 registers),
//    or, when 64-row blocks would leave CUs idle, RT = 1 with W = 8 (two waves per SIMD in 256
//    registers each).  When (query blocks x kv heads) still cannot cover the CUs, up to kWMaxSplit
//    workgroups share a block's tiles and the last to finish merges their partials through the
//    workspace.
//  * Scores, transposed: S^T = K . Q^T with v_mfma_f32_32x32x16_f16.  The A operand (32 keys x 16
//    dims) is one key row per lane: K tiles are loaded from the pool row-contiguously (8 lanes per
//    128-byte line) and staged in the wave's LDS K buffer, from which each lane reads its fragments.
//    MFMA K-step s takes dims 16 s + 8 half .. + 7 (a permutation of the head dims applied to both
//    operands).  The B operand (the queries) is held for the whole kernel.
//  * O^T += V^T . P^T: the probabilities stay in registers (a lane's 16 scores of a 32-key tile are
//    the B operands of two K = 16 steps); V goes through registers to the wave's own LDS tile as it
//    is in the pool, [key][dim] (16-byte chunks XOR-swizzled by row), and the A operand comes from
//    transposing LDS reads (ds_read_b64_tr_b16).
//  * Pipeline: tile i + 1's scores are computed while tile i's probabilities are formed, and the
//    next tiles' K and V loads are spread between the MFMAs.  Keys past the end or in an invalid
//    page read zeros and are masked (only in the tiles that hold such keys).
//  * Online softmax in base 2, per lane and row tile (one lane ^ 32 exchange per tile), with the
//    lazy rescale of the running maximum (slack 2^8); row sums add the fp16 probabilities.
//  * Epilogue: the W key groups merge log-sum-exp style through LDS, each wave finishing its share
//    of the output; then the key-split merge and the fp16 stores.
//  * Fused pre-append (kPrep): the chunk's queries, keys and values arrive as fp32 projections.
//    Each wave first normalises, rotates and casts the K and V rows of the chunk tiles it will
//    read and writes them to the pool, and the workgroup prepares its own queries straight into the
//    LDS staging; the attention then runs as in the plain kernel.
#include "ifn_common.hpp"
#include "decode_rows.hpp"

namespace ifn {

constexpr int kWBlock = 16;    // tokens per page compiled in
constexpr int kWTile = 32;     // keys per tile
constexpr int kWMaxSplit = 16;

// RT row tiles of 32 query rows per wave (and per workgroup); W waves (key groups) per workgroup
template <int D, int G, int RT, int W>
struct WideCfg {
  static constexpr int kThreads = W * kWave;
  static constexpr int kRows = 32 * RT;              // query rows per workgroup
  static constexpr int kQw = kRows / G;              // queries per workgroup
  static constexpr int kKSteps = D / 16;             // MFMA K-steps over the head dims
  static constexpr int kDT = D / 32;                 // 32-dim output tiles
  static constexpr int kBlocks = RT * kDT;           // output blocks: (dim tile, row tile)
  // Each wave finishes kOwnU quarter blocks (4 accumulator rows of a block per lane): whole blocks
  // p = wave + W ob when there are at least W blocks, else a run of quarters of block wave % kBlocks.
  static constexpr int kOwnU = 4 * kBlocks / W;
  // V tile in LDS: two page halves of 16 key rows x D dims, [key][dim] as in the pool and
  // unpadded; the 16-byte chunk c of row r sits at chunk position c ^ 2 (r % 4), so the 4 rows a
  // 16-lane group reads in one transposing load fall on disjoint banks.
  static constexpr int kRowChunks = D / 8;                     // 16-byte chunks per key row
  static constexpr int kHalfInstr = 16 * kRowChunks / kWave;   // DMA instructions per page half
  static constexpr int kHalfBytes = 16 * D * 2;
  static constexpr int kVBufBytes = 2 * kHalfBytes;
  static constexpr int kVInstr = 2 * kHalfInstr;     // 16-byte loads (and LDS writes) per lane per tile
  // V tiles in LDS per wave: i and i + 1 with 4 waves; with 8 (two per SIMD, so half the LDS
  // each) one, rewritten with tile i + 1 once every read of tile i is issued
  static constexpr int kVBufs = W == 8 ? 1 : 2;
  // K tile in LDS: [chunk c][32 key rows] of 16-byte chunks, row r of chunk c at slot r ^ (c % 8),
  // so that a lane's MFMA fragment for K-step s sits at a constant offset of 1 KiB s from one of
  // four lane bases, and every 8 lanes of a 16-byte write or read (one 128-byte LDS cycle) cover
  // the 32 banks once.
  static constexpr int kKInstr = 32 * kRowChunks / kWave;  // 16-byte loads (and writes) per lane
  static constexpr int kKBufBytes = 32 * kRowChunks * 16;
  static constexpr int kWaveBytes = kVBufs * kVBufBytes + kKBufBytes;
  static constexpr int kTileBytes = W * kWaveBytes;
  // The queries, staged once per workgroup: kRows rows x D dims, chunk c of row r at c ^ (r % 8).
  static constexpr int kQBytes = kRows * D * 2;
  static constexpr int kQInstr = kQBytes / 16 / kThreads;  // 16-byte loads per lane
  static constexpr int kQRowsPerWave = kRows / W;          // rows each wave stages
  static constexpr int kMlFloats = W * RT * 32 * 2;
  static constexpr int kMergeBytes = kMlFloats * 4 + W * kBlocks * 16 * kWave * 2;  // (m, l) + O / l in fp16
  static constexpr int kLdsBytes = kTileBytes + kQBytes > kMergeBytes ? kTileBytes + kQBytes : kMergeBytes;
  static_assert(RT == 1 || RT == 2, "one or two row tiles");
  static_assert(kQw * G == kRows, "32 RT rows per workgroup");
  static_assert(W == 4 || W == 8, "4 or 8 waves");
  static_assert((4 * kBlocks) % W == 0 && (kBlocks % W == 0 || W % kBlocks == 0), "every wave finishes the same share");
  static_assert(16 * kRowChunks % kWave == 0 && kRowChunks >= 8, "whole loads per page half; swizzle in range");
  static_assert(kRowChunks % 8 == 0 && kKInstr % 2 == 0, "K loads: 8 rows x 8 chunks each, within one page half");
  static_assert(kQBytes % (16 * kThreads) == 0 && kQRowsPerWave * kRowChunks == kQInstr * kWave, "Q staging");
};

struct WidePlan {
  int64_t n_qb;
  int rt, w, nsplit;
  size_t off_ml, off_o, bytes;
};

// Row tiles per wave: two (64 rows per workgroup, every K and V fragment feeding two MFMA chains)
// unless the (query block, kv head) pairs of 64 rows would fill at most half the CUs and the key
// range is at most 512 tiles; then, for head dim 128, one (32 rows per workgroup), which doubles
// the pairs instead of splitting their keys over workgroups that merge through memory, with 8 waves
// (two per SIMD) in place of 4.  (Past 16K keys the split's fixed cost is paid back: measured at
// 512 queries, equal at 16K keys and 4% in favour of the split at 32K.)
// Key split: enough workgroups to cover the CUs when (query blocks x kv heads) alone does not,
// provided every split still gets at least two tiles per key group.
// key_len > 0: the shared-prefix pass (every row sees keys [0, key_len), query_start unused).
static WidePlan plan_wide(int32_t T, int32_t query_start, int32_t hq, int32_t hkv, int32_t d, int cus,
                          int32_t key_len = 0) {
  WidePlan p;
  const int g = hq / hkv;
  auto blocks = [&](int rows) { return (int64_t(T) + rows / g - 1) / (rows / g); };
  const int64_t max_tiles = ((key_len > 0 ? int64_t(key_len) : int64_t(query_start) + T) + kWTile - 1) / kWTile;
  p.rt = d == 128 && blocks(64) * hkv * 2 <= cus && max_tiles <= 512 ? 1 : 2;
  p.w = p.rt == 1 ? 8 : 4;
  const int rows = 32 * p.rt;
  p.n_qb = blocks(rows);
  const int64_t units = p.n_qb * hkv;
  int ns = 1;
  while (ns < kWMaxSplit && units * ns * 2 <= cus && max_tiles >= int64_t(2 * ns) * 2 * p.w) ns *= 2;
  if (units > kMaxTickets) ns = 1;
  p.nsplit = ns;
  const size_t slots = size_t(units) * ns;
  p.off_ml = kTicketBytes;
  p.off_o = p.off_ml + align256(slots * rows * 2 * sizeof(float));
  p.bytes = ns > 1 ? p.off_o + align256(slots * rows * size_t(d) * sizeof(float)) : 256;
  return p;
}

// The chunk's K and V rows -> the pool at table[pos / 16] * 16 + pos % 16, pos = query_start + t
// (16-byte chunks, grid-stride; rows whose page id is outside the pool are skipped).
__device__ __forceinline__ void wide_store_chunk(f16* __restrict__ pool, int64_t num_pages,
                                                 const int32_t* __restrict__ table, int32_t query_start, int32_t T,
                                                 int32_t hkv, int32_t d, const f16* __restrict__ new_k,
                                                 const f16* __restrict__ new_v, int first, int step) {
  const int chunks = hkv * d / 8;
  const int64_t tok_stride = int64_t(hkv) * d;
  const int items = T * 2 * chunks;  // (< 2^31: checked at launch)
  for (int it = first; it < items; it += step) {
    const int t = it / (2 * chunks);
    const int rem = it - t * 2 * chunks;
    const int kv = rem >= chunks, c = rem - kv * chunks;
    const int pos = query_start + t;
    const int page = table[pos / kWBlock];
    if (page < 0 || int64_t(page) >= num_pages) continue;
    const f16* src = (kv == 0 ? new_k : new_v) + int64_t(t) * tok_stride + c * 8;
    f16* dst = pool + (int64_t(kv) * num_pages * kWBlock + int64_t(page) * kWBlock + pos % kWBlock) * tok_stride + c * 8;
    *reinterpret_cast<u32x4*>(dst) = ld16(src);
  }
}

typedef __attribute__((address_space(3))) unsigned char lds_u8;

// Transposing LDS read of 4 fp16 per lane (ds_read_b64_tr_b16).  (Device compilation only, like the
// other gfx950 builtins below: the host pass does not know them and would drop the kernels' launch
// stubs.)
__device__ __forceinline__ u32x2 ds_read_tr16(const lds_u8* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef short v4s __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(const_cast<lds_u8*>(p))));
#else
  return u32x2{0u, 0u};
#endif
}
// 16-byte buffer load (buffer_load_dwordx4); an offset past the resource's end reads zeros.
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Maximum of lanes l and l ^ 32 (v_permlane32_swap: a VALU exchange, no LDS traffic).
__device__ __forceinline__ float max_lane32(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
#else
  return x;
#endif
}
// No instruction: the value is held in accumulation registers from here on (the queries, read
// only as MFMA operands, which take them from there without copies).
__device__ __forceinline__ void pin_agpr(f16x8& a) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" : "+a"(a));
#endif
}

// No instruction: the values must exist at this point (and the scheduler treats it as a boundary).
template <int RT>
__device__ __forceinline__ void pin_probs(f16x8 (&p)[RT][2]) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (RT == 2)
    asm volatile("" : "+v"(p[0][0]), "+v"(p[0][1]), "+v"(p[1][0]), "+v"(p[1][1]));
  else
    asm volatile("" : "+v"(p[0][0]), "+v"(p[0][1]));
#endif
}

// The kernel's body, run by workgroup bid of grid, with its LDS at smem (WideCfg::kLdsBytes).
// kPrefix: the caller runs only the shared-prefix pass (px.key_len > 0), so the causal limits are
// compiled out (in the one-launch shared-prefix kernel this keeps the loop within its registers).
template <int D, int G, int RT, int W, bool kAppend, bool kPrep, bool kPrefix = false>
__device__ __forceinline__ void prefill_wide_body(
    unsigned char* smem, const int bid, const int grid, f16* out, const f16* q, const f16* pool, int64_t num_pages,
    const int32_t* table, int32_t query_start, int32_t T, int32_t num_kv_heads, int32_t n_qb, int32_t nsplit,
    float scale_log2, PrefillWorkspace ws, PrefillAppend ap, PrefixOut px, PrefillPrep pp) {
  static_assert(!(kAppend && kPrep), "one form of the fused append");
  using C = WideCfg<D, G, RT, W>;
  constexpr int kKS = C::kKSteps;
  constexpr int kDT = C::kDT;
  constexpr int kQw = C::kQw;
  // Workgroup i runs on XCD i % 8: kv head = i % Hkv keeps each head's K/V in one XCD's L2 (for
  // Hkv = 8); query blocks go longest key range first.
  const int kvh = bid % num_kv_heads;
  const int split = (bid / num_kv_heads) % nsplit;
  const int qb = n_qb - 1 - bid / (num_kv_heads * nsplit);
  const int tid = threadIdx.x;
  const int grp = __builtin_amdgcn_readfirstlane(tid / kWave);  // key group = wave
  const int lane = tid % kWave;
  const int col = lane % 32, half = lane / 32;
  const int hq = num_kv_heads * G;
  // (shared-prefix mode: every row sees keys [0, key_len), no causal limit)
  const bool prefix_mode = kPrefix || px.key_len > 0;
  const int total = prefix_mode ? px.key_len : query_start + T;  // keys that exist
  const int q0 = qb * kQw;
  const int key_end = prefix_mode ? total : min(total, query_start + q0 + kQw);  // keys some row sees
  const int min_pos = prefix_mode ? total - 1 : query_start + q0;  // the last key every row sees
  const int n_tiles = int(ceil_div(key_end, kWTile));
  auto tile_of = [&](int i) { return (i * nsplit + split) * W + grp; };
  const int first = split * W + grp;
  const int iters = n_tiles > first ? int(ceil_div(n_tiles - first, W * nsplit)) : 0;

  // This lane's row in each row tile: row = 32 rt + col = g * kQw + query offset.
  int my_q[RT], my_pos[RT], my_head[RT];
  bool q_ok[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int rho = 32 * rt + col;
    my_q[rt] = q0 + rho % kQw;
    my_head[rt] = kvh * G + rho / kQw;
    my_pos[rt] = prefix_mode ? total - 1 : query_start + my_q[rt];
    q_ok[rt] = my_q[rt] < T;
  }

  const int64_t tok_stride = int64_t(num_kv_heads) * D;
  const int64_t v_off = num_pages * kWBlock * tok_stride;
  const int64_t page_elems = int64_t(kWBlock) * tok_stride;
  // (kPrep: the pool is read through the pointer it is written through, so no read is assumed to
  // be independent of the pre-append's stores)
  const f16* head_pool = (kPrep ? static_cast<const f16*>(pp.pool) : pool) + int64_t(kvh) * D;

  if constexpr (kAppend)
    wide_store_chunk(ap.pool, num_pages, table, query_start, T, num_kv_heads, D, ap.new_k, ap.new_v,
                     bid * C::kThreads + tid, grid * C::kThreads);

  // Page ids: a tile of 32 keys spans two pages.  Lane l of a window holds page 2 * tile + (l & 1) of
  // the wave's (l / 2)-th tile of that window (32 tiles), read with v_readlane.  A tile's K and V
  // are requested in the same step, so one window serves both.
  const int seq_pages = int(ceil_div(total, kWBlock));
  struct Window {
    int ids, w;
  };
  Window win_k{-1, -1};
  // (uniform branch, taken once per 32 tiles)
  auto ensure_window = [&](Window& wn, int i) __attribute__((always_inline)) {
    if ((i >> 5) != wn.w) {
      wn.w = i >> 5;
      const int pg = 2 * tile_of(32 * wn.w + lane / 2) + (lane & 1);
      const int id = table[min(pg, seq_pages - 1)];
      wn.ids = pg < seq_pages ? id : -1;
      asm volatile("" ::"v"(wn.ids));  // the window load completes here, not at every readlane
    }
  };
  // pages of tile i, whose window is loaded
  auto tile_pages = [&](Window& wn, int i, int& pa, int& pb) __attribute__((always_inline)) {
    pa = __builtin_amdgcn_readlane(wn.ids, 2 * (i & 31));
    pb = __builtin_amdgcn_readlane(wn.ids, 2 * (i & 31) + 1);
  };
  // Tile flags (uniform): bit 0/1 = first/second page valid.
  auto tile_flags = [&](int pa, int pb) __attribute__((always_inline)) -> int {
    const int oka = pa >= 0 && int64_t(pa) < num_pages, okb = pb >= 0 && int64_t(pb) < num_pages;
    return oka | (okb << 1);
  };

  // The first page-id window is read before the queries, so the first K loads wait for it alone.
  {
    win_k.w = 0;
    const int pg = 2 * tile_of(lane / 2) + (lane & 1);
    const int id = table[min(pg, seq_pages - 1)];
    win_k.ids = pg < seq_pages ? id : -1;
  }
  // The workgroup's queries, each row read once: wave grp loads rows 16 grp .. + 15 (a row past the
  // chunk as zeros), for the LDS staging below.
  lds_u8* const qlds = (lds_u8*)(smem) + C::kTileBytes;
  u32x4 qst[C::kQInstr];
  if constexpr (!kPrep) {
#pragma unroll
    for (int n = 0; n < C::kQInstr; ++n) {
      const int slot = n * kWave + lane, rho = C::kQRowsPerWave * grp + slot / C::kRowChunks, c = slot % C::kRowChunks;
      const int qi = q0 + rho % kQw;
      const u32x4 v = ld16(q + (int64_t(min(qi, T - 1)) * hq + kvh * G + rho / kQw) * D + 8 * c);
      qst[n] = qi < T ? v : u32x4{0u, 0u, 0u, 0u};
    }
  } else {
    using PR = PrepRows<D>;
    const int e = lane % PR::kLanes, sub = lane / PR::kLanes;
    // (1) This wave's tiles of the chunk (keys at or past query_start; query_start % 32 == 0): K
    // normalised and rotated, V cast, both written to the pool at the table's slots.  Rows past the
    // chunk and rows of an invalid page are not written (the attention reads zeros there).  The
    // work is a list of jobs (one wave pass of kRows rows each): the wave's tiles from the first one
    // in the chunk on (tile_of is increasing), kWTile / kRows jobs per tile.  A job's loads are
    // issued one job ahead, before the previous job's arithmetic and stores.  The queries' loads go
    // first, so they are in flight meanwhile.
    constexpr int kOps = kWTile / PR::kRows;
    const int first_tile = split * W + grp, tile_step = W * nsplit;  // tile_of(i) = first_tile + i tile_step
    const int qs_tile = query_start / kWTile;
    const int i0 = qs_tile > first_tile ? int(ceil_div(qs_tile - first_tile, tile_step)) : 0;
    const int nj = iters > i0 ? (iters - i0) * kOps : 0;
    struct Job {
      Pairs8 k, v, cs;
      int page;
    };
    auto job_pos = [&](int j) __attribute__((always_inline)) {  // key position of this lane's row of job j
      return tile_of(i0 + j / kOps) * kWTile + (j % kOps) * PR::kRows + sub;
    };
    auto job_load = [&](int j) __attribute__((always_inline)) -> Job {
      const int tc = min(job_pos(min(j, nj - 1)) - query_start, T - 1);  // (past the list: a valid row again)
      const int64_t src = (int64_t(tc) * num_kv_heads + kvh) * D;
      return Job{load_pairs8<D>(pp.k + src, e), load_pairs8<D>(pp.v + src, e),
                 load_pairs8<D>(pp.rope + int64_t(query_start + tc) * D, e), table[(query_start + tc) / kWBlock]};
    };
    // the queries' inputs (step 2)
    constexpr int kQOps = (C::kQRowsPerWave + PR::kRows - 1) / PR::kRows;
    Pairs8 xq[kQOps], csq[kQOps];
#pragma unroll
    for (int op = 0; op < kQOps; ++op) {
      const int rho = C::kQRowsPerWave * grp + min(op * PR::kRows + sub, C::kQRowsPerWave - 1);
      const int qc = min(q0 + rho % kQw, T - 1);
      xq[op] = load_pairs8<D>(pp.q + (int64_t(qc) * hq + kvh * G + rho / kQw) * D, e);
      csq[op] = load_pairs8<D>(pp.rope + int64_t(query_start + qc) * D, e);
    }
    const Pairs8 wk = load_pairs8<D>(pp.k_norm_w, e);
    if (nj > 0) {
      Job cur = job_load(0);
      for (int j = 0; j < nj; ++j) {
        const Job nxt = job_load(j + 1);
        const int pos = job_pos(j);
        u32x4 klo, khi;
        norm_rope_row<D>(cur.k, wk, cur.cs, pp.eps, klo, khi);
        if (pos - query_start < T && cur.page >= 0 && int64_t(cur.page) < num_pages) {
          f16* kd = pp.pool + (int64_t(cur.page) * kWBlock + pos % kWBlock) * tok_stride + int64_t(kvh) * D;
          f16* vd = kd + v_off;
          *reinterpret_cast<u32x4*>(kd + 8 * e) = klo;
          *reinterpret_cast<u32x4*>(kd + D / 2 + 8 * e) = khi;
          *reinterpret_cast<u32x4*>(vd + 8 * e) = pack_f16x8(cur.v.a[0], cur.v.a[1]);
          *reinterpret_cast<u32x4*>(vd + D / 2 + 8 * e) = pack_f16x8(cur.v.b[0], cur.v.b[1]);
        }
        cur = nxt;
      }
    }
    // (2) The workgroup's queries, normalised and rotated into the LDS staging (chunk c of row rho
    // at c ^ (rho % 8)); wave grp prepares rows kQRowsPerWave grp .. (a row past the chunk as zeros).
    const Pairs8 wq = load_pairs8<D>(pp.q_norm_w, e);
#pragma unroll
    for (int op = 0; op < kQOps; ++op) {
      const int rw = op * PR::kRows + sub;
      const int rho = C::kQRowsPerWave * grp + min(rw, C::kQRowsPerWave - 1);
      const int qi = q0 + rho % kQw;
      u32x4 lo, hi;
      norm_rope_row<D>(xq[op], wq, csq[op], pp.eps, lo, hi);
      if (qi >= T) lo = hi = u32x4{0u, 0u, 0u, 0u};
      if (rw < C::kQRowsPerWave) {
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(qlds + rho * 2 * D + ((e ^ (rho % 8)) * 16)) = lo;
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(
            qlds + rho * 2 * D + (((PR::kLanes + e) ^ (rho % 8)) * 16)) = hi;
      }
    }
    // The pool stores are complete before any of this wave's K or V requests (it reads back only
    // rows it wrote itself; the memory clobber keeps the compiler from hoisting them).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  // The window arrives before the first tiles' K and V are requested.
  asm volatile("" ::"v"(win_k.ids) : "memory");
  f16x8 qreg[RT][kKS];  // Q^T (filled from LDS in the prologue)

  // K and V tiles are read from the pool with 16-byte buffer loads into registers a step ahead of
  // their 16-byte writes into the wave's LDS buffers.  Each page half reads through a buffer
  // resource that ends after the page's keys below the end of the sequence (none for an invalid
  // page; the chunk's rows for a tile of them), so every other row reads zeros: masked keys
  // contribute exactly nothing (their scores are replaced by the mask).
  //  * V, lane l of load n of page half h -> slot 64 n + l: LDS row r = slot / (D / 8) of the half
  //    at chunk position slot % (D / 8), which holds the row's chunk (slot % (D / 8)) ^ 2 (r % 4).
  //  * K, load n (8 key rows x 8 chunks: every 8 consecutive lanes read one 128-byte line),
  //    lane l = 8 a + e: tile row r = 8 (n / (D / 64)) + a, chunk c = 8 (n % (D / 64)) + e.
  const int rsrc_bytes = kAppend ? T * int(tok_stride) * 2 : 0;
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(ap.new_v), 0, rsrc_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(ap.new_k), 0, rsrc_bytes, 0x00020000);
  uint32_t voff[C::kHalfInstr];
#pragma unroll
  for (int n = 0; n < C::kHalfInstr; ++n) {
    const int slot = n * kWave + lane, r = slot / C::kRowChunks;
    const int c = (slot % C::kRowChunks) ^ (2 * (r % 4));
    voff[n] = uint32_t((r * int(tok_stride) + 8 * c) * 2);
  }
  constexpr int kCB = C::kRowChunks / 8;  // chunk blocks per row
  uint32_t koff[C::kKInstr / 2];          // (the same for both page halves)
  uint32_t kwr;                           // LDS write offset (of load 0)
  {
    const int a = lane / 8, e = lane % 8;
#pragma unroll
    for (int n = 0; n < C::kKInstr / 2; ++n) {
      const int r = 8 * ((n / kCB) % 2) + a, c = 8 * (n % kCB) + e;
      koff[n] = uint32_t((r * int(tok_stride) + 8 * c) * 2);
    }
    kwr = uint32_t((e * 32 + (a ^ e)) * 16);
  }
  lds_u8* const vlds = (lds_u8*)(smem) + grp * C::kWaveBytes;
  lds_u8* const klds = vlds + C::kVBufs * C::kVBufBytes;
  // this lane's K fragment of K-step s (key row col, chunk 2 s + half) is at kfrag[s % 4] + 1 KiB s
  const lds_u8* kfrag[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kfrag[j] = klds + half * 512 + (col ^ ((2 * j + half) % 8)) * 16;
  struct VTile {
    __amdgpu_buffer_rsrc_t r[2];
    uint32_t add[2];
  };
  auto kv_tile = [&](int i, int pa, int pb, int fl, int64_t base, __amdgpu_buffer_rsrc_t own)
      __attribute__((always_inline)) -> VTile {
    const int kt = tile_of(i) * kWTile;
    VTile t;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // (page and key count are uniform; readfirstlane keeps the descriptor in scalar registers)
      const bool ok = ((fl >> h) & 1) != 0;
      const int page = __builtin_amdgcn_readfirstlane(ok ? (h == 0 ? pa : pb) : 0);
      // (kPrep: keys from key_end on -- hidden from every row here -- read as zeros, so a tile this
      // wave did not prepare is never read)
      const int keys = __builtin_amdgcn_readfirstlane(ok ? min(max((kPrep ? key_end : total) - (kt + 16 * h), 0), 16) : 0);
      t.r[h] = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(head_pool + base + int64_t(page) * page_elems), 0,
                                                 keys * int(tok_stride) * 2, 0x00020000);
      t.add[h] = 0;
      if constexpr (kAppend) {
        if (kt >= query_start) {  // (uniform) the chunk's own rows; past its end they read zero
          t.r[h] = own;
          t.add[h] = uint32_t(((min(kt - query_start, T) + 16 * h) * int(tok_stride) + kvh * D) * 2);
        }
      }
    }
    return t;
  };
  // load j (of kVInstr) of a tile's V, and its LDS write into buffer dst
  auto v_load = [&](const VTile& t, int j) __attribute__((always_inline)) {
    const int h = j / C::kHalfInstr, n = j % C::kHalfInstr;
    return buf_ld16(t.r[h], voff[n] + t.add[h]);
  };
  auto v_store = [&](lds_u8* dst, int j, u32x4 v) __attribute__((always_inline)) {
    const int h = j / C::kHalfInstr, n = j % C::kHalfInstr;
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(dst + h * C::kHalfBytes + (n * kWave + lane) * 16) = v;
  };
  // load n (of kKInstr) of a tile's K, its LDS write, and the read of K-step s's fragment
  auto k_load = [&](const VTile& t, int n) __attribute__((always_inline)) {
    const int h = n / (C::kKInstr / 2);
    return buf_ld16(t.r[h], koff[n % (C::kKInstr / 2)] + t.add[h]);
  };
  auto k_store = [&](int n, u32x4 v) __attribute__((always_inline)) {
    const int rb = n / kCB, cb = n % kCB;  // row block (8 rows), chunk block (8 chunks)
    // slot c 32 + (r ^ (c % 8)) = 256 cb + 8 rb + [32 e + (a ^ e)]
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(klds + kwr + cb * 4096 + rb * 128) = v;
  };
  auto k_read = [&](int s) __attribute__((always_inline)) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(kfrag[s % 4] + 1024 * s);
  };

  // Transposing V reads: lane = 16 g + 4 rr + q reads key row R = 4 (lane / 32) + rr of a page half,
  // dims 32 dt + 16 (g % 2) + 4 q .. + 3, i.e. logical chunk c = 4 dt + 2 (g % 2) + q / 2 at chunk
  // position c ^ 2 rr = 4 (dt ^ (rr / 2)) + (2 (g % 2) + q / 2) ^ 2 (rr % 2).  The dt part is a
  // constant offset of 64 dt bytes from one of two lane bases, for even and for odd dt.
  int tr_even, tr_odd;
  {
    const int rr = (lane % 16) / 4, q4 = lane % 4, g2 = (lane / 16) % 2;
    const int b2 = rr / 2;
    const int low = (2 * g2 + q4 / 2) ^ (2 * (rr % 2));
    const int base = (4 * half + rr) * 2 * D + 16 * low + 8 * (q4 % 2);
    tr_even = base + 64 * b2;
    tr_odd = base - 64 * b2;
  }

  float m[RT], lsum[RT];
  f32x16 acc[kDT][RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = kNegBig;
    lsum[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) acc[dt][rt] = f32x16{};
  }

  // A tile's first key, pages, page flags, and whether every key is visible to every row of the
  // block (no mask needed); all uniform.
  struct TilePos {
    int kt, pa, pb, fl;
    bool full;
  };
  auto tile_pos = [&](int t) __attribute__((always_inline)) -> TilePos {
    TilePos tp;
    tile_pages(win_k, t, tp.pa, tp.pb);
    tp.fl = tile_flags(tp.pa, tp.pb);
    tp.kt = tile_of(t) * kWTile;
    tp.full = (tp.fl == 3) & (tp.kt + kWTile <= total) & (tp.kt + kWTile - 1 <= min_pos);
    return tp;
  };
  // buffer resources of a tile's K and V
  auto k_tile = [&](int t, const TilePos& tp) __attribute__((always_inline)) {
    return kv_tile(t, tp.pa, tp.pb, tp.fl, 0, rk);
  };
  auto v_tile = [&](int t, const TilePos& tp) __attribute__((always_inline)) {
    return kv_tile(t, tp.pa, tp.pb, tp.fl, v_off, rv);
  };

  // Pipeline.  Step i (one tile) is two scheduling regions:
  //  A: tile i + 1's S MFMAs (K fragments read from the wave's K buffer), tile i + 2's K (loaded
  //     in the previous step) written to that buffer once every fragment is read, tile i + 3's K
  //     loads, and tile i's probabilities and fp16 packing in the MFMAs' shadow;
  //  B: tile i's PV MFMAs (V(i) from LDS through transposing reads), tile i + 1's V (loaded in the
  //     previous step) written to the LDS buffer tile i - 1 used, tile i + 2's V loads, tile i + 1's
  //     row maxima and tile i's row sums between them.
  // Tile i + 1's mask (when some key of it is hidden from some row) sits between the regions; the
  // lazy rescale for tile i + 1 opens the next step.  Every request is unconditional (past the last
  // tile they read zeros).
  u32x4 kr[kKS];
  u32x4 kst[C::kKInstr];  // K two tiles ahead, in flight to LDS
  u32x4 vst[C::kVInstr];  // the next tile's V, in flight to LDS
  auto s_mfma_step = [&](f32x16 (&st)[RT], int s) __attribute__((always_inline)) {  // S^T, K-step s
    const f16x8 kf = as_h8(kr[s]);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      st[rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qreg[rt][s], s == 0 ? f32x16{} : st[rt], 0, 0, 0);
  };
  // Causal mask, end of sequence and invalid pages (scores -> -inf): key kk of the tile is visible
  // to this lane's row iff kk <= lim and its page is valid; the lane's score r is key
  // 8 (r / 4) + 4 half + r % 4.
  auto mask = [&](f32x16 (&st)[RT], const TilePos& ti) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int lim = min(my_pos[rt], total - 1) - ti.kt;
      const int la = ((ti.fl & 1) ? lim : -1) - 4 * half;
      const int lb = ((ti.fl & 2) ? lim : kWBlock - 1) - 4 * half;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 8 * (r / 4) + (r % 4);
        st[rt][r] = c <= (r < 8 ? la : lb) ? st[rt][r] : -INFINITY;
      }
    }
  };
  // Each row's maximum over the tile and the lane ^ 32 partner (log2 units)
  float cand[RT];
  auto row_max = [&](const f32x16 (&st)[RT]) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float mq[4];
#pragma unroll
      for (int a = 0; a < 4; ++a)
        mq[a] = fmaxf(fmaxf(st[rt][4 * a], st[rt][4 * a + 1]), fmaxf(st[rt][4 * a + 2], st[rt][4 * a + 3]));
      cand[rt] = max_lane32(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * scale_log2;
    }
  };
  // Lazy rescale: the reference maximum moves only when a score exceeds it by more than kSlack
  // (log2 units), so P = 2^(s - m) < 2^kSlack; acc and lsum stay relative to m.
  auto rescale = [&]() __attribute__((always_inline)) {
    constexpr float kSlack = 8.f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const bool grow = cand[rt] > m[rt] + kSlack;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // rare after the first tile
        const float mn = grow ? cand[rt] : m[rt];
        const float alpha = exp2_fast(m[rt] - mn);
        lsum[rt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < kDT; ++dt) acc[dt][rt] *= alpha;
        m[rt] = mn;
      }
    }
  };
  // P of a tile in fp16 (the B operands of its PV MFMAs)
  auto numerators = [&](const f32x16 (&sc)[RT], f16x8 (&pb16)[RT][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) pv[r] = exp2_fast(fmaf(sc[rt][r], scale_log2, -m[rt]));
      pb16[rt][0] = f16x8{f16(pv[0]), f16(pv[1]), f16(pv[2]), f16(pv[3]), f16(pv[4]), f16(pv[5]), f16(pv[6]),
                          f16(pv[7])};
      pb16[rt][1] = f16x8{f16(pv[8]), f16(pv[9]), f16(pv[10]), f16(pv[11]), f16(pv[12]), f16(pv[13]),
                          f16(pv[14]), f16(pv[15])};
    }
  };
  // This lane's partial row sums of the fp16 probabilities (the values the PV MFMAs multiply),
  // added to lsum.
  auto add_row_sums = [&](const f16x8 (&pb16)[RT][2]) __attribute__((always_inline)) {
    const f16x2 one = f16x2{f16(1.f), f16(1.f)};
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s = __builtin_amdgcn_fdot2(f16x2{pb16[rt][u][2 * e], pb16[rt][u][2 * e + 1]}, one, s, false);
      lsum[rt] += s;
    }
  };
  // PV batch b of a tile: O^T += V^T . P^T for dim tiles 2 b and 2 b + 1 (8 transposing reads, 8
  // MFMAs).  A = V^T for dims 32 dt + col, keys 16 u + 4 half + 0..3 and 16 u + 8 + 4 half + 0..3
  // (page half u).  after(pr) runs after MFMA pair pr (0..3) of the batch.
  auto pv_batch = [&](auto bc, const lds_u8* ae, const lds_u8* ao, const f16x8 (&pb16)[RT][2], auto&& after)
      __attribute__((always_inline)) {
    constexpr int b = decltype(bc)::value;
    constexpr int d0 = 2 * b, HB = C::kHalfBytes, HI = 16 * D;
    u32x2 rd[8];
    rd[0] = ds_read_tr16(ae + 64 * d0);
    rd[1] = ds_read_tr16(ae + 64 * d0 + HI);
    rd[2] = ds_read_tr16(ae + HB + 64 * d0);
    rd[3] = ds_read_tr16(ae + HB + 64 * d0 + HI);
    rd[4] = ds_read_tr16(ao + 64 * (d0 + 1));
    rd[5] = ds_read_tr16(ao + 64 * (d0 + 1) + HI);
    rd[6] = ds_read_tr16(ao + HB + 64 * (d0 + 1));
    rd[7] = ds_read_tr16(ao + HB + 64 * (d0 + 1) + HI);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f16x4 lo = __builtin_bit_cast(f16x4, rd[4 * j + 2 * u]);
        const f16x4 hi = __builtin_bit_cast(f16x4, rd[4 * j + 2 * u + 1]);
        const f16x8 vf = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          acc[d0 + j][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pb16[rt][u], acc[d0 + j][rt], 0, 0, 0);
        after(2 * j + u);
      }
  };
  // VALU instructions per MFMA in region A: ~50 per row tile for a tile's probabilities, over
  // RT kKS MFMAs (two VALU groups per K-step)
  constexpr int kAValu = (50 * RT + 2 * kKS - 1) / (2 * kKS);
  TilePos p1, p2;  // tiles i + 1 and i + 2
  auto step = [&](f32x16 (&sc)[RT], f32x16 (&sn)[RT], int i) __attribute__((always_inline)) {
    rescale();  // for tile i, whose maxima were taken in the previous step
    ensure_window(win_k, i + 3);
    const TilePos p3 = tile_pos(i + 3);
    const VTile k3 = k_tile(i + 3, p3);
    const VTile v2 = v_tile(i + 2, p2);
    __builtin_amdgcn_sched_barrier(0);
    // region A.  (With two waves per SIMD, the wave in its score MFMAs and exponentials goes first;
    // measured 0.8 us per config-3 layer.)
    if constexpr (W == 8) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < kKS; ++s) kr[s] = k_read(s);
#pragma unroll
    for (int s = 0; s < kKS; ++s) s_mfma_step(sn, s);
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) k_store(n, kst[n]);
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) kst[n] = k_load(k3, n);
    f16x8 pb16[RT][2];
    numerators(sc, pb16);
    // (the probabilities are pinned here, so the exponentials are not sunk to their use in the PV
    // MFMAs below, out of the MFMAs' shadow)
    pin_probs<RT>(pb16);
    static_assert(C::kKInstr == kKS, "one K write and load per K-step");
    // K fragment reads: all first with 4 waves; two ahead of their MFMAs with 8 (registers)
    constexpr int kAhead = W == 4 ? kKS : 2;
    __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
    for (int s = 0; s < kKS; ++s) {
      if (s + kAhead < kKS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, kAValu, 0);  // VALU
      if constexpr (RT == 2) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);       // K write
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);       // K load
      __builtin_amdgcn_sched_group_barrier(0x002, kAValu, 0);  // VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (W == 8) __builtin_amdgcn_s_setprio(0);
    // tile i + 1's mask, when some key of it is hidden from some row
    if (!p1.full) mask(sn, p1);
    // region B
    const lds_u8* const vcur = vlds + (i % C::kVBufs) * C::kVBufBytes;
    const lds_u8* const ae = vcur + tr_even;
    const lds_u8* const ao = vcur + tr_odd;
    lds_u8* const vnext = vlds + ((i + 1) % C::kVBufs) * C::kVBufBytes;
    // Tile i's PV MFMAs; tile i + 1's V goes to LDS (first batch; with one V buffer, the last,
    // after every read of tile i) and tile i + 2's is loaded (last batch) between them.
    auto batch = [&](auto bc) __attribute__((always_inline)) {
      constexpr int b = decltype(bc)::value;
      pv_batch(bc, ae, ao, pb16, [&](const int pr) __attribute__((always_inline)) {
        if constexpr (C::kVBufs == 1) {
          if constexpr (b == kDT / 2 - 1) {
            constexpr int per = C::kVInstr / 4;  // V loads per MFMA pair
#pragma unroll
            for (int t = 0; t < per; ++t) v_store(vnext, per * pr + t, vst[per * pr + t]);
#pragma unroll
            for (int t = 0; t < per; ++t) vst[per * pr + t] = v_load(v2, per * pr + t);
          }
        } else if constexpr (kDT == 4) {
          if constexpr (b == 0) {
            v_store(vnext, 2 * pr, vst[2 * pr]);
            v_store(vnext, 2 * pr + 1, vst[2 * pr + 1]);
          } else {
            vst[2 * pr] = v_load(v2, 2 * pr);
            vst[2 * pr + 1] = v_load(v2, 2 * pr + 1);
          }
        } else {
          v_store(vnext, pr, vst[pr]);
          vst[pr] = v_load(v2, pr);
        }
      });
    };
    static_assert(C::kVInstr == 2 * kDT, "one V load per MFMA pair over the batches");
    batch(std::integral_constant<int, 0>{});
    if constexpr (kDT == 4) batch(std::integral_constant<int, 1>{});
    // tile i + 1's row maxima and tile i's row sums, in the PV MFMAs' shadow
    row_max(sn);
    add_row_sums(pb16);
    __builtin_amdgcn_sched_barrier(0);
    p1 = p2;
    p2 = p3;
  };
  // A wave's last step: tile i's probabilities and PV MFMAs only (no next tile to score or load).
  auto last_step = [&](const f32x16 (&sc)[RT], int i) __attribute__((always_inline)) {
    rescale();
    f16x8 pb16[RT][2];
    numerators(sc, pb16);
    add_row_sums(pb16);
    const lds_u8* const vcur = vlds + (i % C::kVBufs) * C::kVBufBytes;
    auto none = [](int) {};
    pv_batch(std::integral_constant<int, 0>{}, vcur + tr_even, vcur + tr_odd, pb16, none);
    if constexpr (kDT == 4) pv_batch(std::integral_constant<int, 1>{}, vcur + tr_even, vcur + tr_odd, pb16, none);
  };

  // prologue: K(0) and V(0) loads; K(0) to LDS, K(1) loads; S(0); K(1) to LDS, K(2) loads; V(0)
  // to LDS, V(1) loads; tile 0's mask
  f32x16 sa[RT], sb[RT];
  {
    const TilePos p0 = tile_pos(0);
    p1 = tile_pos(1);
    p2 = tile_pos(2);
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) kst[n] = k_load(k_tile(0, p0), n);
#pragma unroll
    for (int j = 0; j < C::kVInstr; ++j) vst[j] = v_load(v_tile(0, p0), j);
    // Q through LDS: Q^T as the B operand, K-step s = dims 16 s + 8 half .. + 7 of row 32 rt + col
    // (kPrep: the staging is written already)
    if constexpr (!kPrep) {
#pragma unroll
      for (int n = 0; n < C::kQInstr; ++n) {
        const int slot = n * kWave + lane, rho = C::kQRowsPerWave * grp + slot / C::kRowChunks, c = slot % C::kRowChunks;
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(qlds + rho * 2 * D + ((c ^ (rho % 8)) * 16)) = qst[n];
      }
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int s = 0; s < kKS; ++s) {
        const int rho = 32 * rt + col, c = 2 * s + half;
        qreg[rt][s] = as_h8(*reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(qlds + rho * 2 * D + ((c ^ (rho % 8)) * 16)));
        if constexpr (W == 4) pin_agpr(qreg[rt][s]);
      }
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) k_store(n, kst[n]);
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) kst[n] = k_load(k_tile(1, p1), n);
    // The barrier above leaves the 4 waves in step; started in step they would reach their load
    // and their MFMA phases together for the whole loop and queue on the CU's shared memory path.
    // Wave grp starts 6 x 64 x grp cycles late instead (a quarter of a step or so apart; measured:
    // 71.9 -> 67.4 us per config-3 layer).
    for (int w = 0; w < grp % 4; ++w) __builtin_amdgcn_s_sleep(6);
#pragma unroll
    for (int s = 0; s < kKS; ++s) kr[s] = k_read(s);
#pragma unroll
    for (int s = 0; s < kKS; ++s) s_mfma_step(sa, s);
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) k_store(n, kst[n]);
#pragma unroll
    for (int n = 0; n < C::kKInstr; ++n) kst[n] = k_load(k_tile(2, p2), n);
#pragma unroll
    for (int j = 0; j < C::kVInstr; ++j) v_store(vlds, j, vst[j]);
#pragma unroll
    for (int j = 0; j < C::kVInstr; ++j) vst[j] = v_load(v_tile(1, p1), j);
    if (!p0.full) mask(sa, p0);
    row_max(sa);
  }
  // Pairs of steps, then the last one or two tiles: the last tile's scores are in sa or sb
  // depending on the parity of iters (one call site for the last step keeps the register
  // allocation of the loop).
  int i = 0;
  for (; i + 2 < iters; i += 2) {
    step(sa, sb, i);
    step(sb, sa, i + 1);
  }
  if (iters > 0) {
    const bool two = i + 2 == iters;
    if (two) step(sa, sb, i);
    f32x16 sl[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) sl[rt] = two ? sb[rt] : sa[rt];
    last_step(sl, iters - 1);
  }

  // every wave's V reads are done before the LDS is reused for the merge
  __syncthreads();

  float lt[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) lt[rt] = lsum[rt] + __shfl_xor(lsum[rt], 32);
  // Key-group merge: every wave writes its (m, l) and all its blocks, normalised (O / l) in fp16,
  // to LDS (half the bytes of fp32 accumulators; O / l is a convex combination of fp16 value rows,
  // so fp16 keeps it to a relative 2^-11); block p = (dim tile p / RT, row tile p % RT) is then
  // finished, quarter by quarter, by the waves that own it, from the W groups' copies in group
  // order, each weighted by e^(m - M) l.  Every quarter a wave finishes has row tile rt_own.
  auto own = [&](int u, int& p, int& r4) __attribute__((always_inline)) {  // owned quarter u
    if constexpr (C::kBlocks >= W) {
      p = grp + W * (u / 4);
      r4 = u % 4;
    } else {
      p = grp % C::kBlocks;
      r4 = (grp / C::kBlocks) * C::kOwnU + u;
    }
  };
  const int rt_own = (C::kBlocks >= W ? grp : grp % C::kBlocks) % RT;
  float* mlb = reinterpret_cast<float*>(smem);                 // [wave][rt][32][2]
  f16x4* accb = reinterpret_cast<f16x4*>(mlb + C::kMlFloats);  // [wave][block][4][lane]: O / l in fp16
  if (half == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      mlb[((grp * RT + rt) * 32 + col) * 2 + 0] = m[rt];
      mlb[((grp * RT + rt) * 32 + col) * 2 + 1] = lt[rt];
    }
  }
  float linv[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) linv[rt] = lt[rt] > 0.f ? 1.f / lt[rt] : 0.f;
#pragma unroll
  for (int p = 0; p < C::kBlocks; ++p)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x16& a = acc[p / RT][p % RT];
      const float iv = linv[p % RT];
      accb[((grp * C::kBlocks + p) * 4 + r4) * kWave + lane] =
          f16x4{f16(a[4 * r4] * iv), f16(a[4 * r4 + 1] * iv), f16(a[4 * r4 + 2] * iv), f16(a[4 * r4 + 3] * iv)};
    }
  __syncthreads();
  float mk[W], lk[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    mk[k] = mlb[((k * RT + rt_own) * 32 + col) * 2];
    lk[k] = mlb[((k * RT + rt_own) * 32 + col) * 2 + 1];
  }
  float mfin = mk[0];
#pragma unroll
  for (int k = 1; k < W; ++k) mfin = fmaxf(mfin, mk[k]);
  float wk[W];
#pragma unroll
  for (int k = 0; k < W; ++k) wk[k] = exp2_fast(mk[k] - mfin);
  float lfin = wk[0] * lk[0];
#pragma unroll
  for (int k = 1; k < W; ++k) lfin = fmaf(wk[k], lk[k], lfin);
  float wl[W];  // weight of wave k's O / l
#pragma unroll
  for (int k = 0; k < W; ++k) wl[k] = wk[k] * lk[k];
  f32x4 o[C::kOwnU];  // the quarters this wave finishes
#pragma unroll
  for (int u = 0; u < C::kOwnU; ++u) {
    int p, r4;
    own(u, p, r4);
    f16x4 x = accb[((0 * C::kBlocks + p) * 4 + r4) * kWave + lane];
    f32x4 y = f32x4{wl[0] * float(x[0]), wl[0] * float(x[1]), wl[0] * float(x[2]), wl[0] * float(x[3])};
#pragma unroll
    for (int k = 1; k < W; ++k) {
      x = accb[((k * C::kBlocks + p) * 4 + r4) * kWave + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = fmaf(wl[k], float(x[e]), y[e]);
    }
    o[u] = y;
  }

  if (prefix_mode) {  // this split's state of (row my_q, kv head kvh, head g)
    if (!q_ok[rt_own]) return;
    const int g = my_head[rt_own] - kvh * G;
    const int64_t pslot = ((int64_t(my_q[rt_own]) * num_kv_heads + kvh) * px.stride + split) * G + g;
    // (8-byte stores at the device coherence point: a workgroup of the same launch may merge them)
    if (grp < RT && half == 0) st_dev8(px.ml + pslot * 2, f32x2{mfin, lfin});
    const float inv = lfin > 0.f ? 1.f / lfin : 0.f;
#pragma unroll
    for (int u = 0; u < C::kOwnU; ++u) {  // dims 32 dt + 8 r4 + 4 half + 0..3 of block p
      int p, r4;
      own(u, p, r4);
      const int64_t at = pslot * D + 32 * (p / RT) + 8 * r4 + 4 * half;
      if (px.oh != nullptr)  // (uniform) normalised, fp16
        st_dev8(px.oh + at, __builtin_bit_cast(f32x2, f16x4{f16(o[u][0] * inv), f16(o[u][1] * inv),
                                                          f16(o[u][2] * inv), f16(o[u][3] * inv)}));
      else
        *reinterpret_cast<f32x4*>(px.o + at) = o[u];
    }
    return;
  }

  if (nsplit > 1) {
    // Cross-workgroup merge: every wave publishes its quarters of this split's partial with 16-byte
    // device-coherent stores (lane-contiguous), waves 0 .. RT - 1 their row tile's (m, l); once all are
    // acknowledged one thread takes the (query block, kv head) ticket.  The last of the nsplit
    // arrivals combines every split's partial, its own included (read back), in split order, so
    // the result does not depend on the arrival order.
    __shared__ uint32_t s_ticket;
    const int64_t pair = int64_t(qb) * num_kv_heads + kvh;
    const int64_t slot = pair * nsplit + split;
    const int64_t nslots = int64_t(n_qb) * num_kv_heads * nsplit;
    const __amdgpu_buffer_rsrc_t r_o = make_rsrc(ws.o, uint32_t(nslots * C::kRows * D * 4));
    const __amdgpu_buffer_rsrc_t r_ml = make_rsrc(ws.ml, uint32_t(nslots * C::kRows * 2 * 4));
    auto o_off = [&](int64_t sl, int p, int r4) __attribute__((always_inline)) {
      return uint32_t((((sl * C::kBlocks + p) * 4 + r4) * kWave + lane) * 16);
    };
    const uint32_t ml_row = uint32_t(rt_own * 32 + col) * 8;
#pragma unroll
    for (int u = 0; u < C::kOwnU; ++u) {
      int p, r4;
      own(u, p, r4);
      st_dev4(r_o, o_off(slot, p, r4), o[u]);
    }
    if (grp < RT && half == 0) st_dev2(r_ml, uint32_t(slot * C::kRows * 8) + ml_row, f32x2{mfin, lfin});
    wait_all_mem();   // this wave's stores are acknowledged
    __syncthreads();  // ... and every other wave's
    if (tid == 0) s_ticket = __hip_atomic_fetch_add(ws.count + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_ticket != uint32_t(nsplit - 1)) return;
    compiler_fence();  // the merge loads below stay behind the ticket
    float mx = kNegBig;
    // (this split's own partial is taken from registers, not read back)
    const float m_own = mfin, l_own = lfin;
    f32x4 mine[C::kOwnU];
#pragma unroll
    for (int u = 0; u < C::kOwnU; ++u) {
      mine[u] = o[u];
      o[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    mx = m_own;
    for (int s2 = 0; s2 < nsplit; ++s2)
      if (s2 != split) mx = fmaxf(mx, ld_dev2(r_ml, uint32_t((pair * nsplit + s2) * C::kRows * 8) + ml_row)[0]);
    lfin = 0.f;
    // splits in batches of kSplitBatch, every load of a batch in flight at once
    constexpr int kSplitBatch = 4;
    for (int s0 = 0; s0 < nsplit; s0 += kSplitBatch) {
#pragma unroll
      for (int sb = 0; sb < kSplitBatch; ++sb) {
        const int s2 = s0 + sb;
        if (s2 < nsplit) {
          const int64_t sl = pair * nsplit + s2;
          f32x2 ml = f32x2{m_own, l_own};
          f32x4 x[C::kOwnU];
#pragma unroll
          for (int u = 0; u < C::kOwnU; ++u) x[u] = mine[u];
          if (s2 != split) {  // (uniform)
            ml = ld_dev2(r_ml, uint32_t(sl * C::kRows * 8) + ml_row);
#pragma unroll
            for (int u = 0; u < C::kOwnU; ++u) {
              int p, r4;
              own(u, p, r4);
              x[u] = ld_dev4(r_o, o_off(sl, p, r4));
            }
          }
          const float wsp = exp2_fast(ml[0] - mx);
          lfin = fmaf(wsp, ml[1], lfin);
#pragma unroll
          for (int u = 0; u < C::kOwnU; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[u][e] = fmaf(wsp, x[u][e], o[u][e]);
        }
      }
    }
    mfin = mx;
    if (tid == 0) reset_ticket(ws.count + pair);
  }

  if (!q_ok[rt_own]) return;
  const float inv = lfin > 0.f ? 1.f / lfin : 0.f;
  f16* orow = out + (int64_t(my_q[rt_own]) * hq + my_head[rt_own]) * D;
#pragma unroll
  for (int u = 0; u < C::kOwnU; ++u) {  // dims 32 dt + 8 r4 + 4 half + 0..3 of block p
    int p, r4;
    own(u, p, r4);
    const int dt = p / RT;
    const f32x4 y = o[u];
    *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * r4 + 4 * half) =
        f16x4{f16(y[0] * inv), f16(y[1] * inv), f16(y[2] * inv), f16(y[3] * inv)};
  }
}

template <int D, int G, int RT, int W, bool kAppend, bool kPrep>
__global__ __launch_bounds__(W * kWave) void prefill_wide_kernel(
    f16* __restrict__ out, const f16* __restrict__ q, const f16* __restrict__ pool, int64_t num_pages,
    const int32_t* __restrict__ table, int32_t query_start, int32_t T, int32_t num_kv_heads, int32_t n_qb,
    int32_t nsplit, float scale_log2, PrefillWorkspace ws, PrefillAppend ap, PrefixOut px, PrefillPrep pp) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[WideCfg<D, G, RT, W>::kLdsBytes];
  prefill_wide_body<D, G, RT, W, kAppend, kPrep>(smem, int(blockIdx.x), int(gridDim.x), out, q, pool, num_pages, table,
                                                 query_start, T, num_kv_heads, n_qb, nsplit, scale_log2, ws, ap, px, pp);
}

typedef void (*WideKernel)(f16*, const f16*, const f16*, int64_t, const int32_t*, int32_t, int32_t, int32_t, int32_t,
                           int32_t, float, PrefillWorkspace, PrefillAppend, PrefixOut, PrefillPrep);

enum class WideMode { kPlain, kAppend, kPrep };

// (row tiles and waves: 2 and 4 for every shape; 1 and 8 for head dim 128)
static WideKernel pick_wide(int d, int g, int rt, int w, WideMode mode) {
#define IFN_WIDE_CASE(DD, GG, RR, WW)                                                                \
  if (d == DD && g == GG && rt == RR && w == WW)                                                     \
    return mode == WideMode::kAppend ? prefill_wide_kernel<DD, GG, RR, WW, true, false>              \
           : mode == WideMode::kPrep ? prefill_wide_kernel<DD, GG, RR, WW, false, true>              \
                                     : prefill_wide_kernel<DD, GG, RR, WW, false, false>;
  IFN_WIDE_CASE(64, 1, 2, 4) IFN_WIDE_CASE(64, 2, 2, 4) IFN_WIDE_CASE(64, 4, 2, 4) IFN_WIDE_CASE(64, 8, 2, 4)
  IFN_WIDE_CASE(128, 1, 2, 4) IFN_WIDE_CASE(128, 2, 2, 4) IFN_WIDE_CASE(128, 4, 2, 4) IFN_WIDE_CASE(128, 8, 2, 4)
  IFN_WIDE_CASE(128, 1, 1, 8) IFN_WIDE_CASE(128, 2, 1, 8) IFN_WIDE_CASE(128, 4, 1, 8) IFN_WIDE_CASE(128, 8, 1, 8)
#undef IFN_WIDE_CASE
  return nullptr;
}

bool wide_prefill_supported(int32_t hq, int32_t hkv, int32_t d) {
  return hkv >= 1 && hq % hkv == 0 && pick_wide(d, hq / hkv, 2, 4, WideMode::kPlain) != nullptr;
}

size_t wide_prefill_ws_bytes(int32_t T, int32_t query_start, int32_t hq, int32_t hkv, int32_t d, int cus) {
  return plan_wide(T, query_start, hq, hkv, d, cus).bytes;
}

int wide_prefill_launch(f16* out, const f16* q, const f16* pool, int64_t num_pages, const int32_t* table,
                        int32_t query_start, int32_t T, int32_t hq, int32_t hkv, int32_t d, float scale_log2,
                        void* workspace, size_t workspace_bytes, const PrefillAppend& ap, int cus,
                        hipStream_t stream, const PrefillPrep* prep) {
  const WidePlan p = plan_wide(T, query_start, hq, hkv, d, cus);
  const WideMode mode = prep != nullptr ? WideMode::kPrep : ap.pool != nullptr ? WideMode::kAppend : WideMode::kPlain;
  WideKernel k = pick_wide(d, hq / hkv, p.rt, p.w, mode);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
  if (prep != nullptr && (ap.pool != nullptr || query_start % kWTile != 0)) return IFN_ERR_UNSUPPORTED;
  if (p.n_qb * hkv * p.nsplit > int64_t(1) << 31) return IFN_ERR_UNSUPPORTED;
  // (the fused append indexes the chunk's K and V rows with 32-bit byte offsets)
  if (ap.pool != nullptr && int64_t(T) * hkv * d * 2 >= int64_t(1) << 31) return IFN_ERR_UNSUPPORTED;
  PrefillWorkspace ws{nullptr, nullptr, nullptr};
  if (p.nsplit > 1) {
    if (workspace == nullptr || workspace_bytes < p.bytes) return IFN_ERR_WORKSPACE;
    IFN_CHECK_ALIGN16(workspace);
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    ws.count = reinterpret_cast<uint32_t*>(wsb);
    ws.ml = reinterpret_cast<float*>(wsb + p.off_ml);
    ws.o = reinterpret_cast<float*>(wsb + p.off_o);
  }
  k<<<dim3(unsigned(p.n_qb * hkv * p.nsplit)), dim3(unsigned(p.w * kWave)), 0, stream>>>(
      out, q, pool, num_pages, table, query_start, T, hkv, int(p.n_qb), p.nsplit, scale_log2, ws, ap,
      PrefixOut{nullptr, nullptr, 0, 0, nullptr}, prep != nullptr ? *prep : PrefillPrep{});
  return ifn_launch_status();
}

int wide_prefix_splits(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int32_t key_len, int cus) {
  return plan_wide(batch, 0, hq, hkv, d, cus, key_len).nsplit;
}

int wide_prefix_pass(const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages, int32_t key_len,
                     int32_t batch, int32_t hq, int32_t hkv, int32_t d, float scale_log2, float* px_ml, float* px_o,
                     f16* px_oh, int32_t stride, int cus, hipStream_t stream) {
  if (key_len < 1) return IFN_ERR_INVALID_ARGUMENT;
  const WidePlan p = plan_wide(batch, 0, hq, hkv, d, cus, key_len);
  WideKernel k = pick_wide(d, hq / hkv, p.rt, p.w, WideMode::kPlain);
  if (k == nullptr) return IFN_ERR_UNSUPPORTED;
  if (p.n_qb * hkv * p.nsplit > int64_t(1) << 31 || stride < p.nsplit) return IFN_ERR_UNSUPPORTED;
  k<<<dim3(unsigned(p.n_qb * hkv * p.nsplit)), dim3(unsigned(p.w * kWave)), 0, stream>>>(
      nullptr, q, pool, num_pages, prefix_pages, 0, batch, hkv, int(p.n_qb), p.nsplit, scale_log2,
      PrefillWorkspace{nullptr, nullptr, nullptr}, PrefillAppend{nullptr, nullptr, nullptr},
      PrefixOut{px_ml, px_o, key_len, stride, px_oh}, PrefillPrep{});
  return ifn_launch_status();
}


// ---- shared-prefix decode in one launch ------------------------------------------------------
// Rows that begin with the same prefix pages (a cascade row: at least px.pages pages long) are
// decoded by one grid of two kinds of workgroup, one per CU:
//  * workgroups [0, npre): the prefix pass -- prefill_wide_body in prefix mode over the prefix keys
//    (32 query rows of one kv head and one key split per workgroup), which leaves a state per
//    (row, kv head, head of the group, split) at the device coherence point;
//  * workgroups [npre, npre + ndec): the whole-row decode of the rows' own keys (decode_rows_body,
//    kFused: a cascade row's states are always published).
// Each (cascade row, kv head) has one ticket, counting the decode ranges that hold the row's keys
// and the prefix workgroups (one per key split) that hold its query rows.  Whichever arrives last -- either kind --
// merges the row's heads of that kv head (its split states in range order, then its prefix states:
// the same arithmetic either way) and writes them.  No workgroup waits for another, so the two kinds run side by side: the prefix pass's MFMA
// work on its CUs while the others stream the private pages.  Shorter rows are decoded as usual.
template <int D, int G, int HKV>
struct FusedLayout {  // the decode role's LDS arrays, laid over the prefix role's tile buffers
  using L = RowsLds<D, G, HKV, false, true, 2 * HKV>;
  static constexpr size_t kAcc = 0;
  static constexpr size_t kM = kAcc + sizeof(f32x4) * kRowsWaves * HKV * L::GR * (D / 4);
  static constexpr size_t kL = kM + sizeof(float) * kRowsWaves * L::HQ;
  static constexpr size_t kApp = (kL + sizeof(float) * kRowsWaves * L::HQ + 15) / 16 * 16;
  static constexpr size_t kQ = kApp + 16;
  static constexpr size_t kWsum = kQ + 16;
  static constexpr size_t kTicket = kWsum + sizeof(int) * kRowsWaves;
  static constexpr size_t kCum = kTicket + 2 * HKV * sizeof(uint32_t);
  static constexpr size_t kCasc = kCum + sizeof(int) * (kRowsMaxBatch + 1);
  static constexpr size_t kBytes = kCasc + kRowsMaxBatch;
};

template <int D, int G>
__global__ __launch_bounds__(8 * kWave) void shared_prefix_fused_kernel(
    const f16* __restrict__ pool, const int32_t* __restrict__ block_tables, const f16* __restrict__ q, int32_t batch,
    int32_t max_pages, int32_t max_len, int32_t ndec, int64_t num_pages, f16* __restrict__ out,
    const int32_t* __restrict__ seq_lens, const uint8_t* __restrict__ active, float scale_log2, DecodeWorkspace ws,
    DecodePrefix px, const int32_t* __restrict__ prefix_pages, int32_t n_qb, int32_t nsplit, int32_t npre) {
  constexpr int HKV = 8;
  using C = WideCfg<D, G, 1, 8>;
  using FL = FusedLayout<D, G, HKV>;
  using L = typename FL::L;
  static_assert(C::kThreads == kRowsThreads, "both roles run 8 waves");
  constexpr size_t kBytes = C::kLdsBytes > FL::kBytes ? C::kLdsBytes : FL::kBytes;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kBytes];
  const int bid = int(blockIdx.x), tid = int(threadIdx.x);
  const int pk = px.pages * kRowsBlock;  // prefix keys
  const int cap = min(max_pages * kRowsBlock, max_len);

  if (bid >= npre) {  // the private pages
    L sh{*reinterpret_cast<int(*)[kRowsMaxBatch + 1]>(smem + FL::kCum),
         *reinterpret_cast<int(*)[kRowsWaves]>(smem + FL::kWsum),
         *reinterpret_cast<float(*)[kRowsWaves][L::HQ]>(smem + FL::kM),
         *reinterpret_cast<float(*)[kRowsWaves][L::HQ]>(smem + FL::kL),
         *reinterpret_cast<f32x4(*)[kRowsWaves][HKV * L::GR][D / 4]>(smem + FL::kAcc),
         *reinterpret_cast<uint32_t(*)[2 * HKV]>(smem + FL::kTicket),
         *reinterpret_cast<uint8_t(*)[kRowsMaxBatch]>(smem + FL::kCasc),
         *reinterpret_cast<f16(*)[1][8]>(smem + FL::kApp),
         *reinterpret_cast<f16(*)[1][8]>(smem + FL::kQ)};
    decode_rows_body<D, G, HKV, kRowsStages, false, true, false, true, kRowsBlock, true>(
        sh, bid - npre, nullptr, pool, block_tables, q, batch, max_pages, max_len, ndec, num_pages, out, seq_lens,
        active, scale_log2, ws, DecodeAppend{nullptr, nullptr, nullptr, nullptr}, DecodePrep{}, px);
    return;
  }

  // The prefix pass for (query block qb, kv head bid % Hkv, key split): its states, stored at the
  // device coherence point.
  prefill_wide_body<D, G, 1, 8, false, false, true>(
      smem, bid, npre, out, q, pool, num_pages, prefix_pages, 0, batch, HKV, n_qb, nsplit, scale_log2,
      PrefillWorkspace{nullptr, nullptr, nullptr}, PrefillAppend{nullptr, nullptr, nullptr},
      PrefixOut{px.ml, px.o, pk, px.nstates, const_cast<f16*>(px.oh)}, PrefillPrep{});
  wait_all_mem();   // this wave's state stores acknowledged
  __syncthreads();  // ... and every other wave's; the tile buffers are free
  // The decode role's split of the rows' own keys (the same offsets and ranges), to find where a
  // cascade row's split states sit.
  int* s_cum = reinterpret_cast<int*>(smem);
  int* s_wsum = s_cum + kRowsMaxBatch + 1;
  int* s_rec = s_wsum + kRowsWaves;  // per query row of the block: (first range, ranges) if last, else -1
  const int T = build_offsets(s_cum, s_wsum, seq_lens, active, batch, cap, pk);
  const int64_t nr = range_count(ndec, T);
  constexpr int kQw = C::kQw;  // batch rows per query block
  const int q0 = (n_qb - 1 - bid / (HKV * nsplit)) * kQw;
  const int kvh = bid % HKV;
  const int npx = px.nstates - 1;  // prefix states per (row, head): nsplit
  if (tid < kQw) {
    const int b = q0 + tid;
    int first = -1, nrg = 0;
    if (b < batch && row_keys(seq_lens, active, b, cap) >= pk) {
      const int cb = s_cum[b] + row_start_cost(batch), len = s_cum[b + 1] - cb;
      int f = 0;
      if (len > 0) {  // (T >= len > 0)
        f = int(div_floor((int64_t(cb) + 1) * nr - 1, T));
        nrg = int(div_floor((int64_t(cb) + len) * nr - 1, T)) - f + 1;
      }
      const uint32_t t = __hip_atomic_fetch_add(fused_ticket(ws.count, batch, HKV, b, kvh), 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      if (t == uint32_t(nrg + npx - 1)) first = f;
    }
    s_rec[2 * tid] = first;
    s_rec[2 * tid + 1] = nrg;
  }
  __syncthreads();
  compiler_fence();  // the merge loads below stay behind the tickets
  const uint32_t n_slots = uint32_t(batch) + uint32_t(ndec);
  const RowsMerge<D, G, HKV, true, kFusedMergeBatch> mg{make_rsrc(ws.o, n_slots * L::HQ * D * 2u),
                                      make_rsrc(ws.ml, n_slots * L::HQ * 2u * 4u), px, out};
  // the block's rows this workgroup arrived last at: heads kvh * G .. kvh * G + G - 1 of each
  constexpr int D4 = D / 4;
  for (int idx = tid; idx < kQw * G * D4; idx += kRowsThreads) {
    const int j = idx / (G * D4), rem = idx % (G * D4);
    const int first = s_rec[2 * j];
    if (first < 0) continue;
    const int64_t b = q0 + j;
    mg.item(b, b + first, s_rec[2 * j + 1], true, kvh * G + rem / D4, rem % D4);
  }
  if (tid < kQw && s_rec[2 * tid] >= 0) reset_ticket(fused_ticket(ws.count, batch, HKV, q0 + tid, kvh));
}

int shared_prefix_fused_launch(f16* out, const f16* q, const f16* pool, int64_t num_pages, const int32_t* prefix_pages,
                               const int32_t* block_tables, int32_t max_pages, const int32_t* seq_lens,
                               const uint8_t* active, int32_t batch, int32_t hq, int32_t hkv, int32_t d,
                               int32_t max_len, float scale_log2, void* workspace, int blocks, const DecodePrefix& px,
                               int max_states, int cus, hipStream_t stream) {
  // Built for head dim 128, 8 kv heads and groups 2 and 4 (Qwen3-0.6B, Qwen3-8B).  The prefix pass
  // takes npre = ceil(batch / (32 / G)) x 8 x nsplit workgroups: two key splits while that is at most
  // half the CUs, else one while it is at most a quarter; the rest of the CUs decode the private
  // pages.  (Config 5, 36 layers: 128 + 128 workgroups measured 47.5 us, 64 + 192 52.3 us -- the
  // prefix pass reads HBM under the decode's stream, and its workgroups' key loops are latency
  // bound; when the prefixes stay in the last-level cache, as with a few layers, 64 + 192 is the
  // faster, 42.3 against 45.6 us.)  Prefixes of at most 8192 keys (a prefix workgroup's share grows
  // with the prefix); otherwise the two launches.
  if (d != 128 || hkv != 8 || (hq != 16 && hq != 32) || px.pages < 1) return IFN_ERR_UNSUPPORTED;
  const int g = hq / hkv;
  const int64_t n_qb = (int64_t(batch) + 32 / g - 1) / (32 / g);
  const int64_t key_len = int64_t(px.pages) * kRowsBlock;
  const int nsplit = 2 * (n_qb * hkv * 2) <= cus && max_states >= 3 ? 2 : 1;
  const int64_t npre = n_qb * hkv * nsplit;
  const int64_t ndec = (int64_t(cus) - npre) / kRowsXcds * kRowsXcds;
  if (nsplit + 1 > max_states || (nsplit == 1 && 4 * npre > cus) || ndec < kRowsXcds || ndec > blocks ||
      key_len > 8192 || int64_t(batch) * (hkv + 1) > kMaxTickets)  // (a ticket per row, then per (cascade row, kv head))
    return IFN_ERR_UNSUPPORTED;
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  size_t off_ml, off_o;
  rows_ws_layout(batch, hq, d, blocks, &off_ml, &off_o);
  DecodeWorkspace ws;
  ws.count = reinterpret_cast<uint32_t*>(wsb);
  ws.ml = reinterpret_cast<float*>(wsb + off_ml);
  ws.o = reinterpret_cast<float*>(wsb + off_o);
  const DecodePrefix pxf{px.ml, px.o, px.pages, nsplit + 1, px.oh};
  auto k = g == 4 ? shared_prefix_fused_kernel<128, 4> : shared_prefix_fused_kernel<128, 2>;
  k<<<dim3(unsigned(npre + ndec)), dim3(kRowsThreads), 0, stream>>>(
      pool, block_tables, q, batch, max_pages, max_len, int32_t(ndec), num_pages, out, seq_lens, active, scale_log2,
      ws, pxf, prefix_pages, int32_t(n_qb), nsplit, int32_t(npre));
  return ifn_launch_status();
}

}  // namespace ifn
