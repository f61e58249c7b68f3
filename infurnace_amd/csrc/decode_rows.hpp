// Paged GQA decode over whole token rows (gfx950), for pools whose token row -- num_kv_heads x
// head_dim fp16 -- is 2 KiB: Qwen3-0.6B and Qwen3-8B (8 KV heads x 128), and 4 x 256 / 16 x 64.
//
// Replaces the reference's documented paged_attention for decode
// (docs/architecture.md:246; placeholder src/infurnace/kernels/paged_attention.py) whose contiguous
// semantics are src/infurnace/executor/tinygrad/model.py:196-200: read positions [0, pos], upcast
// fp16 K/V to fp32, scaled_dot_product_attention with scale 1/sqrt(head_dim) and query head h ->
// kv head h / group.
//
// Decode is HBM-bound.  On MI355X a gather of 16-token pages reads fastest when every load
// instruction takes whole, contiguous token rows, so this kernel is organised around rows:
//
//  * Workgroup ranges over the flat token list.  The tokens of all rows, row after row, form one
//    list; workgroup w (one per CU, 8 waves) takes positions [T w / N, T (w+1) / N), so ragged
//    batches cost every CU the same bytes.  In a call of several rows every non-empty row is counted
//    kRowStartCost positions longer than its keys (virtual positions in front of it): a range
//    that ends one row and starts the next pays a second start-up and merge, and gets that many
//    keys fewer.
//    Workgroups are remapped so that each XCD streams a contiguous eighth of the list.  A range is
//    cut into pieces at row boundaries.
//  * Inside a piece the 8 waves interleave by token: wave w takes positions a + w + 8 i, so at
//    any moment the workgroup reads 8 consecutive token rows of one page (16 KiB of K and 16 KiB
//    of V, contiguous).  A wave reads a whole token row -- every kv head -- with two 16-byte loads
//    per lane for K and two for V: lane = (64 / Hkv) * kv_head + col holds 16-byte chunks col and
//    col + 64 / Hkv of its head, so each load instruction reads 1 KiB in 128-byte runs.  The wave
//    keeps an S-stage register ring of tokens in flight; page ids sit one per lane (64 per
//    window) and are read with v_readlane.
//  * q.k uses v_dot2_f32_f16 (fp32 accumulation) and a DPP reduction over the head's lanes; the
//    online softmax runs in base 2 per (lane, query head of the kv head's group).  Each K/V row
//    is fetched once and reused from registers by every query head of its GQA group.
//  * At the end of a piece the 8 waves merge log-sum-exp style through LDS, so one state per
//    (row, workgroup) leaves the CU.  A row held by one workgroup is written directly; a row split
//    over several workgroups is merged by the workgroup that arrives last (device-coherent
//    16-byte state stores, one ticket per row, taken once at the end of the range).
//  * Shared-prefix mode (kCascade): rows that begin with a prefix already attended by the prefix
//    pass stream only their own pages, and the workgroup that finishes such a row merges the
//    prefix pass's states into it before writing fp16.
//  * Optional step plan (decode_plan_kernel): the split depends only on the lengths, the tables
//    and the appended slots, which every layer of a decode step shares.  Built once per step, the
//    plan holds the rows' offsets in the token list and, per range, its first pieces and first
//    64 page ids, so a workgroup starts its first K/V loads one round trip after launch instead
//    of three (lengths -> offsets -> page ids -> rows).
#pragma once

#include "ifn_common.hpp"

namespace ifn {


constexpr int kRowsWaves = 8;
constexpr int kRowsThreads = kRowsWaves * kWave;
constexpr int kRowsMaxBatch = 4096;  // rows per call (LDS offset table)
constexpr int kRowsBlock = 16;       // tokens per page compiled in
constexpr int kRowsXcds = 8;         // MI355X: workgroups dispatched round-robin over 8 XCDs
constexpr int kMergeBatch = 16;      // split states loaded per round trip of the final merge
constexpr int kFusedMergeBatch = 4;  // the same in the one-launch shared-prefix kernel
constexpr int kBurst = 4;            // a wave's run of at most this many tokens is requested at once
constexpr int kRowsStages = 2;       // tokens in flight per wave (the ring's depth)
// Cost of starting a row, in tokens.  A range that holds the end of one row and the start of the
// next pays a second start-up, a second merge of its waves and possibly two split merges, so the
// split counts each non-empty row as kRowStartCost tokens longer (virtual tokens in front of it).
constexpr int kRowStartCost = 24;
// The cost the split charges a call's rows: none for a single row (every range then holds one
// piece of it, so no range starts a second row), which keeps one row of 512 keys at 16 ranges
// of 32 keys -- one burst per wave and one round trip of split states in the final merge.
__host__ __device__ __forceinline__ int row_start_cost(int batch) { return batch > 1 ? kRowStartCost : 0; }
// Fewest virtual positions per range.  A row split over n ranges is merged by one workgroup that
// reads n partial states (Hq x D floats each), so short batches are split over fewer workgroups:
// one row of 512 keys takes 16 ranges of 32 positions instead of one range per CU.
constexpr int kMinRangePositions = 32;

// floor(num / den) for 0 <= num < 2^52 and den > 0: a double quotient (off by less than one)
// corrected by one step -- a few instructions instead of the 64-bit integer division routine.
__device__ __forceinline__ int64_t div_floor(int64_t num, int64_t den) {
  int64_t q = int64_t(double(num) / double(den));
  if (q * den > num) --q;
  else if ((q + 1) * den <= num) ++q;
  return q;
}

// Ranges of a call: one per workgroup, at most, and none empty of positions.
__device__ __forceinline__ int64_t range_count(int64_t nb, int64_t T) {
  return min(nb, (T + kMinRangePositions - 1) / kMinRangePositions);
}

// Step plan (int32 words).  Header: magic, batch, ranges nr, virtual positions T, grid, whether
// appended slots were given, the row-length cap, the shared-prefix keys pk (0: none).  Then the
// rows' offsets cum[batch + 1], then one record per workgroup range: [0] pieces of the range;
// [1 + 6 p ..] piece p < kPlanPieces: row, first key a, end key e, first range of the row, ranges of
// the row, and the row's appended slot (or, in shared-prefix mode, which has no append, the key of
// the row's first streamed key: pk for a cascade row, else 0); [64 + i] page id i of the first
// piece's first window.
constexpr int32_t kPlanMagic = 0x504c4e31;
constexpr int kPlanHdr = 16;
constexpr int kPlanRec = 128;
constexpr int kPlanPieces = 3;
constexpr int kPlanIds = 64;
static inline __host__ __device__ int64_t plan_rec0(int32_t batch) { return (kPlanHdr + batch + 1 + 63) / 64 * 64; }
static inline size_t plan_words(int32_t batch, int blocks) { return size_t(plan_rec0(batch) + int64_t(blocks) * kPlanRec); }

// Workspace: [tickets: kTicketBytes][ml][o].  Slot = row + range index: the workgroups holding a
// row are consecutive ranges, so (row, range) -> row + range is unique and below batch + ranges.
// A split state is (m, l) in fp32 and the normalised output O / l in fp16 (a convex combination of
// value rows, so fp16 keeps it to a relative 2^-11): the last arrival of a long row reads every
// state of it, and halving the bytes it reads halves that step.
static inline size_t rows_ws_layout(int32_t batch, int32_t hq, int32_t d, int64_t ranges, size_t* off_ml,
                                    size_t* off_o) {
  const size_t slots = size_t(batch) + size_t(ranges);
  size_t off = kTicketBytes;
  *off_ml = off;
  off = align256(off + slots * hq * 2 * sizeof(float));
  *off_o = off;
  off = align256(off + slots * hq * d * sizeof(uint16_t));
  return off;
}

// Keys of row b (0 for inactive rows), clamped to cap; and the slot its appended token goes to
// (-1 for none: inactive rows and slots outside the pool store nothing, as store_kv).
__device__ __forceinline__ int row_keys(const int32_t* seq_lens, const uint8_t* active, int b, int cap) {
  const int sl = seq_lens[b];
  const int act = active != nullptr ? int(active[b]) : 1;
  return act != 0 ? max(0, min(sl, cap)) : 0;
}
__device__ __forceinline__ int row_slot(const int32_t* slots, const uint8_t* active, int b, int64_t num_slots) {
  const int64_t sl = slots[b];
  const bool act = active == nullptr || active[b] != 0;
  return act && sl >= 0 && sl < num_slots ? int(sl) : -1;
}

// Offsets of the rows in the split's virtual token list, into s_cum[0 .. batch] (all threads of the
// workgroup call it; returns the total).  Row b occupies [s_cum[b], s_cum[b + 1]); its keys are the
// last of those positions, after row_start_cost(batch) virtual ones when it has any.  Shared-prefix mode
// (pk > 0): a row of at least pk keys (a cascade row, flagged in s_casc) streams only its keys
// after the first pk.
// s_len (optional): the rows' keys, already in LDS (and published by a barrier).
__device__ __forceinline__ int build_offsets(int* s_cum, int* s_wsum, const int32_t* seq_lens,
                                             const uint8_t* active, int batch, int cap, int pk = 0,
                                             uint8_t* s_casc = nullptr, const int* s_len = nullptr) {
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, nwaves = blockDim.x / kWave;
  int running = 0;
  for (int base = 0; base < batch; base += blockDim.x) {
    const int i = base + tid;
    int len = i < batch ? (s_len != nullptr ? s_len[i] : row_keys(seq_lens, active, i, cap)) : 0;
    const bool casc = pk > 0 && len >= pk;
    if (s_casc != nullptr && i < batch) s_casc[i] = casc ? 1 : 0;
    if (casc) len -= pk;
    if (len > 0) len += row_start_cost(batch);
    int x = len;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == kWave - 1) s_wsum[wave] = x;
    __syncthreads();
    int wpre = 0, tot = 0;
    for (int w = 0; w < nwaves; ++w) {
      const int v = s_wsum[w];
      wpre += w < wave ? v : 0;
      tot += v;
    }
    if (i < batch) s_cum[i] = running + wpre + x - len;
    running += tot;
    __syncthreads();
  }
  if (tid == 0) s_cum[batch] = running;
  __syncthreads();
  return running;
}

// The row holding virtual position t (t < s_cum[batch]): the last b with s_cum[b] <= t, which skips
// rows without keys.
__device__ __forceinline__ int locate_row(const int* s_cum, int batch, int64_t t) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_cum[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// A piece: keys [a, e) of row b, in range `first` .. first + nranges - 1 of the row's ranges, and
// the row's appended slot.  off: the key position of the row's first streamed key (the prefix
// length for a cascade row, else 0), already added to a and e.
struct RowPiece {
  int b, a, e, first, nranges, slot, off;
};

// Step plan: one workgroup writes the header, the offsets and every range's record.
constexpr int kPlanThreads = 1024;
constexpr int kPlanTabWords = 16384;  // block tables up to this many entries are staged in LDS
template <int PB>  // tokens per page
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(
    int32_t* __restrict__ plan, const int32_t* __restrict__ block_tables, int32_t max_pages,
    const int32_t* __restrict__ seq_lens, const uint8_t* __restrict__ active, const int32_t* __restrict__ slots,
    int64_t num_pages, int32_t batch, int32_t max_len, int32_t nb, int32_t pk) {
  __shared__ int s_cum[kRowsMaxBatch + 1];
  __shared__ int s_wsum[kPlanThreads / kWave];
  __shared__ int s_p0[3][kPlanThreads];  // first piece of range r: row, a, e (rows < 0: none)
  __shared__ int s_slot[kRowsMaxBatch];   // appended slot of each row (-1: none)
  __shared__ int s_len[kRowsMaxBatch];    // keys of each row
  __shared__ int s_tab[kPlanTabWords];    // the block table, when it fits
  const int tid = threadIdx.x;
  const int cap = min(max_pages * PB, max_len);
  const int64_t num_slots = num_pages * PB;
  // Every load the plan depends on goes out at launch, in one round trip: the rows' lengths, flags
  // and slots and, when it fits in LDS (config 2: 32 KB), the whole block table -- so that the page
  // ids of the ranges' first windows come from LDS instead of a second round trip.
  const int64_t tab_words = int64_t(batch) * max_pages;
  const bool tab_lds = tab_words <= kPlanTabWords;
  constexpr int kRowsPer = kRowsMaxBatch / kPlanThreads, kTabPer = kPlanTabWords / kPlanThreads;
  // Unconditional loads (indices clamped, absent arrays read through a stand-in), selected after
  // every load is out: a load under a condition makes the compiler wait for it at the join.
  const uint8_t* act_src = active != nullptr ? active : reinterpret_cast<const uint8_t*>(seq_lens);
  const int32_t* slot_src = slots != nullptr ? slots : seq_lens;
  int r_len[kRowsPer], r_slot[kRowsPer], r_tab[kTabPer];
  uint8_t r_act[kRowsPer];
#pragma unroll
  for (int k = 0; k < kRowsPer; ++k) {
    const int i = min(tid + k * kPlanThreads, batch - 1);
    r_len[k] = seq_lens[i];
    r_act[k] = act_src[i];
    r_slot[k] = slot_src[i];
  }
  if (tab_lds) {
#pragma unroll
    for (int k = 0; k < kTabPer; ++k) r_tab[k] = block_tables[min(int64_t(tid + k * kPlanThreads), tab_words - 1)];
  }
#pragma unroll
  for (int k = 0; k < kRowsPer; ++k) {
    const int i = tid + k * kPlanThreads;
    if (i < batch) {
      const bool act = active == nullptr || r_act[k] != 0;
      const int sl = slots != nullptr ? r_slot[k] : -1;
      s_len[i] = act ? max(0, min(r_len[k], cap)) : 0;           // row_keys
      s_slot[i] = act && sl >= 0 && sl < num_slots ? sl : -1;  // row_slot
    }
  }
  if (tab_lds) {
#pragma unroll
    for (int k = 0; k < kTabPer; ++k) {
      const int i = tid + k * kPlanThreads;
      if (i < tab_words) s_tab[i] = r_tab[k];
    }
  }
  __syncthreads();
  // (pk > 0: a row of at least pk keys streams only its keys after the first pk)
  const int T = build_offsets(s_cum, s_wsum, seq_lens, active, batch, cap, pk, nullptr, s_len);
  const int nr = int(range_count(nb, T));
  if (tid == 0) {
    plan[0] = kPlanMagic;
    plan[1] = batch;
    plan[2] = nr;
    plan[3] = T;
    plan[4] = nb;
    plan[5] = slots != nullptr ? 1 : 0;
    plan[6] = cap;
    plan[7] = pk;
  }
  for (int i = tid; i <= batch; i += kPlanThreads) plan[kPlanHdr + i] = s_cum[i];
  int32_t* recs = plan + plan_rec0(batch);
  for (int r = tid; r < nb; r += kPlanThreads) {
    int32_t* rec = recs + int64_t(r) * kPlanRec;
    int n = 0;
    int p0b = -1, p0a = 0, p0e = 0;
    if (r < nr) {
      const int64_t t0 = div_floor(int64_t(T) * r, nr), t1 = div_floor(int64_t(T) * (r + 1), nr);
      auto range_of = [&](int64_t t) -> int { return int(div_floor((t + 1) * nr - 1, T)); };
      int b = locate_row(s_cum, batch, t0);
      while (b < batch) {
        const int cb = s_cum[b] + row_start_cost(batch);
        const int len = s_cum[b + 1] - cb;
        if (len > 0) {
          if (cb >= t1) break;
          const int a = int(max<int64_t>(t0, cb) - cb);
          const int e = int(min<int64_t>(t1, int64_t(cb) + len) - cb);
          if (a < e) {
            if (n < kPlanPieces) {
              int32_t* pc = rec + 1 + 6 * n;
              const int first = range_of(cb);
              pc[0] = b;
              pc[1] = a;
              pc[2] = e;
              pc[3] = first;
              pc[4] = range_of(int64_t(cb) + len - 1) - first + 1;
              pc[5] = slots != nullptr ? s_slot[b] : (pk > 0 && s_len[b] >= pk ? pk : 0);
            }
            if (n == 0) {  // (the first window's pages count from the row's first key)
              const int off = pk > 0 && s_len[b] >= pk ? pk : 0;
              p0b = b;
              p0a = a + off;
              p0e = e + off;
            }
            ++n;
          }
          if (int64_t(cb) + len >= t1) break;
        }
        ++b;
      }
    }
    rec[0] = n;
    s_p0[0][r] = p0b;
    s_p0[1][r] = p0a;
    s_p0[2][r] = p0e;
  }
  __syncthreads();
  // The first window's page ids.  Wave w takes ranges w, w + 16, ...: lane i loads id i of a
  // range (one coalesced 256-byte load per range), and all of a wave's loads are issued before
  // its first store.
  constexpr int kPlanWaves = kPlanThreads / kWave;
  constexpr int kIdBatch = 16;
  static_assert(kPlanIds == kWave, "one id per lane");
  const int wave = tid / kWave, lane = tid % kWave;
  for (int r0 = wave; r0 < nb; r0 += kPlanWaves * kIdBatch) {
    int id[kIdBatch];
#pragma unroll
    for (int k = 0; k < kIdBatch; ++k) {
      const int r = min(r0 + k * kPlanWaves, nb - 1);
      const int b = s_p0[0][r];
      const int pg0 = b >= 0 ? s_p0[1][r] / PB : 0;
      const int npg = b >= 0 ? (s_p0[2][r] - 1) / PB - pg0 + 1 : 1;
      const int64_t at = int64_t(max(b, 0)) * max_pages + pg0 + min(lane, npg - 1);
      id[k] = tab_lds ? s_tab[at] : block_tables[at];
    }
#pragma unroll
    for (int k = 0; k < kIdBatch; ++k) {
      const int r = r0 + k * kPlanWaves;
      if (r < nb) recs[int64_t(r) * kPlanRec + 64 + lane] = s_p0[0][r] >= 0 ? id[k] : 0;
    }
  }
}

// A wave's two 8-dim halves of a token row's head: lane (hd, col) holds dims 8 col .. 8 col + 7 and
// D/2 + 8 col .. D/2 + 8 col + 7 of head hd -- exactly the rotary pairs (i, i + D/2) of its 8 dims,
// since 8 x (lanes per head) = D/2 for a 2 KiB row.  Loads the fp32 values of one head row.
template <int D>
__device__ __forceinline__ void load_pairs(const float* row, int col, float (&x1)[8], float (&x2)[8]) {
  const f32x4 a0 = *reinterpret_cast<const f32x4*>(row + 8 * col);
  const f32x4 a1 = *reinterpret_cast<const f32x4*>(row + 8 * col + 4);
  const f32x4 b0 = *reinterpret_cast<const f32x4*>(row + D / 2 + 8 * col);
  const f32x4 b1 = *reinterpret_cast<const f32x4*>(row + D / 2 + 8 * col + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x1[j] = a0[j];
    x1[4 + j] = a1[j];
    x2[j] = b0[j];
    x2[4 + j] = b1[j];
  }
}

// RMSNorm + rotary of one head held as load_pairs leaves it (LPH lanes per head), in the rounding
// and summation order of the pre-append kernel: pair i = 8 col + j of the head sits in register j
// of lane col, so the butterfly over pairs (i ^ 1, i ^ 2, i ^ 4, then i ^ 8, ...) is a tree over
// the registers followed by the DPP sum over the head's lanes.  Pairs i >= D/2 of a 64-lane
// butterfly would add zeros, which leave the sum unchanged.
template <int D, int LPH>
__device__ __forceinline__ void norm_rope_head(float (&x1)[8], float (&x2)[8], const float (&w1)[8],
                                               const float (&w2)[8], const float (&c)[8], const float (&s)[8],
                                               float eps) {
  float p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) p[j] = pair_sq(x1[j], x2[j]);
  const float s01 = p[0] + p[1], s23 = p[2] + p[3], s45 = p[4] + p[5], s67 = p[6] + p[7];
  float ss = (s01 + s23) + (s45 + s67);
  ss = sum_lanes<LPH>(ss);
  const float rs = rms_inv(ss, D, eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) norm_rope_pair(x1[j], x2[j], rs, w1[j], w2[j], c[j], s[j]);
}

__device__ __forceinline__ u32x4 pack_h8(const float (&x)[8]) {
  return __builtin_bit_cast(u32x4, f16x8{f16(x[0]), f16(x[1]), f16(x[2]), f16(x[3]), f16(x[4]), f16(x[5]),
                                         f16(x[6]), f16(x[7])});
}

// The kernel's LDS arrays, by reference (the kernel declares them; a kernel that runs this body on
// some of its workgroups lays them over its other LDS).
template <int D, int G, int HKV, bool kPrep, bool kCascade, int NT = 2>
struct RowsLds {
  static constexpr int HQ = HKV * G, GR = G < 2 ? G : 2, ROW = HKV * D;
  int (&s_cum)[kRowsMaxBatch + 1];  // rows' offsets in the virtual token list
  int (&s_wsum)[kRowsWaves];
  float (&s_m)[kRowsWaves][HQ];
  float (&s_l)[kRowsWaves][HQ];
  f32x4 (&s_acc)[kRowsWaves][HKV * GR][D / 4];
  uint32_t (&s_ticket)[NT];  // tickets taken at the end of a range (kFused: per kv head of two rows)
  uint8_t (&s_casc)[kCascade ? kRowsMaxBatch : 1];  // kCascade: row b is a cascade row
  // kPrep: the appended token's fp16 K and V rows, prepared at the start of its piece
  f16 (&s_app)[kPrep ? 2 : 1][kPrep ? ROW : 8];
  // kPrep: the piece's fp16 query, head g of every kv head in the layout of a token row
  f16 (&s_q)[kPrep ? G : 1][kPrep ? ROW : 8];
};

// The merges of the whole-row kernel, over split states (m, l) fp32 and O / l fp16 at slots of the
// workspace (r_ml, r_o) and, for a cascade row, its prefix states (px).  kDev: the prefix states were
// written in the same launch, by other workgroups, so they are read at the device coherence point.
// MB: split states per round trip.
template <int D, int G, int HKV, bool kDev, int MB = kMergeBatch>
struct RowsMerge {
  static constexpr int HQ = HKV * G, D4 = D / 4;
  // A batch of split states (MB per round trip) and of prefix states (4 per round trip).
  struct Ld {
    f32x2 ml[MB];
    f32x2 o[MB];  // 4 fp16 dims of O / l
  };
  struct Px {
    f32x2 ml[4];
    f16x4 o[4];
  };
  __amdgpu_buffer_rsrc_t r_o, r_ml;
  DecodePrefix px;
  f16* out;

  __device__ __forceinline__ uint32_t ml_off(int64_t s, int qh) const { return uint32_t((s * HQ + qh) * 2 * 4); }
  __device__ __forceinline__ uint32_t o_off(int64_t s, int qh, int d4) const {
    return uint32_t(((s * HQ + qh) * D + 4 * d4) * 2);
  }
  // Log-sum-exp merge of a split row's np states (slots slot0 .. slot0 + np - 1, in range order)
  // for query head qh, dims 4 d4 .. 4 d4 + 3.  Every lane loads each state's (m, l) itself (the
  // lanes of a query head read the same 8 bytes, one request) and its 4 dims of O / l, MB states per
  // round trip, and reduces them on its own: no lane exchanges, whose latency would sit on the last
  // workgroup's path.  issue sends the first round trip (so that a caller can overlap
  // it with other work), finish the rest and the arithmetic.  Only the cnt states that exist are
  // loaded (cnt is uniform).
  __device__ __forceinline__ void load(int64_t s0, int cnt, int qh, int d4, Ld& ld) const {
#pragma unroll
    for (int u = 0; u < MB; ++u) {
      if (u < cnt) {
        ld.ml[u] = ld_dev2(r_ml, ml_off(s0 + u, qh));
        ld.o[u] = ld_dev2(r_o, o_off(s0 + u, qh, d4));
      }
    }
  }
  __device__ __forceinline__ void issue(int64_t slot0, int np, int qh, int d4, Ld& ld) const {
    load(slot0, min(MB, np), qh, d4, ld);
  }
  __device__ __forceinline__ void finish(int64_t slot0, int np, int qh, int d4, Ld& ld, float& M, float& L,
                                         f32x4& O) const {
    for (int j0 = 0; j0 < np; j0 += MB) {
      const int cnt = min(MB, np - j0);
      if (j0 > 0) load(slot0 + j0, cnt, qh, d4, ld);
      __builtin_amdgcn_sched_barrier(0);
      float gm = kNegBig;
#pragma unroll
      for (int u = 0; u < MB; ++u)
        if (u < cnt) gm = fmaxf(gm, ld.ml[u][0]);
      const float nm = fmaxf(M, gm);
      const float sc = exp2_fast(M - nm);
      O = f32x4{O[0] * sc, O[1] * sc, O[2] * sc, O[3] * sc};
      L *= sc;
      M = nm;
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        if (u < cnt) {
          const float w = exp2_fast(ld.ml[u][0] - M) * ld.ml[u][1];  // weight of O / l: e^(m - M) l
          const f16x4 oh = __builtin_bit_cast(f16x4, ld.o[u]);
          L += w;
          O = f32x4{fmaf(w, float(oh[0]), O[0]), fmaf(w, float(oh[1]), O[1]), fmaf(w, float(oh[2]), O[2]),
                    fmaf(w, float(oh[3]), O[3])};
        }
      }
    }
  }
  // Cascade row b, query head qh, dims 4 d4 .. 4 d4 + 3: the row's own state (M, L, unnormalised O)
  // merged with the prefix states (m, l and O / l in fp16), 4 per round trip.  The caller loads the
  // first 4 into pb with px_load before the row's own merge, so that their round trip overlaps it.
  __device__ __forceinline__ void px_load(int64_t b, int qh, int d4, int s0, Px& pb) const {
    const int npx = px.nstates - 1;
    const int64_t st0 = (b * HKV + qh / G) * px.nstates * G + qh % G;  // state s: st0 + s * G
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t st = st0 + int64_t(min(s0 + u, npx - 1)) * G;
      if constexpr (kDev) {
        pb.ml[u] = ld_dev8(px.ml + st * 2);
        pb.o[u] = __builtin_bit_cast(f16x4, ld_dev8(px.oh + st * D + 4 * d4));
      } else {
        pb.ml[u] = *reinterpret_cast<const f32x2*>(px.ml + st * 2);
        pb.o[u] = *reinterpret_cast<const f16x4*>(px.oh + st * D + 4 * d4);
      }
    }
  }
  __device__ __forceinline__ void cascade_out(int64_t b, int qh, int d4, float M, float L, f32x4 O, Px& pb) const {
    const int npx = px.nstates - 1;
    for (int s0 = 0; s0 < npx; s0 += 4) {
      if (s0 > 0) px_load(b, qh, d4, s0, pb);
      const f32x2* mlv = pb.ml;
      const f16x4* ov = pb.o;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (s0 + u < npx) {
          const float nm = fmaxf(M, mlv[u][0]);
          const float a = exp2_fast(M - nm), cl = exp2_fast(mlv[u][0] - nm) * mlv[u][1];
          L = fmaf(L, a, cl);
          O = f32x4{fmaf(O[0], a, cl * float(ov[u][0])), fmaf(O[1], a, cl * float(ov[u][1])),
                    fmaf(O[2], a, cl * float(ov[u][2])), fmaf(O[3], a, cl * float(ov[u][3]))};
          M = nm;
        }
      }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *reinterpret_cast<f16x4*>(out + (b * HQ + qh) * D + 4 * d4) =
        f16x4{f16(O[0] * inv), f16(O[1] * inv), f16(O[2] * inv), f16(O[3] * inv)};
  }
  // A merged row's output: fp16, or (cascade rows) merged with the prefix states first.
  __device__ __forceinline__ void write_row(int64_t b, int qh, int d4, float M, float L, f32x4 O, bool casc,
                                            Px& pb) const {
    if (casc) {
      cascade_out(b, qh, d4, M, L, O, pb);
      return;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *reinterpret_cast<f16x4*>(out + (b * HQ + qh) * D + 4 * d4) =
        f16x4{f16(O[0] * inv), f16(O[1] * inv), f16(O[2] * inv), f16(O[3] * inv)};
  }
  // Query head qh, dims 4 d4 .. 4 d4 + 3 of row b, merged whole: its np split states at slot0 ..
  // slot0 + np - 1 (none: a cascade row with no key after the prefix), then for a cascade row its
  // prefix states.  The same arithmetic, in the same order, as the merges of the kernel's split
  // rows, so the output does not depend on which workgroup arrives last.
  __device__ __forceinline__ void item(int64_t b, int64_t slot0, int np, bool casc, int qh, int d4) const {
    Px pb;
    Ld ld;
    if (casc) px_load(b, qh, d4, 0, pb);
    issue(slot0, np, qh, d4, ld);
    float M = kNegBig, L = 0.f;
    f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
    finish(slot0, np, qh, d4, ld, M, L, O);
    write_row(b, qh, d4, M, L, O, casc, pb);
  }
};

// kFused: the ticket of cascade row b's kv head h (after one per row for the split rows).
__device__ __forceinline__ uint32_t* fused_ticket(uint32_t* count, int32_t batch, int hkv, int64_t b, int h) {
  return count + batch + b * hkv + h;
}

// kAppend: the step's store_kv is fused in (ap); kStream: K/V row loads carry the non-temporal
// hint (each row read once per launch; wrong when rows of the batch share pages).  S: tokens in
// flight per wave.  plan: a step plan for exactly these lengths, tables and slots, or null.
// kPrep: the pre-append is fused in as well (pp): the query rows and the appended K/V rows come
// from fp32 projections, normalised, rotated and cast here (q is unused; ap.slots / ap.pool
// give the store's slots and pool, ap.new_k / ap.new_v are unused).
// kCascade: shared-prefix mode (px, px.pages > 0).  A row of at least px.pages pages (a cascade
// row) streams only the pages after them; the workgroup that finishes the row then merges its
// state with the prefix pass's states 0 .. nstates - 2 of each segment (seg = row * Hkv + kv head:
// ml[((seg * nstates + s) * G + g) * 2 + {0,1}], o[((seg * nstates + s) * G + g) * D + dim], written
// by an earlier launch on the stream) and writes fp16.  A row of exactly that length is its prefix
// states alone.  Shorter rows are attended in full.  A plan is one built for px.pages.
// kFused (with kCascade): the body runs on some workgroups of a launch whose other workgroups run
// the prefix pass (shared_prefix_fused_kernel): a cascade row's states are always published, and
// the ticket of each (row, kv head) -- fused_ticket -- counts the ranges holding the row and the
// prefix workgroups of that kv head; whoever arrives last merges those heads.  Rows of exactly the
// prefix length are left to the prefix workgroups.
// The arguments the first loads depend on come first (plan, pool, tables, query, the sizes and the
// grid), so that they can be preloaded into scalar registers at dispatch.  nb_arg: the workgroups
// running the body (gridDim.x for decode_rows_kernel).  PB: tokens per page.
// The kernel's body, run by workgroup bid of nb_arg.
template <int D, int G, int HKV, int S, bool kAppend, bool kStream, bool kPrep, bool kCascade, int PB, bool kFused>
__device__ __forceinline__ void decode_rows_body(
    const RowsLds<D, G, HKV, kPrep, kCascade, kFused ? 2 * HKV : 2>& sh, const int bid, const int32_t* plan, const f16* pool,
    const int32_t* block_tables, const f16* q, int32_t batch, int32_t max_pages, int32_t max_len, int32_t nb_arg,
    int64_t num_pages, f16* out, const int32_t* seq_lens, const uint8_t* active, float scale_log2, DecodeWorkspace ws,
    DecodeAppend ap, DecodePrep pp, DecodePrefix px) {
  constexpr int LPH = kWave / HKV;  // lanes per kv head
  constexpr int ROW = HKV * D;      // fp16 elements per token row
  constexpr int HQ = HKV * G;
  constexpr int GR = G < 2 ? G : 2;  // query heads per kv head merged per LDS round
  constexpr int D4 = D / 4;
  constexpr bool kApp = kAppend || kPrep;  // the step's appended rows are stored by this launch
  static_assert(ROW == 2 * kWave * 8, "a token row is two 16-byte chunks per lane");
  static_assert(G % GR == 0, "merge rounds cover the group");
  static_assert(!(kAppend && kPrep), "one append mode");
  static_assert(!(kCascade && (kAppend || kPrep)), "shared-prefix mode has no append");
  static_assert(!kPrep || (8 * LPH == D / 2), "a lane's two chunks are rotary partners");
  auto& s_cum = sh.s_cum;
  auto& s_wsum = sh.s_wsum;
  auto& s_m = sh.s_m;
  auto& s_l = sh.s_l;
  auto& s_acc = sh.s_acc;
  auto& s_ticket = sh.s_ticket;
  auto& s_casc = sh.s_casc;
  auto& s_app = sh.s_app;
  auto& s_q = sh.s_q;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int cap = min(max_pages * PB, max_len);
  const int pk = kCascade ? max(px.pages, 0) * PB : 0;  // prefix keys of a cascade row
  const int64_t num_slots = num_pages * PB;
  const int64_t nb = nb_arg;
  // XCD remap, as a select (a branch here would make the first kernel-argument loads wait apart)
  const int nbi = nb_arg;
  const int64_t blk = (nbi % kRowsXcds) == 0 ? (bid % kRowsXcds) * (nbi / kRowsXcds) + bid / kRowsXcds : bid;
  // split partials: O [slot][HQ][D] and (m, l) [slot][HQ][2], slot < batch + grid; and the merges
  const uint32_t n_slots = uint32_t(batch) + uint32_t(nb);
  const __amdgpu_buffer_rsrc_t r_o = make_rsrc(ws.o, n_slots * HQ * D * 2u);
  const __amdgpu_buffer_rsrc_t r_ml = make_rsrc(ws.ml, n_slots * HQ * 2u * 4u);
  // (kFused: 4 split states per round trip -- a cascade row's private keys span few ranges -- which
  // keeps the merges' scalar registers few in a kernel that shares them with the prefix pass)
  using MG = RowsMerge<D, G, HKV, kFused, kFused ? kFusedMergeBatch : kMergeBatch>;
  using PxBatch = typename MG::Px;
  using MergeLd = typename MG::Ld;
  const MG mg{r_o, r_ml, px, out};

  // Plan header, this range's record (its piece count and first piece) and its first page ids: one
  // round trip, issued first.  Every word is loaded before any is tested (the header check is a
  // bitwise and, not a chain of dependent loads).  The record is read before the header is checked;
  // the entry point has checked that the buffer holds a record for every workgroup and is 16-byte
  // aligned, so the reads stay inside it.
  bool planned = false;
  int64_t T = 0;
  int rec_n = 0;
  int ids_pl = 0, cum_pf = 0;
  i32x4 rec_a = i32x4{0, 0, 0, 0}, rec_b = i32x4{0, 0, 0, 0};  // rec[0 .. 7]: pieces, piece 0 (6 words), -
  const int32_t* rec = nullptr;
  if (plan != nullptr) {
    rec = plan + plan_rec0(batch) + blk * kPlanRec;
    const i32x4 h0 = *reinterpret_cast<const i32x4*>(plan);      // magic, batch, ranges, T
    const i32x4 h1 = *reinterpret_cast<const i32x4*>(plan + 4);  // grid, slots given, cap, 0
    rec_a = *reinterpret_cast<const i32x4*>(rec);
    rec_b = *reinterpret_cast<const i32x4*>(rec + 4);
    ids_pl = rec[64 + lane];
    cum_pf = plan[kPlanHdr + min(tid, batch)];
    planned = (h0[0] == kPlanMagic) & (h0[1] == batch) & (h1[0] == int(nb)) & (h1[2] == cap) &
              (!kApp | (h1[1] != 0)) & (h1[3] == pk);
    T = h0[3];
    rec_n = rec_a[0];
  }

  // Fused append: 16-byte chunks of every appended K and V row, spread over the grid.  No wave of
  // this launch reads these slots (the attention takes the appended token from new_k / new_v).
  // A thread's first chunk and its slot are loaded at launch; the chunk is stored once the
  // attention work is done.
  constexpr int kAppChunks = ROW / 8;  // per row of K (and of V)
  const int64_t app_items = kAppend ? int64_t(batch) * 2 * kAppChunks : 0;
  auto app_src = [&](int64_t it) __attribute__((always_inline)) {
    const int b = int(it / (2 * kAppChunks)), rem = int(it % (2 * kAppChunks));
    return (rem / kAppChunks == 0 ? ap.new_k : ap.new_v) + int64_t(b) * ROW + (rem % kAppChunks) * 8;
  };
  auto app_dst = [&](int64_t it, int slot) __attribute__((always_inline)) -> f16* {  // null: nothing to store
    const int rem = int(it % (2 * kAppChunks));
    return slot < 0 ? nullptr : ap.pool + (int64_t(rem / kAppChunks) * num_slots + slot) * ROW + (rem % kAppChunks) * 8;
  };
  const int64_t app_first = int64_t(bid) * kRowsThreads + tid;
  u32x4 app_data = u32x4{0u, 0u, 0u, 0u};
  int app_slot = -1;
  if constexpr (kAppend) {
    if (app_first < app_items) {
      app_data = ld16(app_src(app_first));
      app_slot = row_slot(ap.slots, active, int(app_first / (2 * kAppChunks)), num_slots);
    }
  }
  // Active rows with no keys get zeros (workgroup 0, at its end); their lengths and flags are
  // requested now and only tested there, so nothing waits for them at launch.
  int zero_sl = 1, zero_act = 0;
  if (bid == 0 && tid < batch) {
    zero_sl = seq_lens[tid];
    zero_act = active != nullptr ? int(active[tid]) : 1;
  }
  // kPrep: this wave's first item of the fallback store below, looked up at launch so that the end
  // of the kernel does not wait on it.
  const int64_t fb_first = int64_t(bid) + nb * (kRowsWaves - 1 - wave);
  const int64_t fb_step = nb * kRowsWaves;
  auto fb_item = [&](int64_t it, int& pos, int& slot) __attribute__((always_inline)) -> bool {
    const int b = int(it >> 1);
    pos = pp.positions[b];
    slot = row_slot(ap.slots, active, b, num_slots);
    return slot >= 0 && pos >= 0 && pos < pp.max_pos && pos >= row_keys(seq_lens, active, b, cap);
  };
  int fb_pos0 = 0, fb_slot0 = -1;
  bool fb_need0 = false;
  if constexpr (kPrep) {
    if (fb_first < 2 * int64_t(batch)) fb_need0 = fb_item(fb_first, fb_pos0, fb_slot0);
  }
  auto finish = [&]() __attribute__((always_inline)) {
    if constexpr (kPrep) {
      // The appended rows the attention did not take (their position is not among the row's keys:
      // rows without keys, or a position past them), normalised and rotated (K) or cast (V) and
      // stored as the pre-append kernel stores them; the others were stored by the wave that
      // prepared them for the attention.  A position outside the table, an inactive row or a slot
      // outside the pool stores nothing.  Item i = (row i / 2, K or V) goes to workgroup i % grid,
      // wave 7 - (i / grid) % 8, once the workgroup's attention work is done.
      const int hd = lane / LPH, col = lane % LPH;
      for (int64_t it = fb_first; it < 2 * int64_t(batch); it += fb_step) {
        const int b = int(it >> 1), kind = int(it & 1);
        int pos = fb_pos0, slot = fb_slot0;
        const bool need = it == fb_first ? fb_need0 : fb_item(it, pos, slot);
        if (!need) continue;
        float x1[8], x2[8];
        load_pairs<D>((kind == 0 ? pp.k : pp.v) + int64_t(b) * ROW + hd * D, col, x1, x2);
        if (kind == 0) {
          float w1[8], w2[8], c[8], sn[8];
          load_pairs<D>(pp.k_norm_w, col, w1, w2);
          load_pairs<D>(pp.rope + int64_t(pos) * D, col, c, sn);
          norm_rope_head<D, LPH>(x1, x2, w1, w2, c, sn, pp.eps);
        }
        f16* dst = ap.pool + (int64_t(kind) * num_slots + slot) * ROW + hd * D + 8 * col;
        st16(dst, pack_h8(x1));
        st16(dst + D / 2, pack_h8(x2));
      }
    }
    if constexpr (kAppend) {
      if (app_first < app_items) {
        f16* d0 = app_dst(app_first, app_slot);
        if (d0 != nullptr) st16(d0, app_data);
      }
      for (int64_t it = app_first + nb * kRowsThreads; it < app_items; it += nb * kRowsThreads) {
        f16* d = app_dst(it, row_slot(ap.slots, active, int(it / (2 * kAppChunks)), num_slots));
        if (d != nullptr) st16(d, ld16(app_src(it)));
      }
    }
    if (bid == 0) {
      for (int b0 = 0; b0 < batch; b0 += kRowsThreads) {
        const int b = b0 + tid;
        bool z = false, es = false;
        if (b < batch) {
          const bool live = b0 == 0 ? zero_act != 0 : (active == nullptr || active[b] != 0);
          const int len = b0 == 0 ? (zero_act != 0 ? max(0, min(zero_sl, cap)) : 0) : row_keys(seq_lens, active, b, cap);
          z = live && len == 0;
          es = kCascade && !kFused && pk > 0 && len == pk;  // (kFused: the prefix workgroups merge them)
        }
        if constexpr (kCascade) {
          uint64_t em = __ballot(es);
          while (em != 0) {  // this wave's cascade rows with no key after the prefix
            const int j = __builtin_ctzll(em);
            em &= em - 1;
            const int64_t row = b0 + wave * kWave + j;
            for (int i = lane; i < HQ * D4; i += kWave) {
              PxBatch pb;
              mg.px_load(row, i / D4, i % D4, 0, pb);
              mg.cascade_out(row, i / D4, i % D4, kNegBig, 0.f, f32x4{0.f, 0.f, 0.f, 0.f}, pb);
            }
          }
        }
        uint64_t mask = __ballot(z);
        while (mask != 0) {  // this wave's rows without keys, one at a time
          const int j = __builtin_ctzll(mask);
          mask &= mask - 1;
          const int64_t row = b0 + wave * kWave + j;
          for (int i = lane; i < HQ * D; i += kWave) out[row * HQ * D + i] = f16(0.f);
        }
      }
    }
  };

  // Unplanned (or a plan for other shapes): the offsets are built here, before anything else.
  // Planned: they go to LDS at the first merge barrier, for pieces the record does not describe.
  if (!planned) T = build_offsets(s_cum, s_wsum, seq_lens, active, batch, cap, pk, kCascade ? s_casc : nullptr);
  bool have_cum = !planned;
  // ws.plan_out (an unplanned call that builds the step's plan for the later layers): the same words
  // decode_plan_kernel writes -- workgroup 0 the header and the offsets, each workgroup its range's
  // record as it finds its pieces.
  int32_t* const pout = kFused || planned ? nullptr : ws.plan_out;
  int32_t* const prec = pout != nullptr ? pout + plan_rec0(batch) + blk * kPlanRec : nullptr;
  if (pout != nullptr && bid == 0) {
    if (tid == 0) {
      pout[0] = kPlanMagic;
      pout[1] = batch;
      pout[2] = int(range_count(nb, T));
      pout[3] = int(T);
      pout[4] = int(nb);
      pout[5] = kApp ? 1 : 0;
      pout[6] = cap;
      pout[7] = pk;
    }
    for (int i = tid; i <= batch; i += kRowsThreads) pout[kPlanHdr + i] = s_cum[i];
  }
  auto ensure_cum = [&]() __attribute__((always_inline)) {  // planned: s_cum valid after the next barrier
    if (!have_cum) {
      if (tid <= batch) s_cum[tid] = cum_pf;
      for (int i = tid + kRowsThreads; i <= batch; i += kRowsThreads) s_cum[i] = plan[kPlanHdr + i];
      have_cum = true;
    }
  };

  // nr <= min(workgroups, T) ranges, so that no range is empty (the split merge counts ranges).  A
  // range may still hold no key (only virtual positions); it then has no piece and takes no ticket.
  const int64_t nr = range_count(nb, T);
  if (blk >= nr) {
    if (prec != nullptr && tid <= kPlanIds) prec[tid == kPlanIds ? 0 : kPlanIds + tid] = 0;  // no piece
    finish();
    return;
  }
  const int64_t t0 = div_floor(T * blk, nr), t1 = div_floor(T * (blk + 1), nr);
  auto range_of = [&](int64_t t) -> int64_t { return div_floor((t + 1) * nr - 1, T); };
  // The piece after row prev (prev < 0: the range's first piece); b >= batch: none.
  auto next_piece = [&](int prev) -> RowPiece {
    RowPiece P;
    P.b = batch;
    P.a = P.e = P.first = P.slot = P.off = 0;
    P.nranges = 1;
    int b = prev < 0 ? locate_row(s_cum, batch, t0) : prev + 1;
    for (; b < batch; ++b) {
      const int cb = s_cum[b] + row_start_cost(batch);
      const int len = s_cum[b + 1] - cb;
      if (len <= 0) continue;
      if (cb >= t1) break;
      P.a = int(max<int64_t>(t0, cb) - cb);
      P.e = int(min<int64_t>(t1, int64_t(cb) + len) - cb);
      if (P.a >= P.e) break;
      P.b = b;
      P.first = int(range_of(cb));
      P.nranges = int(range_of(int64_t(cb) + len - 1)) - P.first + 1;
      P.slot = kApp ? row_slot(ap.slots, active, b, num_slots) : -1;
      // (planned: s_casc is not built; a piece the record does not hold is rare)
      if (kCascade && (planned ? row_keys(seq_lens, active, b, cap) >= pk : s_casc[b] != 0)) {
        P.off = pk;
        P.a += pk;
        P.e += pk;
      }
      break;
    }
    P.b = __builtin_amdgcn_readfirstlane(P.b);
    return P;
  };
  auto plan_piece = [&](int p) -> RowPiece {  // piece p < kPlanPieces of the record, clamped to the call
    int pc[6];
    if (p == 0) {  // loaded with the header
      pc[0] = rec_a[1]; pc[1] = rec_a[2]; pc[2] = rec_a[3];
      pc[3] = rec_b[0]; pc[4] = rec_b[1]; pc[5] = rec_b[2];
    } else {
#pragma unroll
      for (int j = 0; j < 6; ++j) pc[j] = rec[1 + 6 * p + j];
    }
    RowPiece P;
    P.b = min(max(pc[0], 0), batch - 1);
    // (kCascade: word 5 is the row's first streamed key, 0 or pk; the keys stay inside the cap)
    P.off = kCascade ? (pc[5] == pk ? pk : 0) : 0;
    P.a = min(max(pc[1] + P.off, 0), cap - 1);
    P.e = min(max(pc[2] + P.off, P.a + 1), cap);
    P.first = min(max(pc[3], 0), int(nr) - 1);
    P.nranges = min(max(pc[4], 1), int(nr) - P.first);
    P.slot = kCascade ? -1 : pc[5];
    return P;
  };

  const int hd = lane / LPH, col = lane % LPH;
  const int off0 = hd * D + 8 * col, off1 = off0 + 8 * LPH;  // this lane's two chunks of a token row
  const int64_t v_off = num_pages * PB * int64_t(ROW);

  int pend_n = 0, pend_b0 = 0, pend_b1 = 0, pend_f0 = 0, pend_f1 = 0, pend_np0 = 0, pend_np1 = 0;
  bool pend_c0 = false, pend_c1 = false;  // kCascade: the pending row is a cascade row

  constexpr int kItems = HKV * GR * D4;  // wave-merge items per round: one per thread at most
  static_assert(kItems <= kRowsThreads, "one merge item per thread and round");
  auto item_qh = [&](int r) { const int hg = tid / D4; return (hg / GR) * G + r * GR + hg % GR; };
  const int d4i = tid % D4;

  int prev = -1;
  int npieces = 0;
  for (int pi = 0;; ++pi) {  // one piece (row segment) per iteration; uniform over the workgroup
    if (planned && pi >= rec_n) break;
    const bool from_plan = planned && pi < kPlanPieces;
    const RowPiece P = from_plan ? plan_piece(pi) : next_piece(prev);
    if (P.b >= batch) break;
    const int b = P.b, a = P.a, e = P.e, slot_b = P.slot;
    prev = b;
    npieces = pi + 1;
    if (prec != nullptr && pi < kPlanPieces && tid < 6) {  // the piece's record (keys before the prefix offset)
      const int w = tid == 0 ? b : tid == 1 ? a - P.off : tid == 2 ? e - P.off : tid == 3 ? P.first
                  : tid == 4 ? P.nranges : (kApp ? slot_b : P.off);
      prec[1 + 6 * pi + tid] = w;
    }

    // Query rows (b, hd * G + g), chunks col and col + LPH; the piece's page ids, one per lane.
    f16x8 qv[G][2];
    // kPrep: the query comes from the fp32 projection (RMSNorm, rotary at the row's position, fp16;
    // zero when the position is outside the table), as the pre-append kernel writes it: wave g < G
    // prepares query head g of every kv head.  When the row's appended token (at its position) is
    // in this piece, wave G prepares its fp16 K row (normalised, rotated) and wave G + 1 its V row
    // (cast), to LDS -- where the wave that consumes the token reads them in place of the pool row --
    // and to the pool at the row's slot (the step's store of that row).  Each wave holds at most one
    // fp32 row, its weights and the rotary row.  The fp32 loads are issued here and the arithmetic
    // runs once the ring's first request is out, so the two round trips overlap; the workgroup then
    // exchanges the results through LDS at one barrier.
    int app_pos = -1;  // position of the row's appended token when it is in this piece (uniform)
    int app_page = -1;  // page id of the appended token's position
    bool pos_ok = false, k_maker = false, v_maker = false;
    const bool q_maker = kPrep && wave < G;
    float pc[8], psn[8], pw1[8], pw2[8], px1[8], px2[8];
    if constexpr (kPrep) {
      const int pos = pp.positions[b];
      pos_ok = pos >= 0 && pos < pp.max_pos;
      if (pos_ok && slot_b >= 0 && pos >= a && pos < e) {
        app_pos = pos;
        k_maker = wave == G;
        v_maker = wave == G + 1;
        app_page = block_tables[int64_t(b) * max_pages + pos / PB];  // read when the token comes up
      }
      if (q_maker || k_maker) {
        load_pairs<D>(pp.rope + int64_t(pos_ok ? pos : 0) * D, col, pc, psn);
        load_pairs<D>(q_maker ? pp.q_norm_w : pp.k_norm_w, col, pw1, pw2);
      }
      if (q_maker || k_maker || v_maker)
        load_pairs<D>(q_maker ? pp.q + (int64_t(b) * HQ + hd * G + wave) * D
                              : (k_maker ? pp.k : pp.v) + int64_t(b) * ROW + hd * D,
                      col, px1, px2);
    } else {
      const f16* qrow = q + (int64_t(b) * HQ + hd * G) * D;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        qv[g][0] = as_h8(ld16(qrow + g * D + 8 * col));
        qv[g][1] = as_h8(ld16(qrow + g * D + 8 * (col + LPH)));
      }
    }
    // kPrep, after the ring's first request (every wave of the workgroup calls it)
    auto prep_compute = [&]() __attribute__((always_inline)) {
      if (q_maker || k_maker) norm_rope_head<D, LPH>(px1, px2, pw1, pw2, pc, psn, pp.eps);
      const u32x4 h0 = pack_h8(px1), h1 = pack_h8(px2);
      if (q_maker) {
        *reinterpret_cast<u32x4*>(&s_q[wave][off0]) = pos_ok ? h0 : u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(&s_q[wave][off1]) = pos_ok ? h1 : u32x4{0u, 0u, 0u, 0u};
      }
      if (k_maker || v_maker) {
        const int kv = v_maker ? 1 : 0;
        *reinterpret_cast<u32x4*>(&s_app[kv][off0]) = h0;
        *reinterpret_cast<u32x4*>(&s_app[kv][off1]) = h1;
        f16* dst = ap.pool + (int64_t(kv) * num_slots + slot_b) * ROW;
        st16(dst + off0, h0);
        st16(dst + off1, h1);
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < G; ++g) {
        qv[g][0] = *reinterpret_cast<const f16x8*>(&s_q[g][off0]);
        qv[g][1] = *reinterpret_cast<const f16x8*>(&s_q[g][off1]);
      }
    };
    const int pg0 = a / PB;
    const int npg = (e - 1) / PB - pg0 + 1;
    const int32_t* bt = block_tables + int64_t(b) * max_pages + pg0;
    int ids0 = pi == 0 && from_plan ? ids_pl : bt[min(lane, npg - 1)];
    int ids1 = bt[min(lane + kWave, npg - 1)];
    if (prec != nullptr && pi == 0 && wave == 0) prec[kPlanIds + lane] = ids0;  // the first window's page ids
    int cur_w = 0;

    // this wave's tokens: positions a + wave + 8 i, i < nw
    const int rem = e - a - wave;
    const int nw = rem > 0 ? (rem + kRowsWaves - 1) / kRowsWaves : 0;
    auto rel_page = [&](int i) { return (a + wave + kRowsWaves * i) / PB - pg0; };
    auto page_of = [&](int i) -> int {
      const int rp = rel_page(i);
      return (rp >> 6) == cur_w ? __builtin_amdgcn_readlane(ids0, rp & 63) : __builtin_amdgcn_readlane(ids1, rp & 63);
    };
    auto shift = [&](int i) {  // token i's page enters the next 64-page window of the piece
      if ((rel_page(i) >> 6) != cur_w) {
        ids0 = ids1;
        ++cur_w;
        ids1 = bt[min(kWave * (cur_w + 1) + lane, npg - 1)];
      }
    };
    auto issue = [&](int i, u32x4 (&kr)[2], u32x4 (&vr)[2], bool& ok) {
      const int p = a + wave + kRowsWaves * i;
      const int phys = page_of(i);
      ok = phys >= 0 && int64_t(phys) < num_pages;
      const int64_t tok = int64_t(ok ? phys : 0) * PB + p % PB;
      const f16* kb = pool + tok * ROW;
      const f16* vb = pool + v_off + tok * ROW;
      if constexpr (kAppend) {
        if (ok && tok == slot_b) {  // the appended token (uniform): read it from new_k / new_v
          kb = ap.new_k + int64_t(b) * ROW;
          vb = ap.new_v + int64_t(b) * ROW;
        }
      }
      kr[0] = kStream ? ld16_stream(kb + off0) : ld16(kb + off0);
      kr[1] = kStream ? ld16_stream(kb + off1) : ld16(kb + off1);
      vr[0] = kStream ? ld16_stream(vb + off0) : ld16(vb + off0);
      vr[1] = kStream ? ld16_stream(vb + off1) : ld16(vb + off1);
    };

    float m[G], l[G], acc[G][16];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegBig;
      l[g] = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[g][j] = 0.f;
    }
    auto consume = [&](u32x4 (&kr)[2], u32x4 (&vr)[2], bool ok) {
      if (!ok) {  // a page id outside the pool contributes no key (uniform)
        vr[0] = u32x4{0u, 0u, 0u, 0u};
        vr[1] = u32x4{0u, 0u, 0u, 0u};
      }
      float vf[16];
      const f16x8 v0 = as_h8(vr[0]), v1 = as_h8(vr[1]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        vf[j] = float(v0[j]);
        vf[8 + j] = float(v1[j]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = dot8(qv[g][0], as_h8(kr[0]), 0.f);
        s = dot8(qv[g][1], as_h8(kr[1]), s);
        s = sum_lanes<LPH>(s);
        s = ok ? s * scale_log2 : -INFINITY;
        const float mn = fmaxf(m[g], s);
        const float alpha = exp2_fast(m[g] - mn);
        const float pr = exp2_fast(s - mn);
        l[g] = fmaf(l[g], alpha, pr);
        m[g] = mn;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[g][j] = fmaf(pr, vf[j], acc[g][j] * alpha);
      }
    };

    // S-stage register ring: token i + S - 1 is requested while token i is consumed.  The
    // requests are unconditional (past the wave's last token they re-read that token, which the
    // caches still hold), so the number of loads in flight is fixed and every wait counts exactly
    // -- a conditional request would make the compiler wait for all loads before each token.
    // The scheduling barriers keep the loads ahead of the arithmetic.
    u32x4 kb_[S][2], vb_[S][2];
    bool okb[S];
    // This wave's tokens i0 .. i1 - 1 through the ring; with_prep: the piece's preparation (kPrep)
    // runs on every wave between the first requests and the first token.
    auto ring = [&](int i0, int i1, bool with_prep) __attribute__((always_inline)) {
      // A short run (at most kBurst tokens: short calls, row heads and tails) requests every token
      // at once -- one round trip instead of one per S - 1 tokens.  The requests are unconditional
      // (indices clamped), so the waits count exactly here too.  (Not with kPrep, whose prepared
      // rows are live across the first requests.)
      if (!kPrep && i1 > i0 && i1 - i0 <= kBurst) {
        u32x4 kq[kBurst][2], vq[kBurst][2];
        bool okq[kBurst];
#pragma unroll
        for (int s = 0; s < kBurst; ++s) issue(min(i0 + s, i1 - 1), kq[s], vq[s], okq[s]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kBurst; ++s)
          if (i0 + s < i1) {
            shift(i0 + s);
            consume(kq[s], vq[s], okq[s]);
          }
        return;
      }
      if (i1 > i0) {
#pragma unroll
        for (int s = 0; s < S - 1; ++s) issue(min(i0 + s, i1 - 1), kb_[s], vb_[s], okb[s]);
      }
      if constexpr (kPrep) {
        if (with_prep) {
          __builtin_amdgcn_sched_barrier(0);
          prep_compute();
        }
      }
      if (i1 > i0) {
        int i = i0;
        for (; i + S <= i1; i += S) {
#pragma unroll
          for (int s = 0; s < S; ++s) {
            shift(i + s);
            const int sn = (s + S - 1) % S;
            issue(min(i + s + S - 1, i1 - 1), kb_[sn], vb_[sn], okb[sn]);
            __builtin_amdgcn_sched_barrier(0);
            consume(kb_[s], vb_[s], okb[s]);
          }
        }
#pragma unroll
        for (int s = 0; s < S - 1; ++s)
          if (i + s < i1) {
            shift(i + s);
            consume(kb_[s], vb_[s], okb[s]);
          }
      }
    };
    // kPrep: the wave that holds the row's appended token takes the ring up to it, the token itself
    // (from LDS when its slot is that position's slot in the table, as the step writes it; else the
    // pool row, as the two-launch step would read it), then the rest of its tokens.
    const int i_app = kPrep && app_pos >= 0 && (app_pos - a) % kRowsWaves == wave ? (app_pos - a) / kRowsWaves : nw;
    ring(0, i_app, true);
    if constexpr (kPrep) {
      if (i_app < nw) {
        shift(i_app);
        const int phys = app_page;
        bool ok = phys >= 0 && int64_t(phys) < num_pages;
        u32x4 kr[2], vr[2];
        if (ok && int64_t(phys) * PB + app_pos % PB == slot_b) {
          kr[0] = *reinterpret_cast<const u32x4*>(&s_app[0][off0]);
          kr[1] = *reinterpret_cast<const u32x4*>(&s_app[0][off1]);
          vr[0] = *reinterpret_cast<const u32x4*>(&s_app[1][off0]);
          vr[1] = *reinterpret_cast<const u32x4*>(&s_app[1][off1]);
        } else {
          issue(i_app, kr, vr, ok);
        }
        consume(kr, vr, ok);
        ring(i_app + 1, nw, false);
      }
    }

    // Merge the 8 waves through LDS: (m, l) of every query head, then the accumulators in rounds of
    // GR heads per kv head.  One thread per 4 output dims combines the waves' states (round r: item
    // tid < Hkv * GR * D / 4, at most one per thread).
    ensure_cum();
    const bool split = P.nranges != 1;      // the row is held by several ranges
    // kFused: a cascade row's state is always published; the prefix workgroups of the same launch
    // count towards its ticket, and whichever workgroup arrives last merges it
    const bool fcasc = kFused && P.off > 0;
    const bool publish = split || fcasc;
    const int64_t slot = int64_t(b) + blk;  // split-partial slot of (row b, this range)
    if (col == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_m[wave][hd * G + g] = m[g];
        s_l[wave][hd * G + g] = l[g];
      }
    }
#pragma unroll
    for (int r = 0; r < G / GR; ++r) {
#pragma unroll
      for (int gg = 0; gg < GR; ++gg) {
        const int g = r * GR + gg;
        f32x4* dst = s_acc[wave][hd * GR + gg];
        dst[2 * col] = f32x4{acc[g][0], acc[g][1], acc[g][2], acc[g][3]};
        dst[2 * col + 1] = f32x4{acc[g][4], acc[g][5], acc[g][6], acc[g][7]};
        dst[2 * (col + LPH)] = f32x4{acc[g][8], acc[g][9], acc[g][10], acc[g][11]};
        dst[2 * (col + LPH) + 1] = f32x4{acc[g][12], acc[g][13], acc[g][14], acc[g][15]};
      }
      __syncthreads();
      if (tid < kItems) {
        const int hg = tid / D4, d4 = d4i;
        const int qh = item_qh(r);
        PxBatch pb;
        if (kCascade && !publish && P.off > 0) mg.px_load(b, qh, d4, 0, pb);
        float mw[kRowsWaves];
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) {
          mw[w] = s_m[w][qh];
          M = fmaxf(M, mw[w]);
        }
        float L = 0.f;
        f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) {
          const float wt = exp2_fast(mw[w] - M);
          L = fmaf(wt, s_l[w][qh], L);
          const f32x4 a4 = s_acc[w][hg][d4];
          O = f32x4{fmaf(wt, a4[0], O[0]), fmaf(wt, a4[1], O[1]), fmaf(wt, a4[2], O[2]), fmaf(wt, a4[3], O[3])};
        }
        if (!publish) {
          mg.write_row(b, qh, d4, M, L, O, kCascade && P.off > 0, pb);
        } else {  // publish this range's state of the row; its ticket is taken at the end
          const float inv = L > 0.f ? 1.f / L : 0.f;
          const f16x4 oh = f16x4{f16(O[0] * inv), f16(O[1] * inv), f16(O[2] * inv), f16(O[3] * inv)};
          st_dev2(r_o, mg.o_off(slot, qh, d4), __builtin_bit_cast(f32x2, oh));
          if (d4 == 0) st_dev2(r_ml, mg.ml_off(slot, qh), f32x2{M, L});
        }
      }
      __syncthreads();
    }
    if (kFused && fcasc && !split) {
      // kFused: a cascade row held by this range alone -- its tickets now (one per kv head; the
      // prefix workgroups count too), and the merge of the kv heads this workgroup arrives last at
      wait_all_mem();
      __syncthreads();
      if (tid < HKV)
        s_ticket[tid] = __hip_atomic_fetch_add(fused_ticket(ws.count, batch, HKV, b, tid), 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      compiler_fence();
      uint32_t mask = 0;
#pragma unroll
      for (int h = 0; h < HKV; ++h) mask |= uint32_t(s_ticket[h] == uint32_t(px.nstates - 1)) << h;
      for (int idx = tid; idx < HQ * D4; idx += kRowsThreads)
        if ((mask >> (idx / D4 / G)) & 1u) mg.item(b, slot, 1, true, idx / D4, idx % D4);
      if (tid < HKV && ((mask >> tid) & 1u)) reset_ticket(fused_ticket(ws.count, batch, HKV, b, tid));
      __syncthreads();  // (s_ticket is read above before it is written again)
    }
    if (split) {
      // only the first and the last piece of a range can be split
      if (pend_n == 0) {
        pend_b0 = b; pend_f0 = P.first; pend_np0 = P.nranges; pend_c0 = P.off > 0;
      } else {
        pend_b1 = b; pend_f1 = P.first; pend_np1 = P.nranges; pend_c1 = P.off > 0;
      }
      ++pend_n;
    }
  }

  if (prec != nullptr) {
    if (tid == 0) prec[0] = npieces;
    if (npieces == 0 && tid < kPlanIds) prec[kPlanIds + tid] = 0;  // (only virtual positions)
  }
  if (!kFused && pend_n > 0) {
    // Tickets for the range's split rows: every partial store of the workgroup acknowledged first.
    wait_all_mem();
    __syncthreads();
    if (tid < pend_n)
      s_ticket[tid] = __hip_atomic_fetch_add(ws.count + (tid == 0 ? pend_b0 : pend_b1), 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    compiler_fence();  // the merge loads below stay behind the ticket
    // The rows this workgroup arrived last at are merged together: both rows' first round trips go
    // out before either is reduced.
    const bool last0 = s_ticket[0] == uint32_t(pend_np0 - 1);
    const bool last1 = pend_n > 1 && s_ticket[1] == uint32_t(pend_np1 - 1);
    if (last0 || last1) {
      const int64_t s00 = int64_t(pend_b0) + pend_f0, s10 = int64_t(pend_b1) + pend_f1;
      for (int idx = tid; idx < HQ * D4; idx += kRowsThreads) {
        const int qh = idx / D4, d4 = idx % D4;
        PxBatch p0, p1;
        MergeLd l0, l1;
        if (last0) {
          if (kCascade && pend_c0) mg.px_load(pend_b0, qh, d4, 0, p0);  // with the first round trip
          mg.issue(s00, pend_np0, qh, d4, l0);
        }
        if (last1) {
          if (kCascade && pend_c1) mg.px_load(pend_b1, qh, d4, 0, p1);
          mg.issue(s10, pend_np1, qh, d4, l1);
        }
        if (last0) {
          float M = kNegBig, L = 0.f;
          f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
          mg.finish(s00, pend_np0, qh, d4, l0, M, L, O);
          mg.write_row(pend_b0, qh, d4, M, L, O, kCascade && pend_c0, p0);
        }
        if (last1) {
          float M = kNegBig, L = 0.f;
          f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
          mg.finish(s10, pend_np1, qh, d4, l1, M, L, O);
          mg.write_row(pend_b1, qh, d4, M, L, O, kCascade && pend_c1, p1);
        }
      }
      if (tid == 0) {
        if (last0) reset_ticket(ws.count + pend_b0);
        if (last1) reset_ticket(ws.count + pend_b1);
      }
    }
  }
  if (kFused && pend_n > 0) {
    // Tickets for the range's split rows, every partial store of the workgroup acknowledged first:
    // one per kv head of a cascade row (the prefix workgroups count too), one per row otherwise.
    wait_all_mem();
    __syncthreads();
    if (tid < 2 * HKV) {
      const int r = tid / HKV, h = tid % HKV;
      const bool c = r == 0 ? pend_c0 : pend_c1;
      const int pb_ = r == 0 ? pend_b0 : pend_b1;
      if (r < pend_n && (c || h == 0))
        s_ticket[tid] = __hip_atomic_fetch_add(c ? fused_ticket(ws.count, batch, HKV, pb_, h) : ws.count + pb_, 1u,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    compiler_fence();  // the merge loads below stay behind the tickets
    // kv heads of each pending row this workgroup arrived last at
    const int npx = px.nstates - 1;
    uint32_t mk0 = 0, mk1 = 0;
#pragma unroll
    for (int h = 0; h < HKV; ++h) {
      mk0 |= uint32_t(pend_c0 ? s_ticket[h] == uint32_t(pend_np0 + npx - 1) : s_ticket[0] == uint32_t(pend_np0 - 1)) << h;
      mk1 |= uint32_t(pend_n > 1 && (pend_c1 ? s_ticket[HKV + h] == uint32_t(pend_np1 + npx - 1)
                                             : s_ticket[HKV] == uint32_t(pend_np1 - 1))) << h;
    }
    if ((mk0 | mk1) != 0) {
      const int64_t s00 = int64_t(pend_b0) + pend_f0, s10 = int64_t(pend_b1) + pend_f1;
      for (int idx = tid; idx < HQ * D4; idx += kRowsThreads) {
        const int qh = idx / D4, d4 = idx % D4;
        const bool last0 = (mk0 >> (qh / G)) & 1u, last1 = (mk1 >> (qh / G)) & 1u;
        PxBatch p0, p1;
        MergeLd l0, l1;
        if (last0) {
          if (pend_c0) mg.px_load(pend_b0, qh, d4, 0, p0);  // with the first round trip
          mg.issue(s00, pend_np0, qh, d4, l0);
        }
        if (last1) {
          if (pend_c1) mg.px_load(pend_b1, qh, d4, 0, p1);
          mg.issue(s10, pend_np1, qh, d4, l1);
        }
        if (last0) {
          float M = kNegBig, L = 0.f;
          f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
          mg.finish(s00, pend_np0, qh, d4, l0, M, L, O);
          mg.write_row(pend_b0, qh, d4, M, L, O, pend_c0, p0);
        }
        if (last1) {
          float M = kNegBig, L = 0.f;
          f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
          mg.finish(s10, pend_np1, qh, d4, l1, M, L, O);
          mg.write_row(pend_b1, qh, d4, M, L, O, pend_c1, p1);
        }
      }
      if (tid < 2 * HKV) {
        const int r = tid / HKV, h = tid % HKV;
        const bool c = r == 0 ? pend_c0 : pend_c1;
        const int pb_ = r == 0 ? pend_b0 : pend_b1;
        if (((r == 0 ? mk0 : mk1) >> h) & 1u) {
          if (c) reset_ticket(fused_ticket(ws.count, batch, HKV, pb_, h));
          else if (h == 0) reset_ticket(ws.count + pb_);
        }
      }
    }
  }
  finish();
}

template <int D, int G, int HKV, int S, bool kAppend, bool kStream, bool kPrep = false, bool kCascade = false,
          int PB = kRowsBlock>
__global__ __launch_bounds__(kRowsThreads) void decode_rows_kernel(
    const int32_t* __restrict__ plan, const f16* __restrict__ pool, const int32_t* __restrict__ block_tables,
    const f16* __restrict__ q, int32_t batch, int32_t max_pages, int32_t max_len, int32_t nb_arg,
    int64_t num_pages, f16* __restrict__ out, const int32_t* __restrict__ seq_lens,
    const uint8_t* __restrict__ active, float scale_log2, DecodeWorkspace ws, DecodeAppend ap, DecodePrep pp,
    DecodePrefix px) {
  using L = RowsLds<D, G, HKV, kPrep, kCascade>;
  __shared__ int s_cum[kRowsMaxBatch + 1];
  __shared__ int s_wsum[kRowsWaves];
  __shared__ float s_m[kRowsWaves][L::HQ];
  __shared__ float s_l[kRowsWaves][L::HQ];
  __shared__ f32x4 s_acc[kRowsWaves][HKV * L::GR][D / 4];
  __shared__ uint32_t s_ticket[2];
  __shared__ uint8_t s_casc[kCascade ? kRowsMaxBatch : 1];
  __shared__ __attribute__((aligned(16))) f16 s_app[kPrep ? 2 : 1][kPrep ? L::ROW : 8];
  __shared__ __attribute__((aligned(16))) f16 s_q[kPrep ? G : 1][kPrep ? L::ROW : 8];
  decode_rows_body<D, G, HKV, S, kAppend, kStream, kPrep, kCascade, PB, false>(
      L{s_cum, s_wsum, s_m, s_l, s_acc, s_ticket, s_casc, s_app, s_q}, int(blockIdx.x), plan, pool, block_tables, q, batch, max_pages, max_len, nb_arg, num_pages, out, seq_lens,
      active, scale_log2, ws, ap, pp, px);
}

}  // namespace ifn
