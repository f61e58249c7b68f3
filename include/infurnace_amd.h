/*
 * infurnace_amd -- C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * One shared library, libinfurnace_hip.so, built from infurnace_amd/csrc/.
 * Every pointer argument is a DEVICE pointer owned by the caller (for example
 * torch.Tensor.data_ptr() of a ROCm tensor).  `stream` is a hipStream_t (NULL
 * = the default stream); every launch is asynchronous on it, so a store_kv
 * followed by a paged attention call on the same stream satisfies the
 * reference's write-before-read rule (docs/architecture.md:249-250).
 *
 * The library never allocates device memory.  Scratch space is a
 * caller-provided workspace.  Its first 256 KiB are split-KV tickets; they
 * must be zero when the workspace is created, and every call returns the
 * tickets it used to zero.  No kernel waits on another workgroup (a split is
 * merged by whichever workgroup arrives last), so no call can stall on the
 * device.  No C++ exception crosses this boundary: every
 * entry point returns IFN_OK (0) or a negative IFN_ERR_* code, checked on the
 * host before any launch (shape, alignment and workspace checks) or after it
 * (hipGetLastError).  Entry points hold no mutable global state, so distinct
 * streams may call them concurrently with distinct workspaces.
 *
 * Reference interfaces replaced (tylerguest/infurnace).  The reference's
 * modules for this path are 0-byte placeholders; their documented contract is
 *   docs/architecture.md:242-246   store_kv(kv_pool, slot_mapping, active_mask, new_k, new_v)
 *                                  paged_attention(query, kv_pool, block_tables,
 *                                                  sequence_lengths, active_mask)
 *   docs/architecture.md:225-235   kv_pool[layer, K_or_V, physical_page, page_offset,
 *                                  kv_head, head_dim]; slot = page * page_size + offset
 * and the code they replace is the contiguous store + SDPA at
 *   src/infurnace/executor/tinygrad/model.py:191-200 (decode) and :116-138 (prefill).
 *
 * Layouts (all C-contiguous, fp16 = IEEE binary16):
 *   kv pool, one layer   [2][num_pages][block_size][num_kv_heads][head_dim]   (K = 0, V = 1)
 *   kv pool, all layers  [num_layers][2][num_pages][block_size][num_kv_heads][head_dim]
 *   new_k / new_v        [num_tokens][num_kv_heads][head_dim]
 *   slot_mapping         int32 [num_tokens]; slot = page * block_size + offset
 *   active_mask          uint8 [rows]; 0 = inactive (may be NULL = all active)
 *   block_tables         int32 [batch][max_pages_per_seq]
 *   decode query/out     [batch][num_q_heads][head_dim]
 *   prefill query/out    [num_q_tokens][num_q_heads][head_dim]
 * Queries and K/V must be finite: the prefill is compiled assuming its scores
 * are never NaN, and its output is unspecified for NaN or Inf inputs.
 * Query head h reads kv head h / (num_q_heads / num_kv_heads) (GQA, as
 * tinygrad's scaled_dot_product_attention(enable_gqa=True) at model.py:200).
 */
#ifndef INFURNACE_AMD_H
#define INFURNACE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IFN_OK 0
#define IFN_ERR_INVALID_ARGUMENT (-1) /* null pointer, bad shape, bad count */
#define IFN_ERR_UNSUPPORTED (-2)      /* (head_dim, group, block_size) not compiled */
#define IFN_ERR_ALIGNMENT (-3)        /* device pointers must be 16-byte aligned */
#define IFN_ERR_WORKSPACE (-4)        /* workspace missing or smaller than required */
#define IFN_ERR_HIP (-5)              /* the HIP runtime reported a launch error */

/* Human-readable name of a status code (static string, never NULL). */
const char* ifn_status_string(int status);

/* ABI version: bumped whenever a signature or layout in this header changes. */
int ifn_abi_version(void);

/*
 * KV append: for each token t with active_mask[t] != 0 and
 * 0 <= slot_mapping[t] < num_pages * block_size, copy new_k[t] / new_v[t]
 * (num_kv_heads * head_dim fp16 each) into the K / V half of the layer's pool
 * at that slot.  Every other token writes nothing (inactive rows never touch a
 * shared dummy location).  Bit-exact copy.  Two active tokens with the same
 * slot race; the Python wrapper rejects that in its debug check.
 * Replaces: store_kv, docs/architecture.md:245 (placeholder
 * src/infurnace/kernels/kv_store.py, 0 B); contiguous precedent
 * src/infurnace/executor/tinygrad/model.py:191-196 and :134-138.
 * Requires head_dim % 8 == 0 and 16-byte aligned pointers.
 */
int ifn_store_kv(void* kv_pool_layer, int64_t num_pages, const int32_t* slot_mapping,
                 const uint8_t* active_mask, const void* new_k, const void* new_v,
                 int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                 int32_t block_size, void* stream);

/*
 * The same append for num_layers layers in one launch: kv_pool is the full
 * [num_layers][2][num_pages][block_size][num_kv_heads][head_dim] pool and
 * new_k / new_v are [num_layers][num_tokens][num_kv_heads][head_dim].  The
 * slot mapping and mask are shared by all layers (one token occupies the same
 * slot in every layer, docs/architecture.md:225-235).
 * Replaces: the per-layer store of model.py:134-138 repeated over the layer
 * loop at model.py:98 (one launch instead of num_layers).
 */
int ifn_store_kv_layers(void* kv_pool, int32_t num_layers, int64_t num_pages,
                        const int32_t* slot_mapping, const uint8_t* active_mask,
                        const void* new_k, const void* new_v, int32_t num_tokens,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        void* stream);

/* Workspace bytes ifn_paged_decode needs for these shapes (0 is never returned;
 * a negative-valued shape returns 0 and ifn_paged_decode rejects it). */
size_t ifn_paged_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t block_size, int32_t max_seq_len);

/*
 * Paged decode attention, one query token per sequence:
 *   out[b, h] = softmax(scale * q[b, h] . K[b, h/g, 0:L]^T) . V[b, h/g, 0:L],
 * L = seq_lens[b], keys gathered page by page through block_tables[b]
 * (fp16 in, fp32 accumulation, fp16 out).  scale <= 0 selects 1/sqrt(head_dim).
 * Rows with active_mask[b] == 0 write nothing.  An active row with L == 0
 * writes zeros.  L is clamped to [0, max_pages_per_seq * block_size] and to
 * max_seq_len; a page id outside [0, num_pages) contributes no keys (no
 * out-of-bounds read).  max_seq_len must be an upper bound of seq_lens: every
 * row's length is clamped to it, so a smaller value truncates attention.
 * Page loads are streamed (non-temporal hint): each page is expected to be read
 * by one row of the batch.  Batches whose rows share pages go through
 * ifn_paged_decode_shared_prefix (shared_pages == 0 when the shared pages are
 * not a common leading run), which keeps pages in the caches.
 * The workspace must be zero-filled once when created; every call leaves its
 * counters at zero again, so one workspace serves any number of calls on one
 * stream (calls overlapping on two streams need two workspaces).
 * Replaces: paged_attention (decode), docs/architecture.md:246 (placeholder
 * src/infurnace/kernels/paged_attention.py, 0 B); contiguous semantics
 * src/infurnace/executor/tinygrad/model.py:196-200.
 */
int ifn_paged_decode(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                     const int32_t* block_tables, int32_t max_pages_per_seq,
                     const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int32_t max_seq_len, float scale, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * The decode step's append and attention in one launch: the result (output and
 * pool) equals ifn_store_kv(kv_pool_layer, num_pages, slot_mapping,
 * active_mask, new_k, new_v, batch, ...) followed by ifn_paged_decode(...) on
 * the same stream.  new_k / new_v are [batch][num_kv_heads][head_dim] fp16;
 * row b appends at slot_mapping[b] when active (out-of-range slots store
 * nothing, as in ifn_store_kv).  The attention takes the appended token from
 * new_k / new_v instead of reading it back, so the store needs no ordering
 * against the reads.  Precondition (true for any paged KV state): an appended
 * slot is not read by another row of the same call.  Same workspace as
 * ifn_paged_decode.
 * Replaces: store_kv then paged_attention of one decode step
 * (docs/architecture.md:245-246,249-253; contiguous form
 * src/infurnace/executor/tinygrad/model.py:191-200).
 */
int ifn_paged_decode_append(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                            const int32_t* block_tables, int32_t max_pages_per_seq,
                            const int32_t* seq_lens, const uint8_t* active_mask,
                            const int32_t* slot_mapping, const void* new_k, const void* new_v,
                            int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t block_size, int32_t max_seq_len, float scale, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Step plan of a decode batch.  Every layer of a decode step attends with the
 * same block_tables, seq_lens, active_mask and (for the fused append)
 * slot_mapping; the split of the batch's keys over the CUs depends on nothing
 * else.  ifn_paged_decode_plan computes it once into `plan` (a device buffer
 * of ifn_paged_decode_plan_bytes), and the *_planned entry points below then
 * start each workgroup's page loads one round trip after launch instead of
 * three.  A plan is valid for calls with exactly the inputs it was built
 * from; it holds no pointers, so it may be built on one stream and used on
 * another once ordered after it.  plan_bytes == 0 means these shapes decode
 * without a plan (the planned entry points then ignore it).  slot_mapping may
 * be NULL for a plan used only by ifn_paged_decode_planned; a plan used by
 * ifn_paged_decode_append_planned must be built with the step's slots (else
 * that call computes the split itself).
 * Replaces: nothing in the reference (its decode step recomputes nothing per
 * layer because its SDPA reads contiguous rows, model.py:196-200); this is
 * the per-step half of paged_attention's decode (docs/architecture.md:246).
 */
size_t ifn_paged_decode_plan_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t block_size, int32_t max_pages_per_seq,
                                   int32_t max_seq_len);
int ifn_paged_decode_plan(void* plan, size_t plan_bytes, const int32_t* block_tables,
                          int32_t max_pages_per_seq, const int32_t* seq_lens, const uint8_t* active_mask,
                          const int32_t* slot_mapping, int64_t num_pages, int32_t batch,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t max_seq_len, void* stream);

/*
 * ifn_paged_decode and ifn_paged_decode_append with a step plan (NULL: none).
 * Same arguments, results and workspace otherwise; the output is bit-identical
 * to the unplanned call.  A plan built for other shapes or another batch size
 * is detected and ignored; one built from other lengths or tables of the same
 * shapes is not, and gives wrong results.
 * Replaces: paged_attention (decode), docs/architecture.md:246, and store_kv
 * then paged_attention (docs/architecture.md:245-246), as the unplanned calls.
 */
int ifn_paged_decode_planned(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                             const int32_t* block_tables, int32_t max_pages_per_seq,
                             const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t block_size, int32_t max_seq_len, float scale, const void* plan,
                             size_t plan_bytes, void* workspace, size_t workspace_bytes, void* stream);
int ifn_paged_decode_append_planned(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                                    const int32_t* block_tables, int32_t max_pages_per_seq,
                                    const int32_t* seq_lens, const uint8_t* active_mask,
                                    const int32_t* slot_mapping, const void* new_k, const void* new_v,
                                    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size, int32_t max_seq_len, float scale,
                                    const void* plan, size_t plan_bytes, void* workspace,
                                    size_t workspace_bytes, void* stream);

/*
 * The first layer's decode of a step, building the step's plan as it goes:
 * the same arguments as the *_planned calls above (and as
 * ifn_paged_decode_prep_append below), but `plan` is written, not read.  The
 * call decodes as the unplanned one does (bit-identical output) and leaves in
 * `plan` exactly the words ifn_paged_decode_plan would write for its inputs
 * (with slot_mapping for the append and pre-append forms, without for the plain
 * one), so the step's later layers run planned with no separate plan launch.
 * plan_bytes as ifn_paged_decode_plan_bytes; shapes that decode without a plan
 * (plan_bytes == 0) ignore `plan` and write nothing.  Later calls must be
 * ordered after this one (the same stream, or an event).
 * Replaces: as the unplanned calls (paged_attention's decode,
 * docs/architecture.md:245-246); it folds ifn_paged_decode_plan, which has no
 * reference counterpart, into the step's first launch.
 */
int ifn_paged_decode_planning(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                              const int32_t* block_tables, int32_t max_pages_per_seq,
                              const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                              int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, int32_t max_seq_len, float scale, void* plan,
                              size_t plan_bytes, void* workspace, size_t workspace_bytes, void* stream);
int ifn_paged_decode_append_planning(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                                     const int32_t* block_tables, int32_t max_pages_per_seq,
                                     const int32_t* seq_lens, const uint8_t* active_mask,
                                     const int32_t* slot_mapping, const void* new_k, const void* new_v,
                                     int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t block_size, int32_t max_seq_len, float scale,
                                     void* plan, size_t plan_bytes, void* workspace,
                                     size_t workspace_bytes, void* stream);
int ifn_paged_decode_prep_append_planning(void* out, const float* q, const float* k, const float* v,
                                          const float* q_norm_weight, const float* k_norm_weight,
                                          const float* rope_table, int32_t max_positions,
                                          const int32_t* positions, const int32_t* slot_mapping,
                                          void* kv_pool_layer, int64_t num_pages, const int32_t* block_tables,
                                          int32_t max_pages_per_seq, const int32_t* seq_lens,
                                          const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                          int32_t max_seq_len, float scale, float eps, void* plan,
                                          size_t plan_bytes, void* workspace, size_t workspace_bytes,
                                          void* stream);

/*
 * ifn_paged_decode without a workspace argument: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It allocates nothing: the split-KV
 * tickets and partial states live in a fixed device array of
 * ifn_paged_decode_noalloc_max_bytes() bytes per GPU (16 MiB), held until
 * the process ends.  Calls whose ifn_paged_decode_workspace_bytes exceed it
 * return IFN_ERR_WORKSPACE.  The first call on a device resolves the array's
 * address on the host; the array is zero from load (static storage), so no
 * call puts anything on `stream` but the decode itself, and a call made under
 * graph capture records only that.  Every call on a GPU shares that GPU's
 * array, so calls that overlap on one GPU (two streams, host threads or graph
 * replays) race: serialise them.
 * Output is bit-identical to ifn_paged_decode's.
 * Replaces: nothing in the reference (no counterpart); it serves the callers
 * that cannot allocate, with ifn_paged_decode's semantics.
 */
size_t ifn_paged_decode_noalloc_max_bytes(void);
int ifn_paged_decode_noalloc(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                             const int32_t* block_tables, int32_t max_pages_per_seq,
                             const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t block_size, int32_t max_seq_len, float scale, void* stream);

/* Workspace bytes ifn_paged_decode_shared_prefix needs for these shapes. */
size_t ifn_paged_decode_shared_prefix_workspace_bytes(int32_t batch, int32_t num_q_heads,
                                                      int32_t num_kv_heads, int32_t head_dim,
                                                      int32_t block_size, int32_t shared_pages);

/*
 * ifn_paged_decode for a batch whose rows share leading pages (a prefix-cache
 * hit): prefix_pages[0 .. shared_pages) are pages that every row of at least
 * shared_pages * block_size keys holds, in that order, at the start of its
 * block table.  The shared pages are read once for all rows (an MFMA pass of
 * every row's queries over them, split over keys), each row streams only its
 * own pages, and the two are merged as partial softmax states.  For head_dim
 * 128 with 8 kv heads and 16 or 32 query heads, and batches whose prefix pass
 * fits half the CUs (prefixes up to 8192 keys), that is one launch: part of
 * the grid runs the prefix pass while the rest streams the private pages, and
 * whichever workgroup finishes a (row, kv head) last merges it.  Otherwise
 * the prefix pass is one launch and the decode a second, which merges the
 * states itself when the token row (num_kv_heads x head_dim fp16) is 2 KiB,
 * else a third, combine launch per (row, kv head) does.  Inputs must be
 * finite (the one-launch form shares the prefill kernel's assumption that
 * scores are never NaN).  Same arguments, output and rules as
 * ifn_paged_decode otherwise; rows shorter than the prefix are attended in
 * full through their own table.  shared_pages == 0 is ifn_paged_decode with
 * cached page loads, for batches whose rows share pages anywhere in their
 * tables (prefix_pages may then be NULL).
 * head_dim 64 or 128 (IFN_ERR_UNSUPPORTED otherwise, as for prefill).
 * The precondition is not checked: a row whose leading table entries differ
 * from prefix_pages is attended as if it held prefix_pages.
 * Replaces: paged_attention (decode) over block tables with identical leading
 * ids -- the prefix cache's shared blocks, docs/roadmap.md:442-470,
 * docs/architecture.md:381-391 -- whose placeholder is
 * src/infurnace/kernels/paged_attention.py (0 B).
 */
int ifn_paged_decode_shared_prefix(void* out, const void* query, const void* kv_pool_layer,
                                   int64_t num_pages, const int32_t* prefix_pages, int32_t shared_pages,
                                   const int32_t* block_tables, int32_t max_pages_per_seq,
                                   const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                                   int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t block_size, int32_t max_seq_len, float scale, void* workspace,
                                   size_t workspace_bytes, void* stream);

/*
 * The step plan of a shared-prefix decode step (ifn_paged_decode_plan for
 * the whole-row kernel's shared-prefix mode): the split of the rows' own keys
 * after the first shared_pages pages, built once per step from the lengths,
 * the active mask and the tables that every layer shares.  plan_bytes as
 * ifn_paged_decode_plan_bytes; block_size 16.  Shapes decoded without a plan
 * (token rows other than 2 KiB) return IFN_OK and write nothing.  With
 * shared_pages == 0 it is ifn_paged_decode_plan without appended slots.
 * Replaces: nothing in the reference (see ifn_paged_decode_plan); this is the
 * per-step half of the shared-prefix decode below.
 */
int ifn_paged_decode_shared_prefix_plan(void* plan, size_t plan_bytes, const int32_t* block_tables,
                                        int32_t max_pages_per_seq, const int32_t* seq_lens,
                                        const uint8_t* active_mask, int32_t shared_pages, int64_t num_pages,
                                        int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t block_size, int32_t max_seq_len,
                                        void* stream);

/*
 * ifn_paged_decode_shared_prefix with a step plan from
 * ifn_paged_decode_shared_prefix_plan (NULL: none).  Same arguments,
 * workspace and output otherwise (bit-identical to the unplanned call; the
 * one-launch form splits the private keys over its own share of the CUs and
 * does not read the plan); a
 * plan for other shapes, batch size or shared_pages is detected and ignored,
 * one built from other lengths or tables of the same shapes gives wrong
 * results.
 * Replaces: as ifn_paged_decode_shared_prefix.
 */
int ifn_paged_decode_shared_prefix_planned(void* out, const void* query, const void* kv_pool_layer,
                                           int64_t num_pages, const int32_t* prefix_pages, int32_t shared_pages,
                                           const int32_t* block_tables, int32_t max_pages_per_seq,
                                           const int32_t* seq_lens, const uint8_t* active_mask, int32_t batch,
                                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                           int32_t block_size, int32_t max_seq_len, float scale,
                                           const void* plan, size_t plan_bytes, void* workspace,
                                           size_t workspace_bytes, void* stream);

/*
 * One prefill chunk's append and causal attention: the result (output and
 * pool) equals storing new_k / new_v ([num_q_tokens][num_kv_heads][head_dim]
 * fp16) at slot block_table[p / 16] * 16 + p % 16 for p = query_start + t
 * (skipped where that page id is outside the pool, as ifn_store_kv skips
 * such slots), then ifn_paged_prefill(...) on the same stream.  With
 * query_start % 32 == 0 this is one launch in which the attention takes the
 * chunk's keys from new_k / new_v; otherwise the store and the attention are
 * two launches.  Same workspace as ifn_paged_prefill.
 * Replaces: store_kv then paged_attention of one prefill chunk
 * (docs/architecture.md:245-246; contiguous form
 * src/infurnace/executor/tinygrad/model.py:116-138).
 */
int ifn_paged_prefill_append(void* out, const void* query, void* kv_pool_layer, int64_t num_pages,
                             const int32_t* block_table, int32_t max_pages, int32_t query_start,
                             int32_t num_q_tokens, const void* new_k, const void* new_v,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t block_size, float scale, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Workspace bytes ifn_paged_prefill needs for these shapes. */
size_t ifn_paged_prefill_workspace_bytes(int32_t num_q_tokens, int32_t query_start,
                                         int32_t num_q_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t block_size);

/*
 * Causal chunked-prefill paged attention for one sequence: query row i sits at
 * absolute position query_start + i and attends keys [0, query_start + i],
 * read through block_table (one row of max_pages int32).  The chunk's own K/V
 * must already be stored (append-then-attend).  fp16 in, fp32 accumulation,
 * fp16 out; QK^T and PV run on MFMA.  scale <= 0 selects 1/sqrt(head_dim).
 * Page ids outside [0, num_pages) contribute no keys.  The workspace follows
 * the same zero-once rule as ifn_paged_decode.
 * Replaces: paged_attention with a multi-token query, docs/architecture.md:246;
 * contiguous semantics src/infurnace/executor/tinygrad/model.py:116-132
 * (mask key_pos <= query_pos, query_pos = start_position + i).
 */
int ifn_paged_prefill(void* out, const void* query, const void* kv_pool_layer, int64_t num_pages,
                      const int32_t* block_table, int32_t max_pages, int32_t query_start,
                      int32_t num_q_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t block_size, float scale, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Pre-append step, fused: for every token t and head, q and k get a per-head
 * RMSNorm over head_dim (x * rsqrt(mean(x^2) + eps) * weight) and the
 * half-split rotary embedding at positions[t]; k and v are then cast to fp16
 * and stored at slot_mapping[t] (tokens with active_mask[t] == 0 or an
 * out-of-range slot store nothing); q is written to q_out as fp16.
 * q: fp32 [num_tokens][num_q_heads][head_dim]; k, v: fp32
 * [num_tokens][num_kv_heads][head_dim]; norm weights fp32 [head_dim];
 * rope_table fp32 [max_positions][head_dim] = cos(pos * f_i) for i < D/2
 * followed by sin(pos * f_i), f_i = base^(-2i/D).  A position outside
 * [0, max_positions) stores nothing and writes a zero q row.  head_dim <= 256.
 * Replaces: the norm/rope/cast/store sequence of
 * src/infurnace/executor/tinygrad/model.py:183-196 (decode) and :109-137
 * (prefill), with _rms_norm :11-13, _precompute_rope :19-23 and _apply_rope
 * :24-27.
 */
int ifn_qk_norm_rope_append(void* q_out, const float* q, const float* k, const float* v,
                            const float* q_norm_weight, const float* k_norm_weight,
                            const float* rope_table, int32_t max_positions,
                            const int32_t* positions, const int32_t* slot_mapping,
                            const uint8_t* active_mask, void* kv_pool_layer, int64_t num_pages,
                            int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t block_size, float eps, void* stream);

/*
 * One decode step of one layer from the fp32 projections, in one launch:
 * the pre-append of ifn_qk_norm_rope_append (q/k RMSNorm and rotary at
 * positions[b], k/v cast to fp16 and stored at slot_mapping[b]) and the
 * attention of ifn_paged_decode_planned over the result.  q: fp32
 * [batch][num_q_heads][head_dim]; k, v: fp32 [batch][num_kv_heads][head_dim];
 * the other arguments as in those two calls (plan may be NULL; a plan must
 * be built with slot_mapping).  `out` and the pool are bit-identical to
 * ifn_qk_norm_rope_append(...) followed by ifn_paged_decode_planned(...) on
 * the normalised fp16 query; the fp16 query itself is not written.  The
 * attention takes row b's appended token from the prepared k/v, at position
 * positions[b] when slot_mapping[b] is that position's slot in the row's
 * table (the decode step's invariant); the slot must not be read by any other
 * row or position of the call.  All float arrays 16-byte aligned; head_dim a
 * multiple of 8.  Shapes whose token row (num_kv_heads x head_dim fp16) is
 * not 2 KiB, or head_dim > 128, return IFN_ERR_UNSUPPORTED (run the two calls
 * instead).
 * Replaces: model.py:183-200 (norm, rope, cast, store and SDPA of a decode
 * step) as docs/architecture.md:245-246's store_kv then paged_attention.
 */
int ifn_paged_decode_prep_append(void* out, const float* q, const float* k, const float* v,
                                 const float* q_norm_weight, const float* k_norm_weight,
                                 const float* rope_table, int32_t max_positions,
                                 const int32_t* positions, const int32_t* slot_mapping,
                                 void* kv_pool_layer, int64_t num_pages, const int32_t* block_tables,
                                 int32_t max_pages_per_seq, const int32_t* seq_lens,
                                 const uint8_t* active_mask, int32_t batch, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 int32_t max_seq_len, float scale, float eps, const void* plan,
                                 size_t plan_bytes, void* workspace, size_t workspace_bytes,
                                 void* stream);

/*
 * One prefill chunk of one layer from the fp32 projections, in one launch:
 * the pre-append of ifn_qk_norm_rope_append (q/k RMSNorm and rotary, k/v cast
 * to fp16 and stored) and the causal attention of ifn_paged_prefill over the
 * result.  Token t of the chunk has position query_start + t, for its rotary
 * angle and for its cache slot block_table[p / 16] * 16 + p % 16 (slots whose
 * page id is outside the pool are not written, and their keys are not
 * attended).  q: fp32 [num_q_tokens][num_q_heads][head_dim]; k, v: fp32
 * [num_q_tokens][num_kv_heads][head_dim]; the other arguments as in those two
 * calls.  `out` and the pool are bit-identical to ifn_qk_norm_rope_append(...)
 * with positions query_start + t and those slots, followed by
 * ifn_paged_prefill(...) on the fp16 query; the fp16 query itself is not
 * written.  Requires query_start % 32 == 0 (else IFN_ERR_UNSUPPORTED: run the
 * two calls), query_start + num_q_tokens <= max_positions, every pointer
 * 16-byte aligned, and the shapes ifn_paged_prefill compiles.  Same workspace
 * as ifn_paged_prefill.
 * Replaces: model.py:109-138 (norm, rope, attention and cache write of a
 * prefill chunk) as docs/architecture.md:245-246's store_kv then
 * paged_attention.
 */
int ifn_paged_prefill_prep_append(void* out, const float* q, const float* k, const float* v,
                                  const float* q_norm_weight, const float* k_norm_weight,
                                  const float* rope_table, int32_t max_positions, void* kv_pool_layer,
                                  int64_t num_pages, const int32_t* block_table, int32_t max_pages,
                                  int32_t query_start, int32_t num_q_tokens, int32_t num_q_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float eps,
                                  float scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Zero the K and V of each listed page in every layer of the full pool
 * [num_layers][2][num_pages][block_size][num_kv_heads][head_dim].  Ids outside
 * [0, num_pages) are skipped.
 * Replaces: ContiguousKVCache.clear_slot,
 * src/infurnace/executor/tinygrad/buffers.py:67-81 (a released sequence's
 * pages return to the freshly allocated state, docs/phase2d.md:10-20).
 */
int ifn_zero_pages(void* kv_pool, int32_t num_layers, int64_t num_pages, const int32_t* page_ids,
                   int32_t num_ids, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                   void* stream);

/*
 * Copy page src_ids[i] to dst_ids[i] (K and V, every layer).  Destination ids
 * must be distinct and must not appear among the sources.  Pairs with an id
 * outside [0, num_pages) are skipped.
 * Serves: the private copy of a partial tail block when a sequence starts from
 * a shared prefix (partial blocks stay private, docs/architecture.md:381-391).
 */
int ifn_copy_pages(void* kv_pool, int32_t num_layers, int64_t num_pages, const int32_t* src_ids,
                   const int32_t* dst_ids, int32_t num_ids, int32_t num_kv_heads, int32_t head_dim,
                   int32_t block_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INFURNACE_AMD_H */
