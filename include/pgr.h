/*
 * pgr.h -- C ABI of the MI355X decode-attention library (libpgr.so).
 *
 * Plain pointers, sizes and status codes only. Device pointers are HIP device addresses,
 * host pointers of the KV store are pinned memory owned by the store, `stream` is a
 * hipStream_t passed as void* (NULL = the default stream). Every call is asynchronous on
 * `stream` unless stated otherwise. Functions returning int return PGR_OK (0) or a negative
 * PGR_ERR_* code; pgr_last_error() then describes the failure (thread-local).
 *
 * Citations name the reference interface each entry point replaces (paths are relative to
 * the reference repository 3xecut0r/rust-llm-pager).
 */
#ifndef PGR_H_
#define PGR_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PGR_OK 0
#define PGR_ERR_INVALID (-1)
#define PGR_ERR_UNSUPPORTED (-2)
#define PGR_ERR_HIP (-3)
#define PGR_ERR_CAPACITY (-4)
#define PGR_ERR_STATE (-5)
#define PGR_ERR_KEY (-6)
#define PGR_ERR_BUDGET (-7)
#define PGR_ERR_INTERNAL (-8) /* internal failure; no exception crosses this boundary */

#define PGR_DTYPE_F16 0
#define PGR_DTYPE_BF16 1
#define PGR_DTYPE_F32 2 /* operator API only (q/k/v and finalize output); the KV store is 16-bit */

/* ---- library ------------------------------------------------------------------------- */

/* ABI version of this header (increments when an entry point is added or changed); 10. */
int pgr_abi_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* pgr_last_error(void);

/* ---- decode attention operator API --------------------------------------------------
 * Shapes follow pager_hf/streaming_attention.py: q [B, Hq, D]; k, v [B, Hkv, Tc, D]
 * contiguous; valid [B, Tc] int32 0/1 or NULL (all valid); active [B] int32 or NULL (all
 * active); online-softmax state m, l [B, Hq] and acc [B, Hq, D] fp32, updated in place.
 * q, k, v share one dtype: fp16, bf16 or fp32. D in {8, 16, 32, 64, 128, 256} (16-bit at
 * 32/64/128 runs on MFMA, the rest on a VALU kernel); Hq / Hkv <= 16; scale > 0; softcap <= 0
 * disables softcapping. Anything else returns PGR_ERR_UNSUPPORTED.
 * `workspace` must hold pgr_attn_workspace_bytes(...) bytes of device memory.
 */
#define PGR_MODE_FOLD 0
#define PGR_MODE_STATS 1
#define PGR_MODE_ACCUMULATE 2
#define PGR_MODE_FOLD_FIXED 3

size_t pgr_attn_workspace_bytes(int64_t batch, int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens,
                                int64_t head_dim, int mode, int64_t tokens_per_block);

/* Fold one KV chunk into (m, l, acc).
 * Replaces streaming_attention_step, pager_hf/streaming_attention.py:452-513
 * (kernel :77-185). */
int pgr_attn_step(const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active, float* m,
                  float* l, float* acc, int64_t batch, int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens,
                  int64_t head_dim, int dtype, float scale, float softcap, void* workspace, size_t workspace_bytes,
                  void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * fold as pgr_attn_step, same kernels and results, with its split-K partials in a static
 * device array of the library (8 MiB per GPU, held until the process ends) instead of a
 * workspace. It calls no allocating routine. A chunk whose partials exceed 8 MiB is
 * rejected with PGR_ERR_CAPACITY. With fp16/bf16 q/k/v, chunks with batch * num_kv_heads
 * <= 496 always fit at head_dim <= 128 and n_rep <= 16. fp32 q/k/v run a kernel with more,
 * smaller partial slots: there chunks with batch * num_kv_heads <= 496 always fit while
 * head_dim * n_rep <= 1024 (head_dim 64 at n_rep 16, 128 at n_rep 8); at head_dim 128 with
 * n_rep 16 a long chunk of even one row is rejected (1 x 16 x 65536 x 128 needs 8.5 MB).
 * Calls share their GPU's array. Outside graph capture the library orders them: a call on
 * another stream than the previous call's waits on the GPU (hipStreamWaitEvent) for the
 * previous call to finish, so calls from several streams or threads run one after another
 * in the order they were made. Calls recorded into graphs are not ordered by the library:
 * replays that may overlap on one GPU race, and the caller must serialize them. */
int pgr_attn_step_noalloc(const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active,
                          float* m, float* l, float* acc, int64_t batch, int64_t num_query_heads,
                          int64_t num_kv_heads, int64_t tokens, int64_t head_dim, int dtype, float scale,
                          float softcap, void* stream);

/* Fold one chunk's K into (m, l) only.
 * Replaces streaming_attention_stats_step, pager_hf/streaming_attention.py:516-560
 * (kernel :188-261). */
int pgr_attn_stats_step(const void* q, const void* k, const int32_t* valid, const int32_t* active, float* m, float* l,
                        int64_t batch, int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens, int64_t head_dim,
                        int dtype, float scale, float softcap, void* workspace, size_t workspace_bytes, void* stream);

/* With final (m, l): acc += P.V and block_mass[b, h, block_id_offset + j] = sum(p)/l per
 * tokens_per_block tile j (tokens_per_block a multiple of 16; block_mass [B, Hq, max_blocks]).
 * Replaces streaming_attention_accumulate_step, pager_hf/streaming_attention.py:563-621
 * (kernel :264-352). */
int pgr_attn_accumulate_step(const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active,
                             const float* m, const float* l, float* acc, float* block_mass, int64_t max_blocks,
                             int64_t block_id_offset, int64_t tokens_per_block, int64_t batch,
                             int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens, int64_t head_dim,
                             int dtype, float scale, float softcap, void* workspace, size_t workspace_bytes,
                             void* stream);

/* With final (m, l): acc += P.V for a non-block chunk (the tail); no mass, no active.
 * Replaces streaming_attention_fold_fixed_step, pager_hf/streaming_attention.py:624-665
 * (kernel :355-430). */
int pgr_attn_fold_fixed_step(const void* q, const void* k, const void* v, const int32_t* valid, const float* m,
                             const float* l, float* acc, int64_t batch, int64_t num_query_heads, int64_t num_kv_heads,
                             int64_t tokens, int64_t head_dim, int dtype, float scale, float softcap, void* workspace,
                             size_t workspace_bytes, void* stream);

/* No counterpart in the reference (its probe times whole calls with torch events,
 * bench/streaming_attention_kernel_scaling_probe.py:42-53). For measurement: with timing on,
 * every operator call of this process records a pair of events around its attention kernel
 * launch (not the merge launch after it); pgr_attn_kernel_time waits for them and returns the
 * summed milliseconds, the number of launches and the K/V bytes they read (K only in stats
 * mode), then forgets them. Process-wide; not for use under graph capture. */
int pgr_attn_set_timing(int32_t on);
int pgr_attn_kernel_time(double* ms, int64_t* launches, int64_t* bytes);
/* No counterpart in the reference. For measurement: the attention (fold) launch of
 * pgr_attn_step, without its merge, over each of n_chunks chunks (k[c], v[c], all of one
 * shape, no masks, no running state: the merge is what reads and updates it), `reps` rounds,
 * back to back between one pair of fence-free events on `stream`; returns the mean
 * microseconds per launch and the K/V bytes each launch reads. The workspace is
 * pgr_attn_step's (pgr_attn_workspace_bytes, fold mode). Synchronous; not under graph
 * capture. */
int pgr_attn_bench_step(const void* q, const void* const* k, const void* const* v, int32_t n_chunks, int64_t batch,
                        int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens, int64_t head_dim, int dtype,
                        float scale, void* workspace, size_t workspace_bytes, int32_t reps, double* us_per_launch,
                        int64_t* bytes_per_launch, void* stream);

/* No counterpart in the reference. For measurement: `reps` launches of a plain streaming read
 * of `bytes` (a positive multiple of 16) by workgroups x 256 threads, nothing written, launch r
 * reading srcs[r % n_src] (16-byte aligned device buffers); each launch between two fence-free
 * events on `stream`. Synchronous; returns the mean microseconds per launch: the ceiling a
 * kernel that reads the same bytes in one launch is measured against. */
int pgr_bench_stream_read(const void* const* srcs, int32_t n_src, int64_t bytes, int32_t workgroups, int32_t reps,
                          double* us_per_launch, void* stream);
/* The same `reps` launches back to back between one pair of fence-free events: the ceiling
 * for pgr_kv_bench_attention's back-to-back launches. */
int pgr_bench_stream_read_back_to_back(const void* const* srcs, int32_t n_src, int64_t bytes, int32_t workgroups,
                                       int32_t reps, double* us_per_launch, void* stream);

/* Fresh state for rows = B * Hq: m[r] = -inf, l[r] = 0, acc[r, :] = 0 (fp32, contiguous), in
 * one launch. Replaces streaming_attention_state_init, pager_hf/streaming_attention.py:444-449
 * (three fills there). */
int pgr_attn_state_init(float* m, float* l, float* acc, int64_t rows, int64_t head_dim, void* stream);

/* out[r, :] = (acc[r, :] / l[r]) rounded to dtype, for rows = B * Hq.
 * Replaces streaming_attention_finalize, pager_hf/streaming_attention.py:668-670. */
int pgr_attn_finalize(const float* acc, const float* l, void* out, int64_t rows, int64_t head_dim, int dtype,
                      void* stream);

/* ---- placement policy ----------------------------------------------------------------
 * Restatement of the Rust pager. Handles are opaque; not thread-safe per handle. */
typedef struct pgr_pager_metrics_s {
  uint64_t tokens;
  uint64_t vram_peak;
  uint64_t ram_peak;
  uint64_t swap_vram_ram;
  uint64_t swap_ram_ssd;
  double attention_mass_total;
  double attention_mass_vram;
} pgr_pager_metrics_t;

/* Replaces PyPager::new, pager/src/lib.rs:16-46 (core.rs:63-85). */
void* pgr_pager_new(uint64_t vram, uint64_t ram, uint64_t recent, uint64_t rebalance_interval, float promote_margin,
                    float ram_promote_margin, const char* policy);
/* Frees a pager handle (PyO3 object drop). */
void pgr_pager_free(void* pager);
/* Replaces PyPager::on_step, lib.rs:48-50 (core.rs:87-98). PGR_ERR_STATE when a rebalance
 * check divides by a zero rebalance_interval (the Rust code panics there). */
int pgr_pager_on_step(void* pager, uint64_t token_idx, uint32_t layer, const float* attention, size_t n);
/* Replaces PyPager::force_rebalance, lib.rs:52-54 (core.rs:100-107). */
int pgr_pager_force_rebalance(void* pager, uint64_t token_idx);
/* Number of blocks the pager tracks (length of tiers()). */
size_t pgr_pager_num_blocks(void* pager);
/* Replaces PyPager::tiers, lib.rs:60-62 (core.rs:113-122): writes min(cap, n) tiers, returns n. */
size_t pgr_pager_tiers(void* pager, uint8_t* out, size_t cap);
/* Replaces PyPager::vram_block_ids, lib.rs:64-66 (core.rs:124-130): writes min(cap, n), returns n. */
size_t pgr_pager_vram_block_ids(void* pager, uint64_t* out, size_t cap);
/* Replaces PyPager::metrics, lib.rs:56-58 (metrics.rs:4-27). */
int pgr_pager_metrics(void* pager, pgr_pager_metrics_t* out);

/* ---- paged KV store and fused decode -------------------------------------------------
 * One store holds the KV cache of many sessions (a session = rows sharing one placement)
 * for num_layers layers: an HBM slot pool per layer, a pinned host mirror per layer, and
 * an HBM staging ring for host-to-device streaming. */
typedef struct pgr_kv_config_s {
  int32_t num_layers;
  int32_t kv_heads;
  int32_t query_heads;
  int32_t head_dim;         /* 16, 32, 64, 128 or 256 */
  int32_t tokens_per_block; /* multiple of 16 */
  int32_t dtype;
  int64_t pool_slots;       /* HBM records (block x row) per layer */
  int64_t host_records;     /* pinned host records per layer */
  int64_t staging_slots;    /* records per staging buffer */
  int32_t staging_buffers;  /* ring depth, >= 1 (2 = double buffering) */
  int32_t blocks_per_workgroup; /* most block entries per workgroup (4..32; 0 = 32) */
  int32_t target_workgroups;    /* workgroups a launch aims for (0 = a multiple of the CU count) */
  int32_t stream_mode;          /* PGR_STREAM_DIRECT (0), _STAGED (1) or _MIRROR (2), see below */
} pgr_kv_config_t;

/* How decode reads host-resident blocks. DIRECT: the attention kernel reads them in place from
 * the pinned host mirror (mapped into the device address space) over the host link, in the
 * same launch as the HBM-resident blocks. STAGED: a copy kernel on the store's side stream
 * copies them into an HBM staging ring, double-buffered against the attention kernel. When a
 * step's host blocks fit one buffer and staging_buffers >= 2, pgr_kv_decode_layer(l) also
 * queues layer l+1's copies right after layer l's attention, so that they run under the
 * caller's work between the two layers. */
/* MIRROR: a ring of n = min(staging_buffers, num_layers) HBM buffers, each holding one layer's
 * share of a step's host records (the span from each row's first to last host record of the
 * step, rows packed; staging_slots records at first, grown by begin_step when a step needs
 * more). pgr_kv_begin_step has a host thread of the store queue, on the store's side stream
 * and behind the work queued on `stream` before begin_step, per layer l: DMA copies of the
 * layer's share into buffer l % n, then a word that the layer's attention launch waits for
 * (one lane per workgroup, a bounded wait of ~20 ms). For l >= n the thread first waits until
 * the merge launch of layer l - n has published the step's token in a pinned word: that
 * layer's attention launch, the buffer's last reader, has finished. A workgroup reads host
 * blocks from the ring buffer, or from the host in place if its word is still clear when the
 * wait ends (same data). The copies run beside whatever the caller runs between the step's
 * layers, including a replayed graph of the layers; the next begin_step waits for them.
 * Layers are expected in order: one decoded before the layers n below it waits its bounded
 * wait and reads the host. pgr_kv_sync waits for the copies queued so far, pgr_kv_destroy
 * for all of them and then ends the thread. For long-context sessions with a model between
 * the layers (a captured decode step, say). */
#define PGR_STREAM_DIRECT 0
#define PGR_STREAM_STAGED 1
#define PGR_STREAM_MIRROR 2

typedef struct pgr_kv_stats_s {
  uint64_t gpu_to_cpu_bytes, cpu_to_gpu_bytes, gpu_to_cpu_copies, cpu_to_gpu_copies;
  double gpu_to_cpu_sec, cpu_to_gpu_sec;
  uint64_t evict_bytes_copied, load_bytes_copied, stream_bytes, stream_copies;
} pgr_kv_stats_t;

/* Per step: resident_tokens / host_tokens / host_blocks count what the attention launches
 * read from HBM and from the host tier (where the bytes are); gather_blocks counts the
 * entries of the step's gather lists (blocks the placement put on the host tier; they differ
 * only for prompt blocks that wait for their first placement, see pgr_kv_apply_tiers).
 * plan_wait_ns: how long pgr_kv_begin_step waited for the GPU to finish reading the pinned
 * plan buffer it reuses (the host runs at most a step ahead of the GPU); the rest of the
 * host's time in the step's calls is its own work. */
typedef struct pgr_kv_step_stats_s {
  int64_t resident_tokens, host_tokens, host_blocks, copies, chunks, launches, work_items, gather_blocks;
  int64_t plan_wait_ns;
} pgr_kv_step_stats_t;

/* Creates a store (allocates HBM pools, pinned host mirror, staging). NULL on failure.
 * Replaces KVBlockStore.__init__, pager_hf/kv_block_store.py:41-56. */
void* pgr_kv_create(const pgr_kv_config_t* cfg);
/* Waits for the store's work and frees it. Call it before the process exits: the HIP runtime
 * tears itself down at exit, and a store still alive then would free device memory into a
 * runtime that no longer exists. */
void pgr_kv_destroy(void* kv);
/* New session with `rows` sequences and room for capacity_tokens tokens; lo_per_row = first
 * valid token per row (left padding), NULL = 0. Returns the session id (>= 0). */
int pgr_kv_add_session(void* kv, int32_t rows, int64_t capacity_tokens, const int32_t* lo_per_row);
int pgr_kv_remove_session(void* kv, int32_t sid);
/* Sliding window / padding: first valid token per row. Replaces the padding and window mask
 * fold of paged_model.py:964-982 (valid iff col > pos - window). */
int pgr_kv_set_lo(void* kv, int32_t sid, const int32_t* lo_per_row);
/* Beam-search row reordering: new row r takes old row src_rows[r]'s whole K/V history on
 * either tier (open block included) and its first valid token; a source row listed twice
 * is duplicated, one never listed is dropped. n_rows must equal the session's row count.
 * Replaces KVBlockStore.reorder_batch_rows, kv_block_store.py:229-254 (and the tail
 * index_select of PagedModel._reorder_batch, paged_model.py:636-644). Synchronous. */
int pgr_kv_reorder_rows(void* kv, int32_t sid, const int32_t* src_rows, int32_t n_rows, void* stream);
/* Declares the length of an empty session (prefill). Full blocks start host-side, holding no
 * data and charged to no tier until the next pgr_kv_apply_tiers places them: one placed on
 * the host then counts against the RAM budget (PGR_ERR_BUDGET past it), as the reference's
 * first offload of a prompt block does (kv_block_store.py:83-99). */
int pgr_kv_set_length(void* kv, int32_t sid, int64_t n_tokens);
/* Writes tokens [0, n_tokens) of (sid, row, layer) from k, v [Hkv, n_src, D] (device).
 * Replaces _build_initial_store + real_past_to_blocks, paged_model.py:1183-1192 and
 * kv_utils.py:38-61. Synchronous. */
int pgr_kv_import(void* kv, int32_t sid, int32_t row, int32_t layer, const void* k, const void* v, int64_t n_src,
                  int64_t n_tokens, void* stream);
/* Reads tokens [0, n_tokens) back into k, v [Hkv, n_tokens, D]. Synchronous.
 * Replaces reconstruct_past_from_store, kv_utils.py:112-178. */
int pgr_kv_export(void* kv, int32_t sid, int32_t row, int32_t layer, void* k, void* v, int64_t n_tokens, void* stream);
/* Registers block `block_id` (== current length / T, length block-aligned) from the reference
 * block layout key, value [L, B, T, Hkv, D] (device). Replaces KVBlockStore.put_gpu,
 * kv_block_store.py:58-67. */
int pgr_kv_put_block(void* kv, int32_t sid, int64_t block_id, const void* key, const void* value, void* stream);
/* Copies block `block_id` out in the reference layout [L, B, T, Hkv, D] (device), wherever it
 * lives, without moving it. Replaces KVBlockStore.get_any / get_gpu, kv_block_store.py:256-274.
 * Synchronous. */
int pgr_kv_get_block(void* kv, int32_t sid, int64_t block_id, void* key, void* value, void* stream);
/* Moves full blocks to the tier the pager assigned (0 = HBM, else host; ids >= n_tiers ->
 * host), ascending by id; writes moved ids. PGR_ERR_BUDGET with *fail_block when an
 * offload would exceed the RAM budget (earlier moves stay done). The record copies of one
 * call go evictions first, then loads (the move lists and byte counts are those of the
 * ascending order). A prompt block placed in HBM for the first time takes an HBM slot only
 * while the pool keeps two slots per row free, the most recent blocks first; the others count
 * as HBM-resident and have their bytes written to and read from the host records until a
 * later call loads or evicts them, so that a pool sized to the placement budget suffices
 * (PGR_ERR_CAPACITY when a load finds no slot). The copies are queued on
 * `stream`, after the work already there, and after the last decode step's launches when
 * those ran on another stream (that stream must still be valid); this store's later calls
 * on another stream wait for the copies through one event recorded here.
 * Replaces KVBlockStore.apply_tiers, kv_block_store.py:206-227 (offload :75-131, load :133-163). */
int pgr_kv_apply_tiers(void* kv, int32_t sid, const uint8_t* tiers, int64_t n_tiers, int64_t* to_gpu, int64_t* n_gpu,
                       int64_t* to_cpu, int64_t* n_cpu, int64_t* fail_block, void* stream);
/* RAM budget in bytes over all sessions (< 0: unlimited). kv_block_store.py:83-108. */
int pgr_kv_set_ram_budget(void* kv, int64_t bytes);
/* Opens a decode step over sessions sids[0..n): their rows, in order, are the sequences
 * (rows of q / k_new / v_new / out) of every decode_layer call of this step. */
int pgr_kv_begin_step(void* kv, const int32_t* sids, int32_t n, void* stream);
/* One layer of the step: appends k_new/v_new [S, Hkv, D] at each sequence's next position,
 * folds every in-scope block (HBM in place, host blocks streamed), writes out [S, Hq, D]
 * and, if mass_accum != NULL, adds the per-block attention mass (mean over the session's
 * rows and query heads) into mass_accum[session_in_step * accum_stride + block]. In a step
 * whose sessions have a pager scoring by mass (pgr_kv_attach_pager), that addition is made
 * for all layers at once, in layer order, by pgr_kv_end_step / pgr_kv_end_step_place (same
 * values; the layers' shares of the step, num_layers x rows x Hq x blocks floats, must fit
 * 64 MiB, else each layer adds its own as it runs).
 * window > 0: this layer's own sliding window (alternating-window models); it also masks
 * the stored positions c <= p - window, p being the current token's position (the rule
 * col > pos - W of paged_model.py:977-982). Tiles wholly below it are not read (the
 * reference reads every block and masks, paged_model.py:961); window <= 0: none.
 * Replaces the patched layer forward's gather + fold loop, paged_model.py:926-1086
 * (gather :878-924, tail append :955, mass :1041-1048). */
int pgr_kv_decode_layer(void* kv, int32_t layer, const void* q, const void* k_new, const void* v_new, void* out,
                        float* mass_accum, int64_t accum_stride, float scale, float softcap, int32_t window,
                        void* stream);
/* Closes the step: every session grows by one token; sessions whose open block became full
 * are written to completed[] (the new block id is then length / T - 1).
 * Replaces _append_new_full_blocks_from_grown_tail, paged_model.py:1210-1233. */
int pgr_kv_end_step(void* kv, int32_t* completed, int32_t* n_completed);
/* No counterpart in the reference (its decode step is not graph-captured). For callers that
 * capture decode steps in a HIP graph: writes up to cap values describing what the open
 * step's launches take as arguments (plan buffer and workspace pointers, grid sizes, mass
 * stride) and returns their number. A graph captured in a step stays valid for any later
 * step with the same values, since pgr_kv_begin_step writes each step's plan to the same
 * buffers before replay. Eager steps guard those buffers themselves (begin_step waits until
 * the GPU has read the buffer it is about to overwrite); captured and replayed launches do
 * not, so a replaying caller calls pgr_kv_step_replayed after each replay. */
int pgr_kv_step_signature(void* kv, int64_t* out, int64_t cap);
/* No counterpart in the reference (see pgr_kv_step_signature). After replaying the open
 * step's decode launches from a captured graph on `stream`: the next pgr_kv_begin_step waits
 * until the work queued on `stream` so far has run before it writes the plan buffer that
 * the replay reads, and placement on another stream waits for it too. */
int pgr_kv_step_replayed(void* kv, void* stream);
/* Attaches a placement handle (pgr_pager_new) to session sid; the store does not own it.
 * scores_from_mass != 0 for attention-scored policies (mass-driven scores). */
int pgr_kv_attach_pager(void* kv, int32_t sid, void* pager, int32_t scores_from_mass);
/* Closes the step like pgr_kv_end_step, then runs the per-step placement glue for every
 * session of the step that has a pager: scores (uniform, or this step's mass_accum averaged
 * over num_layers and normalized to sum 1), on_step(N-1), force_rebalance(N-1) when a block
 * completed, apply_tiers(tiers()). counts[5*i..] = {new block id or -1, n to HBM, n to host,
 * failing block or -1, n scores}; moves / scores (may be NULL) receive each session's moved
 * ids (to HBM then to host) and the scores handed to the pager. On a `stream` other than
 * the one the step's decode_layer calls used, the mass read-back and the tier moves first
 * wait for the step's launches (the decode stream must still be valid).
 * Replaces _forward_step's placement tail and _finalize_streaming_block_attention,
 * paged_model.py:768-812 and :865-876. */
int pgr_kv_end_step_place(void* kv, float* mass_accum, int64_t accum_stride, int32_t num_layers,
                          int32_t* completed, int32_t* n_completed, int64_t* counts, int64_t* moves,
                          int64_t moves_cap, double* scores, int64_t scores_cap, void* stream);
/* info[4] = {n_tokens, n_full_blocks, gpu_blocks, cpu_blocks}. */
int pgr_kv_session_info(void* kv, int32_t sid, int64_t* info);
/* Ascending full-block ids on HBM (gpu != 0) or host. Returns the count.
 * Replaces KVBlockStore.gpu_block_ids / cpu_block_ids, kv_block_store.py:185-189. */
int pgr_kv_block_ids(void* kv, int32_t sid, int32_t gpu, int64_t* out, int64_t cap);
/* Host-resident in-scope block ids streamed for sequence `seq` of the open step (ascending).
 * The gather index list of paged_model.py:907-916. Returns the count. */
int pgr_kv_step_host_blocks(void* kv, int32_t seq, int64_t* out, int64_t cap);
int pgr_kv_step_stats(void* kv, pgr_kv_step_stats_t* out);
/* Replaces KVBlockStore.stats / summary, kv_block_store.py:16-23, 191-204. */
int pgr_kv_stats(void* kv, pgr_kv_stats_t* out);
/* Replaces resident_gpu_bytes / resident_cpu_bytes, kv_block_store.py:179-183. */
int pgr_kv_resident_bytes(void* kv, int64_t* gpu, int64_t* cpu);
/* No counterpart in the reference (its blocks are torch allocations). Device memory the store
 * holds, in bytes: out[5] = {HBM slot pools, mirror-mode ring buffers, staged-mode staging
 * buffers, workspace (step plan, split-K partials, block mass), total}. */
int pgr_kv_hbm_bytes(void* kv, int64_t* out);
/* Bytes of one block of session sid over all layers and rows (kv_nbytes of a reference block). */
int pgr_kv_block_bytes(void* kv, int32_t sid, int64_t* bytes);
/* Event timing of the attention launches (for measurement; eager launches only, none under
 * graph capture) and, in the mirror mode, of each layer's DMA copies on the store's side stream.
 * pgr_kv_copy_time (outside a step) waits for the timed copies and returns their summed
 * milliseconds, the number of layer copy groups and their bytes, then forgets them. */
int pgr_kv_set_timing(void* kv, int32_t on);
int pgr_kv_kernel_time(void* kv, double* ms, int64_t* launches, int64_t* bytes);
/* No counterpart in the reference. For measurement (direct mode): with a step open whose first
 * layer has been decoded, launches the step's attention kernel (without per-block mass) for
 * every layer, `reps` times, back to back between two fence-free events on `stream`, and
 * returns the mean microseconds per launch and the K/V bytes each launch reads. Per-launch
 * events (pgr_kv_set_timing) add the time between each start marker and its dispatch. The
 * launches rewrite the step's split-K partials and each layer's current token: q, k_new and
 * v_new hold num_layers device pointers, each layer's inputs of the step, as given to
 * pgr_kv_decode_layer, with its scale and softcap. The merges are not repeated, so the step's
 * outputs stay as decode_layer wrote them. Synchronous; not under graph capture. */
int pgr_kv_bench_attention(void* kv, const void* const* q, const void* const* k_new, const void* const* v_new,
                           float scale, float softcap, int32_t reps, double* us_per_launch, int64_t* bytes_per_launch,
                           void* stream);
int pgr_kv_copy_time(void* kv, double* ms, int64_t* copies, int64_t* bytes);
/* Waits for all work of the store (both streams). */
int pgr_kv_sync(void* kv);

#ifdef __cplusplus
}
#endif

#endif /* PGR_H_ */
