// Native paged KV store and streaming decode executor.
//
// Memory layout (all of it owned by one PagedKV object):
//   * HBM pool, one arena per layer: `pool_slots` records. A record holds one block of one
//     sequence row for one layer: K [Hkv][T][D] then V [Hkv][T][D] (16-bit elements).
//     A block's slot index is the same in every layer's arena, so one block table serves
//     all layers.
//   * Host mirror, one pinned arena per layer: records addressed by (row, block id), each
//     row owning a contiguous range [host_off, host_off + capacity_blocks). Host-resident
//     blocks with consecutive ids are therefore one contiguous run, and are streamed to the
//     GPU with one multi-MiB copy per run.
//   * Staging ring in HBM (staged stream mode only): `staging_buffers` buffers of
//     `staging_slots` records, filled by host-to-device copies on a side stream and read by
//     the attention kernel in place. In the direct mode (default) the attention kernel reads
//     host blocks straight from the mirror over the host link, and imports, exports and tier
//     moves read and write the mirror in place through its device mapping.
//   * Mirror ring in HBM (mirror stream mode only): min(staging_buffers, num_layers) buffers,
//     each holding one layer's share of a step's host records (grown on demand). Layer l's
//     records go to buffer l % n by DMA once layer l - n has released it.
// Blocks are immutable once full, so a host copy stays valid after the block is loaded back
// to HBM and a later eviction of it needs no copy.
// Residency is logical (the tier the placement decided, what every move list and counter
// reports) and physical (where the record bytes are). They agree except for prompt blocks
// between their import and their first placement: those count as HBM-resident, as the
// reference's initial store holds them (paged_model.py:1183-1192), but only as many as the
// pool has room for get an HBM slot; the rest are written to the host mirror and read from
// there, so that the pool never needs more than the placement budget.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <functional>
#include <mutex>
#include <system_error>
#include <string>
#include <thread>
#include <vector>

#include "pgr_common.h"

namespace pgr {

struct PagedLaunch;

class PlacementPager;

struct PagedKVConfig {
  int num_layers = 1;
  int kv_heads = 0;
  int query_heads = 0;            // query heads (a multiple of kv_heads, at most 16 per KV head)
  int head_dim = 0;
  int tokens_per_block = 0;
  int dtype = kF16;
  int64_t pool_slots = 0;        // HBM records per layer
  int64_t host_records = 0;      // pinned host records per layer
  int64_t staging_slots = 0;     // records per staging buffer (mirror mode: initial records per ring buffer)
  int staging_buffers = 2;       // ring depth (staged mode: staging buffers; mirror mode: ring buffers)
  int blocks_per_workgroup = 32; // most block entries folded by one workgroup (4 waves)
  int target_workgroups = 0;     // workgroups a launch aims for (0: a multiple of the CU count)
  int stream_mode = 0;           // 0: kernels read host blocks in place; 1: staged copies; 2: HBM mirror
};

struct StoreStats {
  // Logical moves, counted the way kv_block_store.py:110-163 counts them.
  uint64_t gpu_to_cpu_bytes = 0, cpu_to_gpu_bytes = 0;
  uint64_t gpu_to_cpu_copies = 0, cpu_to_gpu_copies = 0;
  double gpu_to_cpu_sec = 0.0, cpu_to_gpu_sec = 0.0;
  // Physical copy traffic issued by this object.
  uint64_t evict_bytes_copied = 0;    // D2H bytes actually copied (host copy was stale or absent)
  uint64_t load_bytes_copied = 0;     // H2D bytes into pool slots
  uint64_t stream_bytes = 0;          // H2D bytes streamed into staging for attention
  uint64_t stream_copies = 0;         // H2D copy calls for attention streaming
};

struct StepStats {
  int64_t resident_tokens = 0;  // in-scope tokens read from the HBM pool (incl. the open block)
  int64_t host_tokens = 0;      // in-scope tokens streamed from host (whole blocks)
  int64_t host_blocks = 0;      // (block, row) records read from the host tier (physical residency)
  int64_t copies = 0;           // H2D copy calls per layer
  int64_t chunks = 0;
  int64_t launches = 0;         // attention kernel launches per layer
  int64_t work_items = 0;
  int64_t gather_blocks = 0;    // (block, row) entries of the gather lists (logical host residency)
  int64_t plan_wait_ns = 0;     // begin_step's wait for the GPU to finish reading the plan buffer
};

// Device memory a store holds, in bytes.
struct HbmBytes {
  int64_t pool = 0;       // HBM slot pools, all layers
  int64_t mirror = 0;     // mirror-mode ring buffers
  int64_t staging = 0;    // staged-mode staging buffers
  int64_t workspace = 0;  // step plan, split-K partials, block mass
  int64_t total = 0;
};

// One host thread that runs submitted jobs one at a time: here, the HIP calls that queue a
// step's mirror-mode copies, so that the caller's thread goes on to launch the step while
// they are issued. Started by the first submit.
class HostWorker {
 public:
  HostWorker() = default;
  HostWorker(const HostWorker&) = delete;
  HostWorker& operator=(const HostWorker&) = delete;
  ~HostWorker() { stop(); }
  // Runs `job` on the worker thread (here, at once, if no thread can be started). A job
  // submitted before must have been waited for.
  void submit(std::function<hipError_t()> job);
  // Returns once the submitted job (if any) has run, with its result; hipSuccess if none.
  hipError_t wait();
  bool started() const { return thread_.joinable(); }
  bool busy();  // a submitted job has not finished
  void stop();  // runs a submitted job to its end, then ends the thread

 private:
  void run();
  std::thread thread_;
  std::mutex mu_;
  std::condition_variable cv_;
  std::function<hipError_t()> job_;
  bool pending_ = false;
  bool stop_ = false;
  hipError_t result_ = hipSuccess;
};

class PagedKV {
 public:
  explicit PagedKV(const PagedKVConfig& cfg);
  ~PagedKV();
  int init();  // allocates; returns a Status
  const std::string& error() const { return err_; }

  // Sessions (rows share placement). Returns the session id or a negative Status.
  int add_session(int rows, int64_t capacity_tokens, const int32_t* lo_per_row);
  int remove_session(int sid);
  int set_lo(int sid, const int32_t* lo_per_row);
  // Beam-search row reordering (kv_block_store.py:229-254): new row r takes old row
  // src[r]'s whole history (every block on either tier, the open block included) and its lo;
  // n must equal the session's row count. Synchronous.
  int reorder_rows(int sid, const int32_t* src, int n, hipStream_t stream);

  // Setup: write the first n_tokens of one (session, row, layer) from k, v [Hkv, n_src, D]
  // (device memory, row stride n_src) and set the session length. Blocks go to the pool when
  // resident, to the host mirror otherwise. Requires the session's token count to be
  // n_tokens already (set_length) so residency is known.
  int set_length(int sid, int64_t n_tokens);
  int import_tokens(int sid, int row, int layer, const void* k, const void* v, int64_t n_src, int64_t n_tokens,
                    hipStream_t stream);
  // Read back tokens [0, n) of one (session, row, layer) into k, v [Hkv, n, D] (device).
  int export_tokens(int sid, int row, int layer, void* k, void* v, int64_t n_tokens, hipStream_t stream);

  // Reference-layout block I/O: key, value [L, B, T, Hkv, D] (device). put_block appends
  // block `block_id` (== length / T of a block-aligned session) to HBM; get_block copies a
  // block out wherever it lives.
  int put_block(int sid, int64_t block_id, const void* key, const void* value, hipStream_t stream);
  int get_block(int sid, int64_t block_id, void* key, void* value, hipStream_t stream);

  // Placement (kv_block_store.py:206-227 semantics) for full blocks of a session.
  // tiers[i] == 0 -> HBM, anything else -> host; ids >= n_tiers -> host.
  // Fills to_gpu / to_cpu (ascending) and returns their counts via *n_gpu / *n_cpu.
  // On budget overflow returns kErrBudget with *fail_block set; moves done before it stay.
  int apply_tiers(int sid, const uint8_t* tiers, int64_t n_tiers, int64_t* to_gpu, int64_t* n_gpu, int64_t* to_cpu,
                  int64_t* n_cpu, int64_t* fail_block, hipStream_t stream);
  void set_ram_budget(int64_t bytes) { ram_budget_ = bytes; }
  double ram_usage_ratio() const;

  // Decode step over `sids` (their rows, in order, are the sequences of q/out).
  int begin_step(const int32_t* sids, int n, hipStream_t stream);
  // window > 0: this layer also masks stored positions <= current - window.
  int decode_layer(int layer, const void* q, const void* k_new, const void* v_new, void* out, float* mass_accum,
                   int64_t accum_stride, float scale, float softcap, int window, hipStream_t stream);
  int end_step(int32_t* completed_sessions, int* n_completed);
  // Everything the open step's launches take as arguments besides the caller's tensors:
  // plan buffer and workspace pointers, grid sizes, the mass stride. Launches captured in a
  // graph stay valid for a later step with the same signature (begin_step writes each step's
  // plan to the same buffers).
  // Returns the number of values (writes at most cap), or kErrState outside a step.
  int step_signature(int64_t* out, int64_t cap) const;
  // The open step's launches were replayed from a captured graph on `stream` (no eager
  // decode_layer call made them): marks the step's plan buffer as read once the work queued
  // on `stream` so far has finished, so that a later begin_step does not overwrite it before
  // the replayed launch that reads it has run.
  int step_replayed(hipStream_t stream);

  // Per-step placement glue of paged_model.py:768-812 for sessions with an attached pager:
  // scores (uniform, or this step's block mass averaged over layers and normalized), then
  // pager on_step(N-1), force_rebalance(N-1) if a block completed, apply_tiers(tiers()).
  // Closes the step like end_step. counts gets 5 values per session of the step:
  // {new block id or -1, n moved to HBM, n moved to host, failing block or -1, n scores};
  // moves gets each session's to-HBM then to-host ids, scores the values handed to the
  // pager (before f32 rounding); both may be null.
  int attach_pager(int sid, PlacementPager* pager, bool scores_from_mass);
  int end_step_place(float* mass_accum, int64_t accum_stride, int num_layers, hipStream_t stream,
                     int32_t* completed, int* n_completed, int64_t* counts, int64_t* moves, int64_t moves_cap,
                     double* scores, int64_t scores_cap);

  // Introspection.
  int session_info(int sid, int64_t* n_tokens, int64_t* n_full, int64_t* gpu_blocks, int64_t* cpu_blocks) const;
  int block_ids(int sid, int gpu, int64_t* out, int64_t cap) const;  // ascending
  int step_host_blocks(int seq_index, int64_t* out, int64_t cap) const;
  const StepStats& step_stats() const { return step_stats_; }
  StoreStats stats();
  int64_t block_bytes_all_layers(int sid) const;
  int64_t resident_gpu_bytes() const;
  int64_t resident_cpu_bytes() const;
  HbmBytes hbm_bytes() const;

  // Optional timing of the attention launches (HIP events on the compute stream).
  void set_timing(bool on) { timing_ = on; }
  int kernel_time(double* ms, int64_t* launches, int64_t* bytes);
  // Measurement only: the open step's attention launches (no per-block mass) for every layer,
  // reps times back to back between two fence-free events (direct mode, after the step's
  // first decode_layer). See pgr_kv_bench_attention.
  int bench_attention(const void* const* q, const void* const* k_new, const void* const* v_new, float scale,
                      float softcap, int reps, hipStream_t stream, double* us_per_launch, int64_t* bytes_per_launch);
  // Mirror mode with timing on: the DMA copies of each layer's share, event-timed on the copy
  // stream. Waits for them; returns the summed milliseconds, the layer copy groups and bytes.
  int copy_time(double* ms, int64_t* copies, int64_t* bytes);
  int sync();

  const PagedKVConfig& cfg() const { return cfg_; }

 private:
  struct Row {
    int64_t host_off = -1;
    int32_t lo = 0;
  };
  struct Session {
    bool live = false;
    int rows = 0;
    int64_t n_tokens = 0;
    int64_t capacity_blocks = 0;
    std::vector<Row> row;
    // slot[b * rows + r] for block b, row r; -1 when on host.
    std::vector<int32_t> slot;
    std::vector<uint8_t> host_valid;  // [b * rows + r]
    std::vector<uint8_t> on_gpu;      // logical residency per full block [b]
    // [b]: 1 once block b's bytes are charged to a tier. A prompt's blocks (set_length)
    // hold no data until their first placement, which charges them against the RAM budget.
    std::vector<uint8_t> placed;
    PlacementPager* pager = nullptr;  // not owned
    bool scores_from_mass = false;
  };
  struct CopyCmd {
    int64_t host_rec;   // first host record
    int64_t stage_rec;  // first staging record (global index over all buffers)
    int64_t count;      // records
    int chunk;
  };
  struct PendingTiming {
    hipEvent_t start, stop;
    int64_t bytes;
  };

  int fail(int code, const std::string& msg);
  int hip_fail(hipError_t e, const char* what);
  size_t rec_bytes() const;
  int alloc_slot();
  void free_slot(int32_t s);
  int64_t host_alloc(int64_t n);
  void host_free(int64_t off, int64_t n);
  int ensure_workspace(size_t bytes);
  int default_workgroups() const;
  int ensure_block_capacity(Session& s, int64_t blocks);
  // Physical moves of block b (every row): into HBM slots (a load, copied from the host
  // record if that holds data) or out of them (an eviction, copied to the host record unless
  // that holds the data already). The copies are collected and issued by apply_tiers.
  int load_block(Session& s, int64_t b);
  void evict_block(Session& s, int64_t b);
  int resolve_timing();
  // Block mass of a step run with deferred mass (sessions whose pager scores by mass): each
  // layer's merge writes that layer's normalized per-block weights into mass_w_; one launch
  // at the end of the step averages them over rows and heads, adds them up over the layers
  // in layer order into mass_accum, and clears mass_w_ for the next step.
  int finish_step_mass(float* mass_accum, int64_t accum_stride, hipStream_t stream);
  // Closes the open step (every session grows by one token).
  int close_step(int32_t* completed, int* n_completed);
  // Record index lists for the copy kernels live in pinned host memory that the kernels read
  // in place, in a small ring so a list is not overwritten while a queued kernel still
  // needs it.
  struct IndexBuf {
    int64_t* host = nullptr;  // pinned
    int64_t* dev = nullptr;   // device address of `host`
    size_t cap = 0;           // entries
    hipEvent_t done = nullptr;
    bool pending = false;
  };
  static constexpr int kIndexBufs = 4;
  int acquire_index_buf(size_t n, IndexBuf** out);
  // Copies records (from, to) pairs for every layer in one launch; tables 0 (HBM pool) or
  // num_layers (host mirror) select source and destination. Clears `pairs`.
  int launch_copies(std::vector<int64_t>& pairs, int src_tbl, int dst_tbl, hipStream_t stream);

  PagedKVConfig cfg_;
  std::string err_;
  std::vector<void*> pool_;   // per layer
  std::vector<void*> host_;   // per layer (pinned)
  std::vector<void*> host_dev_;  // per layer: device address of the pinned arena
  void* stage_ = nullptr;
  void* ws_ = nullptr;
  size_t ws_bytes_ = 0;
  int n_cu_ = 0;                  // compute units of the device
  int device_ = 0;                // the device current at init
  void** bases_dev_ = nullptr;  // [pool_0 .. pool_{L-1}, host_dev_0 .. host_dev_{L-1}] on the device
  IndexBuf index_bufs_[kIndexBufs];
  int next_index_buf_ = 0;
  std::vector<int64_t> evict_pairs_, load_pairs_;  // moves of the current apply_tiers call
  // The step plan goes to one of two pinned buffers, alternately, so that the host can write
  // the next step's plan while the GPU still reads this one.
  // In direct mode the GPU's last read of a buffer is the step's first attention launch; the
  // merge launch after it stores the buffer's token into a pinned flag word, which the host
  // polls. An event recorded between the two launches held the merge back by ~4.5 us per
  // step. Staged mode waits on `read` instead.
  struct PlanBuf {
    void* host = nullptr;  // pinned
    void* dev = nullptr;   // its device mapping
    size_t bytes = 0;
    hipEvent_t read = nullptr;  // after the GPU's last read of this buffer
    bool pending = false;
    bool by_flag = false;       // pending on the flag word rather than on `read`
    uint32_t token = 0;         // flag value that marks the pending read as done
    hipStream_t stream = nullptr;  // stream of the pending read
  };
  PlanBuf plan_bufs_[2];
  uint32_t* plan_flags_ = nullptr;      // pinned, one word per plan buffer
  uint32_t* plan_flags_dev_ = nullptr;  // their device mapping
  uint32_t plan_token_ = 0;             // last token handed out
  int wait_plan_flag(const PlanBuf& pb, int idx);
  int plan_buf_ = 0;             // buffer of the open step
  bool plan_on_device_ = false;  // the workspace holds the open step's plan
  size_t plan_aux_bytes_ = 0;    // plan bytes ahead of the work items
  size_t plan_work_off_ = 0;     // offset of the work items in the plan
  float* mass_host_ = nullptr;  // pinned readback of the step's block mass
  size_t mass_host_floats_ = 0;
  hipStream_t copy_stream_ = nullptr;
  hipEvent_t plan_uploaded_ = nullptr;
  hipEvent_t stage_copies_done_ = nullptr;  // after the last staging copy on the copy stream
  // Tier moves run on the stream apply_tiers was given; moves_done_ is recorded there right
  // after them. Work that a later call queues on another stream waits for that event once
  // per stream (moves_waited_), so no stream handle of an earlier call is used again.
  hipStream_t moves_stream_ = nullptr;
  bool moves_queued_ = false;
  hipEvent_t moves_done_ = nullptr;
  std::vector<hipStream_t> moves_waited_;
  int order_after_moves(hipStream_t stream);
  // The launch arguments decode_layer and bench_attention share for `layer` (plan pointers and
  // work items are set per launch).
  void base_launch(PagedLaunch& pl, int layer, const void* q, const void* k_new, const void* v_new, void* out,
                   bool mass, float scale, float softcap, int window) const;
  // The step's decode launches run on the stream decode_layer was given. Placement
  // (end_step_place, apply_tiers) on another stream reads the mass those launches write and
  // evicts records they append to, so it first waits for them: an event recorded on
  // decode_stream_ when such a call comes. The decode stream therefore has to stay valid
  // until the step's placement has been issued.
  hipStream_t decode_stream_ = nullptr;
  bool decode_pending_ = false;
  hipEvent_t decode_done_ = nullptr;
  std::vector<hipStream_t> decode_waited_;
  int order_after_decode(hipStream_t stream);
  int issue_mirror_copies(hipStream_t stream);
  void forget_streams();  // after a device-wide synchronization
  bool stage_copy_pending_ = false;
  std::vector<hipEvent_t> buf_free_;
  std::vector<hipEvent_t> chunk_ready_;
  // Staging under stream capture. A capture may wait only on events recorded in it: the copy
  // stream joins it through cap_fork_, recorded on the capturing stream before the step's
  // first copy, and a copy waits on buf_free_[b] only where this step recorded it, in the
  // same mode (buf_free_cap_ under capture, buf_free_eager_ otherwise). Work recorded
  // before a replay precedes the whole graph on its stream.
  hipEvent_t cap_fork_ = nullptr;
  bool cap_forked_ = false;
  // Mirror mode: a ring of HBM buffers; layer l's share of the step's host records goes to
  // ring_[l % ring_.size()] by DMA on copy_stream_, and mirror_flags_[l] (device words) is
  // set once it has landed. The merge launch of layer l stores the step's token into
  // mirror_release_[l] (pinned): the attention launch of layer l, the buffer's reader, has
  // finished, so the copies of layer l + ring_.size() may overwrite it.
  std::vector<void*> ring_;
  int64_t ring_records_ = 0;  // records per ring buffer
  uint32_t* mirror_flags_ = nullptr;
  uint32_t* mirror_release_ = nullptr;      // pinned, one word per layer
  uint32_t* mirror_release_dev_ = nullptr;  // its device mapping
  uint32_t step_token_ = 0;                 // token of the open (or last) step
  hipEvent_t mirror_go_ = nullptr;    // on the step's stream, after the flags are cleared
  hipEvent_t mirror_done_ = nullptr;  // on copy_stream_, after the step's copies
  bool mirror_pending_ = false;
  // Issues the mirror copies and word writes of a step while begin_step returns: a layer's
  // copies once the layer n before it has released its buffer (a host-side wait on the
  // release word), so the thread runs beside the step's launches. issue_mirror_copies waits
  // for its previous job before it records or waits on mirror_go_ / mirror_done_ again, and
  // so do sync() and the destructor before they drain the copy stream.
  HostWorker mirror_issuer_;
  // The job gives up waiting for a release (it then queues no further copies of the step;
  // those layers read the host in place after their bounded wait) when the store is being
  // destroyed (mirror_cancel_), or when the step is closed and its decode stream has drained
  // without the release (a layer that was not decoded), or after kReleaseWaitLimit.
  std::atomic<bool> mirror_cancel_{false};
  std::atomic<bool> step_closed_{false};
  std::atomic<bool> closed_has_stream_{false};
  std::atomic<hipStream_t> closed_stream_{nullptr};
  std::atomic<int> mirror_waiting_{0};  // the job is waiting for a release
  // Returns true once mirror_release_[layer] holds `token` (or later), false to give up.
  bool wait_release(int layer, uint32_t token);
  std::mutex copy_timing_mu_;
  std::vector<PendingTiming> copy_timing_;  // mirror copy groups timed by the thread's job
  std::vector<std::pair<int64_t, int64_t>> mirror_spans_;  // (first host record, count) per row
  uint64_t mirror_step_bytes_ = 0;                         // bytes copied per layer this step
  // Deferred block mass (see finish_step_mass).
  float* mass_w_ = nullptr;
  size_t mass_w_floats_ = 0;
  bool mass_deferred_ = false;         // the open step runs with deferred mass
  bool mass_w_dirty_ = false;          // a merge of the open step may have written mass_w_
  float* mass_accum_last_ = nullptr;   // mass_accum of the last decode_layer call
  int64_t mass_stride_last_ = 0;
  size_t mass_layer_floats_ = 0;       // floats of one layer's share of mass_w_ in the open step
  std::vector<char> buf_free_cap_;
  std::vector<char> buf_free_eager_;
  std::vector<int32_t> free_slots_;
  std::vector<std::pair<int64_t, int64_t>> host_free_;  // (offset, count), sorted by offset
  std::vector<Session> sessions_;
  int64_t ram_budget_ = -1;
  int64_t cpu_bytes_ = 0;
  int64_t gpu_bytes_ = 0;
  StoreStats stats_;
  std::vector<PendingTiming> move_timing_;  // for the *_sec stats

  // Current step.
  bool in_step_ = false;
  std::vector<int32_t> step_sids_;
  std::vector<int32_t> step_first_;  // first sequence index of each session in the step
  std::vector<SeqInfo> seqs_;
  std::vector<WorkItem> work_;
  std::vector<int> launch_work_begin_;  // per launch: first work item; launches = chunks or 1
  std::vector<int> launch_work_end_;
  std::vector<CopyCmd> copies_;
  std::vector<std::vector<int64_t>> step_host_ids_;
  int n_chunks_ = 0;
  int n_partials_ = 0;
  int partial_stride_ = 0;  // partial slots per sequence (the most work items of any), or 0: packed
  int mass_stride_ = 0;
  std::vector<int64_t> stage_pairs_;      // staged mode: (host record, staging record) pairs
  std::vector<int64_t> chunk_pair_begin_;  // first pair of each chunk, and the end
  int64_t* d_stage_pairs_ = nullptr;       // the pairs in the uploaded plan
  int64_t* d_chunk_begin_ = nullptr;       // chunk_pair_begin_ in the uploaded plan
  bool prefetch_step_ = false;  // staged mode, one chunk per layer: prefetch the next layer
  int prefetched_layer_ = -1;   // layer whose copies are already queued in its buffer
  // Device views into the workspace for the current step.
  SeqInfo* d_seqs_ = nullptr;
  WorkItem* d_work_ = nullptr;
  int32_t* d_sess_rows_ = nullptr;
  int32_t* d_sess_first_ = nullptr;
  float *d_pm_ = nullptr, *d_pl_ = nullptr, *d_pacc_ = nullptr;  // split-K partials
  float *d_mass_m_ = nullptr, *d_mass_s_ = nullptr, *d_mf_ = nullptr, *d_lf_ = nullptr;
  StepStats step_stats_;

  bool timing_ = false;
  std::vector<PendingTiming> timing_pending_;
  std::vector<hipEvent_t> timing_events_;  // resolved launch-timing events, reused
  hipError_t timing_event(hipEvent_t* ev);
  double timing_ms_ = 0.0;
  int64_t timing_launches_ = 0;
  int64_t timing_bytes_ = 0;
};

}  // namespace pgr
