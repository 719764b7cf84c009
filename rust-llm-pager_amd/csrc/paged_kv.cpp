// Native paged KV store and streaming decode executor (see paged_kv.h for the layout).
//
// Reference behaviour it replaces, per decode step and layer (paged_model.py:878-1086):
// a Python loop gathering every block with a blocking .to(device) + permute + torch.cat,
// then one Triton launch per 64-block group (two passes for attention-scoring policies).
// Here one plan per step covers all layers: resident blocks are read in place from the HBM
// pool; host blocks are read in place from the pinned host mirror by the same kernel over
// the host link (direct mode), or copied by a copy kernel into a staging ring on a side
// stream, with one attention launch per staged chunk and the next layer's copies queued
// under the current layer (staged mode); a merge kernel follows.
#include "paged_kv.h"

#include <algorithm>
#include <chrono>
#include <cstring>

#include "pager_core.h"
#include "pgr_kernels.h"

namespace pgr {

namespace {

// Deferred block mass holds one [S][Hq][stride] share per layer; steps that would need more
// than this many floats reduce the mass per layer instead.
constexpr size_t kMassDeferredMaxFloats = (size_t)16 << 20;
// Longest wait of the mirror thread for one release word before it stops queueing copies for
// the step (the layers after it then read the host in place after their bounded wait).
constexpr std::chrono::seconds kReleaseWaitLimit(10);

// V chunk c (16 bytes) of a record's V region holds dims d0, d0 + 1 of four consecutive tokens
// (v_record_index): tile `tile` of head `h`, tokens 16 tile + 4g .. + 3. Maps c to those.
struct VChunk {
  int h, tok0, d0;
};
__device__ __forceinline__ VChunk v_chunk(int c, int tpb, int d) {
  const int per_head = tpb * d / 8;  // 16-byte chunks of one head's V
  const int h = c / per_head;
  const int rem = c - h * per_head;
  const int tile = rem / (2 * d);
  const int q = 2 * (rem - tile * 2 * d);  // first of the chunk's two four-token groups
  const int dn = d / 16;
  const int j = q % dn, n = (q / dn) % 16, g = q / (16 * dn);
  return VChunk{h, tile * 16 + 4 * g, dn * n + j};
}

// One workgroup per block of records: converts tokens of one (row, layer) from the
// [Hkv, n_src, D] layout into records at dst + slot[i] * rec (zero past n_tokens), or back.
__global__ void hf_to_records_kernel(const uint16_t* k, const uint16_t* v, int64_t n_src, int64_t n_tokens,
                                     const int64_t* dst, uint16_t* pool, uint16_t* host, int hkv, int tpb, int d) {
  // Block i of a [Hkv, n_src, D] tensor pair into its record: dst[i] >= 0 is an HBM pool
  // slot, dst[i] < 0 the host mirror record -dst[i] - 1 (written in place over the host
  // link). 16 bytes per store; tokens past n_tokens are zero. K chunk c is 8 dims of one
  // token row; V chunk c is 2 dims of 4 tokens (the record's transposed V tiles), gathered
  // from four 4-byte loads.
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int64_t b = blockIdx.x;
  const int64_t di = dst[b];
  const size_t rec = (size_t)2 * hkv * tpb * d;
  uint16_t* kr = di >= 0 ? pool + (size_t)di * rec : host + (size_t)(-di - 1) * rec;
  uint16_t* vr = kr + (size_t)hkv * tpb * d;
  const int cpr = d / 8;  // 16-byte chunks per token row
  const int per = hkv * tpb * cpr;
  for (int c = threadIdx.x; c < per; c += blockDim.x) {
    const int h = c / (tpb * cpr);
    const int r = c - h * tpb * cpr;
    const int t = r / cpr, cc = r - t * cpr;
    const int64_t tok = b * tpb + t;
    u32x4 kx = {0u, 0u, 0u, 0u};
    if (tok < n_tokens) kx = *reinterpret_cast<const u32x4*>(k + ((size_t)h * n_src + tok) * d + (size_t)cc * 8);
    *reinterpret_cast<u32x4*>(kr + (size_t)(h * tpb + t) * d + (size_t)cc * 8) = kx;
    const VChunk vc = v_chunk(c, tpb, d);
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t vt = b * tpb + vc.tok0 + i;
      p[i] = vt < n_tokens ? *reinterpret_cast<const uint32_t*>(v + ((size_t)vc.h * n_src + vt) * d + vc.d0) : 0u;
    }
    const u32x4 vx = {(p[0] & 0xffffu) | (p[1] << 16), (p[2] & 0xffffu) | (p[3] << 16),
                      (p[0] >> 16) | (p[1] & 0xffff0000u), (p[2] >> 16) | (p[3] & 0xffff0000u)};
    *reinterpret_cast<u32x4*>(vr + (size_t)c * 8) = vx;
  }
}

__global__ void records_to_hf_kernel(const int64_t* src, const uint16_t* pool, const uint16_t* host,
                                     int64_t n_tokens, uint16_t* k, uint16_t* v, int hkv, int tpb, int d) {
  // Record of block i (src[i] >= 0: pool slot; < 0: host mirror record -src[i] - 1, read in
  // place over the host link) into k, v [Hkv, n_tokens, D]. 16 bytes per load.
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int64_t b = blockIdx.x;
  const int64_t si = src[b];
  const size_t rec = (size_t)2 * hkv * tpb * d;
  const uint16_t* kr = si >= 0 ? pool + (size_t)si * rec : host + (size_t)(-si - 1) * rec;
  const uint16_t* vr = kr + (size_t)hkv * tpb * d;
  const int cpr = d / 8;
  const int per = hkv * tpb * cpr;
  for (int c = threadIdx.x; c < per; c += blockDim.x) {
    const int h = c / (tpb * cpr);
    const int r = c - h * tpb * cpr;
    const int t = r / cpr, cc = r - t * cpr;
    const int64_t tok = b * tpb + t;
    const u32x4 kx = *reinterpret_cast<const u32x4*>(kr + (size_t)(h * tpb + t) * d + (size_t)cc * 8);
    if (tok < n_tokens) *reinterpret_cast<u32x4*>(k + ((size_t)h * n_tokens + tok) * d + (size_t)cc * 8) = kx;
    const VChunk vc = v_chunk(c, tpb, d);
    const u32x4 w = *reinterpret_cast<const u32x4*>(vr + (size_t)c * 8);
    const uint32_t p[4] = {(w.x & 0xffffu) | (w.z << 16), (w.x >> 16) | (w.z & 0xffff0000u),
                           (w.y & 0xffffu) | (w.w << 16), (w.y >> 16) | (w.w & 0xffff0000u)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t vt = b * tpb + vc.tok0 + i;
      if (vt < n_tokens) *reinterpret_cast<uint32_t*>(v + ((size_t)vc.h * n_tokens + vt) * d + vc.d0) = p[i];
    }
  }
}

// Copies whole records for every layer: workgroup (i, layer) copies record pairs[2i] of
// bases[src_tbl + layer] to record pairs[2i + 1] of bases[dst_tbl + layer], 16 bytes per
// load and store. A base is a layer's HBM pool or the device address of its pinned host
// mirror, so one launch serves evictions, loads and row copies.
__global__ void copy_records_kernel(void* const* bases, int src_tbl, int dst_tbl, const int64_t* pairs,
                                    int64_t rec_vec) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int layer = blockIdx.y;
  const u32x4* src = static_cast<const u32x4*>(bases[src_tbl + layer]) + (size_t)pairs[2 * blockIdx.x] * rec_vec;
  u32x4* dst = static_cast<u32x4*>(bases[dst_tbl + layer]) + (size_t)pairs[2 * blockIdx.x + 1] * rec_vec;
  for (int64_t i = threadIdx.x; i < rec_vec; i += blockDim.x) dst[i] = src[i];
}

// Staged mode: records of one layer's host mirror (read in place through its device mapping)
// into a staging buffer, by (host record, staging record) pairs: those of one chunk,
// [chunk_begin[0], chunk_begin[1]), read from the uploaded plan so that the launch is the
// same from step to step (a captured graph replays it). A fixed grid of a few dozen
// workgroups keeps the host link busy while leaving the CUs to concurrent work.
constexpr int kStageCopyWorkgroups = 96;
__global__ void stage_copy_kernel(const void* host, void* stage, const int64_t* pairs, const int64_t* chunk_begin,
                                  int64_t rec_vec) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int64_t end = chunk_begin[1];
  for (int64_t p = chunk_begin[0] + blockIdx.x; p < end; p += gridDim.x) {
    const u32x4* src = static_cast<const u32x4*>(host) + (size_t)pairs[2 * p] * rec_vec;
    u32x4* dst = static_cast<u32x4*>(stage) + (size_t)pairs[2 * p + 1] * rec_vec;
    for (int64_t i = threadIdx.x; i < rec_vec; i += blockDim.x) dst[i] = src[i];
  }
}

// Mirror mode: resets the per-layer "mirror filled" words on the step's stream: 0 when the
// step's copies follow, 1 when there is nothing to copy (no launch then waits).
__global__ void mirror_flags_reset_kernel(uint32_t* flags, int n, uint32_t value) {
  if ((int)threadIdx.x < n) flags[threadIdx.x] = value;
}

// Staged mode: the step plan, copied from the pinned plan buffer (read in place through its
// device mapping) into the workspace; in direct mode the step's first attention launch does
// this copy itself. A copy kernel on the compute stream, rather than an SDMA copy, keeps the
// upload on the queue that runs the attention: each hand-off between the copy engine and the
// compute queue cost about 9 and 26 us per step.
__global__ void plan_upload_kernel(const void* src, void* dst, int64_t n_vec) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_vec) static_cast<u32x4*>(dst)[i] = static_cast<const u32x4*>(src)[i];
}

}  // namespace

void HostWorker::submit(std::function<hipError_t()> job) {
  std::unique_lock<std::mutex> lk(mu_);
  if (!thread_.joinable()) {
    try {
      thread_ = std::thread([this] { run(); });
    } catch (const std::system_error&) {  // no thread to be had: the job runs here
      lk.unlock();
      const hipError_t r = job();
      lk.lock();
      result_ = r;
      return;
    }
  }
  job_ = std::move(job);
  pending_ = true;
  lk.unlock();
  cv_.notify_all();
}

hipError_t HostWorker::wait() {
  std::unique_lock<std::mutex> lk(mu_);
  cv_.wait(lk, [this] { return !pending_; });
  const hipError_t r = result_;
  result_ = hipSuccess;
  return r;
}

bool HostWorker::busy() {
  std::lock_guard<std::mutex> lk(mu_);
  return pending_;
}

void HostWorker::stop() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  cv_.notify_all();
  if (thread_.joinable()) thread_.join();
}

void HostWorker::run() {
  std::unique_lock<std::mutex> lk(mu_);
  for (;;) {
    cv_.wait(lk, [this] { return pending_ || stop_; });
    if (!pending_) return;  // stopped, nothing left to run
    std::function<hipError_t()> job = std::move(job_);
    lk.unlock();
    const hipError_t r = job();
    lk.lock();
    result_ = r;
    pending_ = false;
    cv_.notify_all();
  }
}

PagedKV::PagedKV(const PagedKVConfig& cfg) : cfg_(cfg) {}

PagedKV::~PagedKV() {
  // The mirror thread's copies are drained before the thread ends. Ended first, the thread
  // left its last DMA copies in flight: an async-copy tracer (rocprofv3 --memory-copy-trace)
  // then never delivered their completions (it retired the thread's correlation ids as
  // dangling at exit) and its exit-time teardown crashed in __cxa_finalize. So: stop a job
  // still waiting for a release, wait for it, have the thread itself wait for its copies,
  // then end it.
  mirror_cancel_ = true;
  mirror_issuer_.wait();
  if (mirror_issuer_.started() && copy_stream_) {
    hipStream_t cs = copy_stream_;
    mirror_issuer_.submit([cs]() { return hipStreamSynchronize(cs); });
    mirror_issuer_.wait();
  }
  if (copy_stream_) hipStreamSynchronize(copy_stream_);
  hipDeviceSynchronize();
  mirror_issuer_.stop();
  for (void* p : pool_)
    if (p) hipFree(p);
  for (void* p : host_)
    if (p) hipHostFree(p);
  if (stage_) hipFree(stage_);
  if (ws_) hipFree(ws_);
  if (bases_dev_) hipFree(bases_dev_);
  for (IndexBuf& b : index_bufs_) {
    if (b.host) hipHostFree(b.host);
    if (b.done) hipEventDestroy(b.done);
  }
  for (PlanBuf& b : plan_bufs_) {
    if (b.host) hipHostFree(b.host);
    if (b.read) hipEventDestroy(b.read);
  }
  if (plan_flags_) hipHostFree(plan_flags_);
  if (mass_host_) hipHostFree(mass_host_);
  for (hipEvent_t e : buf_free_) hipEventDestroy(e);
  for (hipEvent_t e : chunk_ready_) hipEventDestroy(e);
  for (auto& t : timing_pending_) {
    hipEventDestroy(t.start);
    hipEventDestroy(t.stop);
  }
  for (hipEvent_t e : timing_events_) hipEventDestroy(e);
  for (auto& t : move_timing_) {
    hipEventDestroy(t.start);
    hipEventDestroy(t.stop);
  }
  for (auto& t : copy_timing_) {
    hipEventDestroy(t.start);
    hipEventDestroy(t.stop);
  }
  if (plan_uploaded_) hipEventDestroy(plan_uploaded_);
  if (cap_fork_) hipEventDestroy(cap_fork_);
  if (mirror_go_) hipEventDestroy(mirror_go_);
  if (mirror_done_) hipEventDestroy(mirror_done_);
  for (void* p : ring_)
    if (p) hipFree(p);
  if (mirror_flags_) hipFree(mirror_flags_);
  if (mirror_release_) hipHostFree(mirror_release_);
  if (mass_w_) hipFree(mass_w_);
  if (stage_copies_done_) hipEventDestroy(stage_copies_done_);
  if (moves_done_) hipEventDestroy(moves_done_);
  if (decode_done_) hipEventDestroy(decode_done_);
  if (copy_stream_) hipStreamDestroy(copy_stream_);
}

int PagedKV::fail(int code, const std::string& msg) {
  err_ = msg;
  return code;
}

int PagedKV::hip_fail(hipError_t e, const char* what) {
  err_ = std::string(what) + ": " + hipGetErrorString(e);
  return kErrHip;
}

#define PGR_HIP(call)                                   \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return hip_fail(e_, #call);   \
  } while (0)

// Waits until the merge launch after the buffer's last read has stored the buffer's token
// into its pinned flag word. Polls the word without HIP calls: with a stream query every
// ~25 us in the loop, the next launch on the stream started ~6 us late (by kernel trace),
// as after a recorded event. Only after 2^22 polls (longer than a step) does it query the
// stream, every 2^16 polls after that, to return an error from a failed stream instead of
// spinning.
int PagedKV::wait_plan_flag(const PlanBuf& pb, int idx) {
  auto done = [&] { return (int32_t)(__atomic_load_n(plan_flags_ + idx, __ATOMIC_ACQUIRE) - pb.token) >= 0; };
  for (uint64_t poll = 1; !done(); ++poll) {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
    if (poll < (1u << 22) || (poll & 0xffff) != 0) continue;
    const hipError_t e = hipStreamQuery(pb.stream);
    if (e == hipErrorNotReady) continue;
    if (e != hipSuccess) return hip_fail(e, "hipStreamQuery (plan buffer wait)");
    if (done()) break;
    return fail(kErrState, "plan buffer still marked as read after its stream drained");
  }
  return kOk;
}

// Tier moves run on the stream apply_tiers was given, which records moves_done_ after them.
// Work queued on another stream that reads or reuses records (kernels, copies, slot reuse)
// waits for that event, once per stream; work on the same stream is ordered already.
int PagedKV::order_after_moves(hipStream_t stream) {
  if (!moves_queued_ || moves_stream_ == stream) return kOk;
  if (std::find(moves_waited_.begin(), moves_waited_.end(), stream) != moves_waited_.end()) return kOk;
  PGR_HIP(hipStreamWaitEvent(stream, moves_done_, 0));
  moves_waited_.push_back(stream);
  return kOk;
}

// Placement on a stream other than the step's decode stream waits for the decode launches
// (their appends and block mass) before it reads the mass or copies records. The event is
// recorded on the decode stream when the first such call comes, so a step whose placement
// runs on its own stream pays nothing.
int PagedKV::order_after_decode(hipStream_t stream) {
  if (!decode_pending_ || decode_stream_ == stream) return kOk;
  if (std::find(decode_waited_.begin(), decode_waited_.end(), stream) != decode_waited_.end()) return kOk;
  if (decode_waited_.empty()) PGR_HIP(hipEventRecord(decode_done_, decode_stream_));
  PGR_HIP(hipStreamWaitEvent(stream, decode_done_, 0));
  decode_waited_.push_back(stream);
  return kOk;
}

void PagedKV::forget_streams() {
  moves_queued_ = false;
  moves_waited_.clear();
  decode_pending_ = false;
  decode_waited_.clear();
}

size_t PagedKV::rec_bytes() const {
  return (size_t)2 * cfg_.kv_heads * cfg_.tokens_per_block * cfg_.head_dim * 2;
}

int PagedKV::init() {
  if (cfg_.num_layers <= 0 || cfg_.kv_heads <= 0 || cfg_.tokens_per_block <= 0 || cfg_.tokens_per_block % 16 != 0)
    return fail(kErrInvalid, "num_layers, kv_heads > 0 and tokens_per_block a positive multiple of 16 required");
  if (!paged_head_dim_supported(cfg_.head_dim))
    return fail(kErrUnsupported, "head_dim must be 16, 32, 64, 128 or 256");
  if (cfg_.query_heads <= 0 || cfg_.query_heads % cfg_.kv_heads != 0)
    return fail(kErrInvalid, "query_heads must be a positive multiple of kv_heads");
  if (cfg_.query_heads / cfg_.kv_heads > kMaxRep) return fail(kErrUnsupported, "n_rep above 16 is not supported");
  if (cfg_.dtype != kF16 && cfg_.dtype != kBF16) return fail(kErrInvalid, "dtype must be fp16 or bf16");
  if (cfg_.pool_slots <= 0 || cfg_.host_records < 0 || cfg_.staging_slots <= 0 || cfg_.staging_buffers < 1)
    return fail(kErrInvalid, "pool_slots, staging_slots > 0 and staging_buffers >= 1 required");
  if (cfg_.stream_mode < 0 || cfg_.stream_mode > 2) return fail(kErrInvalid, "stream_mode must be 0, 1 or 2");
  if (cfg_.stream_mode == 2 && cfg_.num_layers > 256) return fail(kErrInvalid, "mirror mode takes at most 256 layers");
  if (cfg_.host_records > INT32_MAX / 2) return fail(kErrInvalid, "host_records too large for 32-bit record indices");
  if (cfg_.pool_slots > INT32_MAX / 2 || cfg_.staging_slots * cfg_.staging_buffers > INT32_MAX / 2)
    return fail(kErrInvalid, "pool or staging too large for 32-bit record indices");
  if (cfg_.blocks_per_workgroup < kWaves) cfg_.blocks_per_workgroup = kWaves;
  int dev = 0;
  PGR_HIP(hipGetDevice(&dev));
  device_ = dev;
  PGR_HIP(hipDeviceGetAttribute(&n_cu_, hipDeviceAttributeMultiprocessorCount, dev));
  const size_t rec = rec_bytes();
  pool_.assign(cfg_.num_layers, nullptr);
  host_.assign(cfg_.num_layers, nullptr);
  host_dev_.assign(cfg_.num_layers, nullptr);
  for (int l = 0; l < cfg_.num_layers; ++l) {
    PGR_HIP(hipMalloc(&pool_[l], rec * (size_t)cfg_.pool_slots));
    if (cfg_.host_records > 0) {
      PGR_HIP(hipHostMalloc(&host_[l], rec * (size_t)cfg_.host_records, hipHostMallocDefault));
      PGR_HIP(hipHostGetDevicePointer(&host_dev_[l], host_[l], 0));
    }
  }
  // The staging ring exists for the staged stream mode only: in the direct mode the kernels
  // and the copy kernels read and write the host mirror in place.
  if (cfg_.stream_mode == 1) PGR_HIP(hipMalloc(&stage_, rec * (size_t)cfg_.staging_slots * cfg_.staging_buffers));
  if (cfg_.stream_mode == 2) {
    // The ring: one buffer per layer up to staging_buffers, each grown by begin_step to the
    // step's host share of a layer.
    ring_.assign(std::min(cfg_.staging_buffers, cfg_.num_layers), nullptr);
    ring_records_ = cfg_.staging_slots;
    for (void*& b : ring_) PGR_HIP(hipMalloc(&b, rec * (size_t)ring_records_));
    PGR_HIP(hipMalloc(reinterpret_cast<void**>(&mirror_flags_), 256 * sizeof(uint32_t)));
    PGR_HIP(hipMemset(mirror_flags_, 0, 256 * sizeof(uint32_t)));
    PGR_HIP(hipHostMalloc(reinterpret_cast<void**>(&mirror_release_), 256 * sizeof(uint32_t), hipHostMallocDefault));
    std::memset(mirror_release_, 0, 256 * sizeof(uint32_t));
    PGR_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&mirror_release_dev_), mirror_release_, 0));
  }
  PGR_HIP(hipStreamCreateWithFlags(&copy_stream_, hipStreamNonBlocking));
  buf_free_.resize(cfg_.staging_buffers);
  chunk_ready_.resize(cfg_.staging_buffers);
  buf_free_cap_.assign(cfg_.staging_buffers, 0);
  buf_free_eager_.assign(cfg_.staging_buffers, 0);
  // Ordering events. They order GPU work against GPU work, or tell the host that the GPU has
  // finished reading a pinned buffer; none guards device writes that the host then reads
  // (the mass read-back synchronizes its stream). So none needs the system-scope release
  // at record time, which writes back the caches: on the event between a plan upload and
  // the attention launch that cost about 2 us per step.
  const unsigned ev_flags = hipEventDisableTiming | hipEventDisableSystemFence;
  for (int i = 0; i < cfg_.staging_buffers; ++i) {
    PGR_HIP(hipEventCreateWithFlags(&buf_free_[i], ev_flags));
    PGR_HIP(hipEventCreateWithFlags(&chunk_ready_[i], ev_flags));
  }
  PGR_HIP(hipEventCreateWithFlags(&plan_uploaded_, ev_flags));
  PGR_HIP(hipEventCreateWithFlags(&cap_fork_, ev_flags));
  PGR_HIP(hipEventCreateWithFlags(&mirror_go_, ev_flags));
  PGR_HIP(hipEventCreateWithFlags(&mirror_done_, ev_flags));
  for (PlanBuf& b : plan_bufs_) PGR_HIP(hipEventCreateWithFlags(&b.read, ev_flags));
  PGR_HIP(hipHostMalloc(reinterpret_cast<void**>(&plan_flags_), 256, hipHostMallocDefault));
  std::memset(plan_flags_, 0, 256);
  PGR_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&plan_flags_dev_), plan_flags_, 0));
  PGR_HIP(hipEventCreateWithFlags(&stage_copies_done_, ev_flags));
  PGR_HIP(hipEventCreateWithFlags(&moves_done_, ev_flags));
  PGR_HIP(hipEventCreateWithFlags(&decode_done_, ev_flags));
  for (IndexBuf& b : index_bufs_) PGR_HIP(hipEventCreateWithFlags(&b.done, ev_flags));
  {
    std::vector<void*> bases(pool_);
    bases.insert(bases.end(), host_dev_.begin(), host_dev_.end());
    PGR_HIP(hipMalloc(&bases_dev_, sizeof(void*) * bases.size()));
    PGR_HIP(hipMemcpy(bases_dev_, bases.data(), sizeof(void*) * bases.size(), hipMemcpyHostToDevice));
  }
  free_slots_.resize(cfg_.pool_slots);
  for (int64_t i = 0; i < cfg_.pool_slots; ++i) free_slots_[i] = (int32_t)(cfg_.pool_slots - 1 - i);
  host_free_.clear();
  if (cfg_.host_records > 0) host_free_.push_back({0, cfg_.host_records});
  return kOk;
}

int PagedKV::alloc_slot() {
  if (free_slots_.empty()) return -1;
  const int s = free_slots_.back();
  free_slots_.pop_back();
  return s;
}

void PagedKV::free_slot(int32_t s) { free_slots_.push_back(s); }

int64_t PagedKV::host_alloc(int64_t n) {
  for (size_t i = 0; i < host_free_.size(); ++i) {
    if (host_free_[i].second >= n) {
      const int64_t off = host_free_[i].first;
      host_free_[i].first += n;
      host_free_[i].second -= n;
      if (host_free_[i].second == 0) host_free_.erase(host_free_.begin() + i);
      return off;
    }
  }
  return -1;
}

void PagedKV::host_free(int64_t off, int64_t n) {
  if (n <= 0) return;
  auto it = std::lower_bound(host_free_.begin(), host_free_.end(), std::make_pair(off, (int64_t)0));
  it = host_free_.insert(it, {off, n});
  // Coalesce with neighbours.
  size_t i = it - host_free_.begin();
  if (i + 1 < host_free_.size() && host_free_[i].first + host_free_[i].second == host_free_[i + 1].first) {
    host_free_[i].second += host_free_[i + 1].second;
    host_free_.erase(host_free_.begin() + i + 1);
  }
  if (i > 0 && host_free_[i - 1].first + host_free_[i - 1].second == host_free_[i].first) {
    host_free_[i - 1].second += host_free_[i].second;
    host_free_.erase(host_free_.begin() + i);
  }
}

int PagedKV::add_session(int rows, int64_t capacity_tokens, const int32_t* lo_per_row) {
  if (rows <= 0 || capacity_tokens <= 0) return fail(kErrInvalid, "rows and capacity_tokens must be positive");
  const int64_t T = cfg_.tokens_per_block;
  Session s;
  s.live = true;
  s.rows = rows;
  s.capacity_blocks = (capacity_tokens + T - 1) / T + 1;
  s.row.resize(rows);
  for (int r = 0; r < rows; ++r) {
    const int64_t off = host_alloc(s.capacity_blocks);
    if (off < 0) {
      for (int q = 0; q < r; ++q) host_free(s.row[q].host_off, s.capacity_blocks);
      return fail(kErrCapacity, "host mirror has no room for this session's capacity");
    }
    s.row[r].host_off = off;
    s.row[r].lo = lo_per_row ? lo_per_row[r] : 0;
  }
  s.slot.assign((size_t)s.capacity_blocks * rows, -1);
  s.host_valid.assign((size_t)s.capacity_blocks * rows, 0);
  s.on_gpu.assign(s.capacity_blocks, 0);
  s.placed.assign(s.capacity_blocks, 0);
  for (size_t i = 0; i < sessions_.size(); ++i)
    if (!sessions_[i].live) {
      sessions_[i] = std::move(s);
      return (int)i;
    }
  sessions_.push_back(std::move(s));
  return (int)sessions_.size() - 1;
}

int PagedKV::remove_session(int sid) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  if (in_step_) return fail(kErrState, "remove_session during a decode step");
  Session& s = sessions_[sid];
  // Slots may still be read by queued kernels or copies: drain before recycling them.
  PGR_HIP(hipDeviceSynchronize());
  forget_streams();
  const int64_t T = cfg_.tokens_per_block;
  const int64_t n_full = s.n_tokens / T;
  for (int64_t b = 0; b < s.capacity_blocks; ++b)
    for (int r = 0; r < s.rows; ++r) {
      const int32_t sl = s.slot[b * s.rows + r];
      if (sl >= 0) free_slot(sl);
    }
  const int64_t bb = block_bytes_all_layers(sid);
  for (int64_t b = 0; b < n_full; ++b) {
    if (s.on_gpu[b])
      gpu_bytes_ -= bb;
    else if (s.placed[b])
      cpu_bytes_ -= bb;
  }
  for (int r = 0; r < s.rows; ++r) host_free(s.row[r].host_off, s.capacity_blocks);
  s = Session();
  return kOk;
}

int PagedKV::set_lo(int sid, const int32_t* lo_per_row) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  Session& s = sessions_[sid];
  for (int r = 0; r < s.rows; ++r) s.row[r].lo = lo_per_row[r];
  return kOk;
}

int PagedKV::acquire_index_buf(size_t n, IndexBuf** out) {
  IndexBuf& b = index_bufs_[next_index_buf_];
  next_index_buf_ = (next_index_buf_ + 1) % kIndexBufs;
  if (b.pending) {
    PGR_HIP(hipEventSynchronize(b.done));
    b.pending = false;
  }
  if (n > b.cap) {
    if (b.host) PGR_HIP(hipHostFree(b.host));
    b.host = nullptr;
    b.dev = nullptr;
    b.cap = 0;
    const size_t want = std::max<size_t>(n, 4096);
    PGR_HIP(hipHostMalloc(reinterpret_cast<void**>(&b.host), want * sizeof(int64_t), hipHostMallocDefault));
    PGR_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&b.dev), b.host, 0));
    b.cap = want;
  }
  *out = &b;
  return kOk;
}

int PagedKV::launch_copies(std::vector<int64_t>& pairs, int src_tbl, int dst_tbl, hipStream_t stream) {
  if (pairs.empty()) return kOk;
  IndexBuf* ib = nullptr;
  int rc = acquire_index_buf(pairs.size(), &ib);
  if (rc != kOk) return rc;
  std::memcpy(ib->host, pairs.data(), pairs.size() * sizeof(int64_t));
  const dim3 grid((unsigned)(pairs.size() / 2), (unsigned)cfg_.num_layers);
  copy_records_kernel<<<grid, 256, 0, stream>>>(bases_dev_, src_tbl, dst_tbl, ib->dev, (int64_t)(rec_bytes() / 16));
  PGR_HIP(hipGetLastError());
  PGR_HIP(hipEventRecord(ib->done, stream));
  ib->pending = true;
  pairs.clear();
  return kOk;
}

int PagedKV::reorder_rows(int sid, const int32_t* src, int n, hipStream_t stream) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  if (in_step_) return fail(kErrState, "reorder_rows during a decode step");
  Session& s = sessions_[sid];
  const int rows = s.rows;
  if (n != rows) return fail(kErrInvalid, "reorder_rows takes one source row per row of the session");
  for (int r = 0; r < rows; ++r)
    if (src[r] < 0 || src[r] >= rows) return fail(kErrInvalid, "source row out of range");
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  // The first new row that takes an old row inherits its records (HBM slots and host
  // range). Every later taker reuses the records of an old row that no new row takes --
  // there are exactly as many of those, and every row of a session holds records for the
  // same blocks -- and gets a copy of its source's data there. So nothing is allocated and
  // copies only ever read inherited records and write dropped ones.
  std::vector<int> heir(rows, -1);
  for (int r = 0; r < rows; ++r)
    if (heir[src[r]] < 0) heir[src[r]] = r;
  std::vector<int> dropped;
  for (int o = 0; o < rows; ++o)
    if (heir[o] < 0) dropped.push_back(o);
  std::vector<int> holder(rows);  // old row whose records new row r takes over
  size_t next_dropped = 0;
  for (int r = 0; r < rows; ++r) holder[r] = heir[src[r]] == r ? src[r] : dropped[next_dropped++];
  const int64_t nb = s.capacity_blocks;
  for (int64_t b = 0; b < nb; ++b)
    for (int r = 1; r < rows; ++r)
      if ((s.slot[b * rows + r] < 0) != (s.slot[b * rows] < 0))
        return fail(kErrState, "rows of a session differ in residency");
  // Queued kernels and copies may still read or write this session's records.
  PGR_HIP(hipDeviceSynchronize());
  forget_streams();
  std::vector<int32_t> slot(s.slot.size(), -1);
  std::vector<uint8_t> hv(s.host_valid.size(), 0);
  std::vector<int64_t> pairs, host_pairs;  // (from record, to record) in the pool / host mirror
  for (int r = 0; r < rows; ++r) {
    const int o = src[r], h = holder[r];
    for (int64_t b = 0; b < nb; ++b) {
      const int32_t from = s.slot[b * rows + o], to = s.slot[b * rows + h];
      slot[b * rows + r] = to;
      if (from >= 0 && h != o) {
        pairs.push_back(from);
        pairs.push_back(to);
      }
      const uint8_t v = s.host_valid[b * rows + o];
      hv[b * rows + r] = v;
      if (v && h != o) {
        host_pairs.push_back(s.row[o].host_off + b);
        host_pairs.push_back(s.row[h].host_off + b);
      }
    }
  }
  if (!pairs.empty() || !host_pairs.empty()) {
    int rc = launch_copies(pairs, 0, 0, stream);
    if (rc == kOk) rc = launch_copies(host_pairs, cfg_.num_layers, cfg_.num_layers, stream);
    if (rc != kOk) return rc;
    PGR_HIP(hipStreamSynchronize(stream));
  }
  std::vector<Row> row(rows);
  for (int r = 0; r < rows; ++r) {
    row[r].host_off = s.row[holder[r]].host_off;
    row[r].lo = s.row[src[r]].lo;
  }
  s.row = std::move(row);
  s.slot = std::move(slot);
  s.host_valid = std::move(hv);
  return kOk;
}

int64_t PagedKV::block_bytes_all_layers(int sid) const {
  const Session& s = sessions_[sid];
  return (int64_t)rec_bytes() * s.rows * cfg_.num_layers;
}

int PagedKV::set_length(int sid, int64_t n_tokens) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  if (in_step_) return fail(kErrState, "set_length during a decode step");
  Session& s = sessions_[sid];
  const int64_t T = cfg_.tokens_per_block;
  if (s.n_tokens != 0) return fail(kErrState, "set_length only applies to an empty session");
  if (n_tokens < 0 || (n_tokens + T - 1) / T >= s.capacity_blocks)
    return fail(kErrCapacity, "n_tokens exceeds the session capacity");
  const int64_t n_full = n_tokens / T;
  // Full blocks start on the host side with no data and uncharged: their first apply_tiers
  // places them, charging HBM or the RAM budget. The open block, if any, gets its HBM slot now.
  for (int64_t b = 0; b < n_full; ++b) {
    s.on_gpu[b] = 0;
    s.placed[b] = 0;
  }
  if (n_tokens % T != 0) {
    for (int r = 0; r < s.rows; ++r) {
      const int sl = alloc_slot();
      if (sl < 0) return fail(kErrCapacity, "HBM pool exhausted");
      s.slot[n_full * s.rows + r] = sl;
    }
  }
  s.n_tokens = n_tokens;
  return kOk;
}

int PagedKV::import_tokens(int sid, int row, int layer, const void* k, const void* v, int64_t n_src, int64_t n_tokens,
                           hipStream_t stream) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  Session& s = sessions_[sid];
  if (row < 0 || row >= s.rows || layer < 0 || layer >= cfg_.num_layers) return fail(kErrInvalid, "row/layer out of range");
  if (n_tokens != s.n_tokens || n_src < n_tokens) return fail(kErrInvalid, "n_tokens must equal the session length");
  if (in_step_) return fail(kErrState, "import during a decode step");
  if (((uintptr_t)k | (uintptr_t)v) % 16 != 0) return fail(kErrInvalid, "k and v must be 16-byte aligned");
  const int64_t T = cfg_.tokens_per_block;
  const int64_t nb = (n_tokens + T - 1) / T;
  if (nb == 0) return kOk;
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  // One launch: resident blocks into their pool slots, host blocks straight into the
  // pinned mirror through its device mapping.
  IndexBuf* ib = nullptr;
  int rc = acquire_index_buf((size_t)nb, &ib);
  if (rc != kOk) return rc;
  for (int64_t b = 0; b < nb; ++b) {
    const int32_t sl = s.slot[b * s.rows + row];
    ib->host[b] = sl >= 0 ? (int64_t)sl : -(s.row[row].host_off + b) - 1;
  }
  hf_to_records_kernel<<<(unsigned)nb, 256, 0, stream>>>(
      static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), n_src, n_tokens, ib->dev,
      static_cast<uint16_t*>(pool_[layer]), static_cast<uint16_t*>(host_dev_[layer]), cfg_.kv_heads, (int)T,
      cfg_.head_dim);
  PGR_HIP(hipGetLastError());
  PGR_HIP(hipEventRecord(ib->done, stream));
  ib->pending = true;
  for (int64_t b = 0; b < nb; ++b)
    if (s.slot[b * s.rows + row] < 0) s.host_valid[b * s.rows + row] = 1;
  return kOk;
}

int PagedKV::export_tokens(int sid, int row, int layer, void* k, void* v, int64_t n_tokens, hipStream_t stream) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  Session& s = sessions_[sid];
  if (row < 0 || row >= s.rows || layer < 0 || layer >= cfg_.num_layers) return fail(kErrInvalid, "row/layer out of range");
  if (n_tokens > s.n_tokens) return fail(kErrInvalid, "n_tokens exceeds the session length");
  if (in_step_) return fail(kErrState, "export during a decode step");
  if (((uintptr_t)k | (uintptr_t)v) % 16 != 0) return fail(kErrInvalid, "k and v must be 16-byte aligned");
  const int64_t T = cfg_.tokens_per_block;
  const int64_t nb = (n_tokens + T - 1) / T;
  if (nb == 0) return kOk;
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  IndexBuf* ib = nullptr;
  int rc = acquire_index_buf((size_t)nb, &ib);
  if (rc != kOk) return rc;
  for (int64_t b = 0; b < nb; ++b) {
    const int32_t sl = s.slot[b * s.rows + row];
    ib->host[b] = sl >= 0 ? (int64_t)sl : -(s.row[row].host_off + b) - 1;
  }
  records_to_hf_kernel<<<(unsigned)nb, 256, 0, stream>>>(
      ib->dev, static_cast<const uint16_t*>(pool_[layer]), static_cast<const uint16_t*>(host_dev_[layer]), n_tokens,
      static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), cfg_.kv_heads, (int)T, cfg_.head_dim);
  PGR_HIP(hipGetLastError());
  PGR_HIP(hipEventRecord(ib->done, stream));
  ib->pending = true;
  PGR_HIP(hipStreamSynchronize(stream));
  return kOk;
}

int PagedKV::put_block(int sid, int64_t block_id, const void* key, const void* value, hipStream_t stream) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  if (in_step_) return fail(kErrState, "put_block during a decode step");
  Session& s = sessions_[sid];
  const int64_t T = cfg_.tokens_per_block;
  if (s.n_tokens % T != 0) return fail(kErrState, "put_block needs a block-aligned session (no open block)");
  if (block_id != s.n_tokens / T) return fail(kErrInvalid, "put_block: block ids must be registered in order");
  if (block_id + 1 >= s.capacity_blocks) return fail(kErrCapacity, "session capacity reached");
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  std::vector<int32_t> slots(s.rows);
  for (int r = 0; r < s.rows; ++r) {
    const int sl = alloc_slot();
    if (sl < 0) {
      for (int q = 0; q < r; ++q) free_slot(slots[q]);
      return fail(kErrCapacity, "HBM pool exhausted");
    }
    slots[r] = sl;
  }
  int32_t* d_slots = nullptr;
  PGR_HIP(hipMalloc(&d_slots, sizeof(int32_t) * s.rows));
  hipError_t e = hipMemcpyAsync(d_slots, slots.data(), sizeof(int32_t) * s.rows, hipMemcpyHostToDevice, stream);
  const size_t layer_elems = (size_t)s.rows * T * cfg_.kv_heads * cfg_.head_dim;
  for (int l = 0; l < cfg_.num_layers && e == hipSuccess; ++l)
    e = launch_ref_to_records(static_cast<const uint16_t*>(key) + l * layer_elems,
                              static_cast<const uint16_t*>(value) + l * layer_elems, pool_[l], d_slots, s.rows,
                              cfg_.kv_heads, (int)T, cfg_.head_dim, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  hipFree(d_slots);
  if (e != hipSuccess) {
    for (int r = 0; r < s.rows; ++r) free_slot(slots[r]);
    return hip_fail(e, "put_block");
  }
  for (int r = 0; r < s.rows; ++r) {
    s.slot[block_id * s.rows + r] = slots[r];
    s.host_valid[block_id * s.rows + r] = 0;
  }
  s.on_gpu[block_id] = 1;
  s.placed[block_id] = 1;
  s.n_tokens += T;
  gpu_bytes_ += block_bytes_all_layers(sid);
  return kOk;
}

int PagedKV::get_block(int sid, int64_t block_id, void* key, void* value, hipStream_t stream) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  if (in_step_) return fail(kErrState, "get_block during a decode step");
  Session& s = sessions_[sid];
  const int64_t T = cfg_.tokens_per_block;
  if (block_id < 0 || block_id >= s.n_tokens / T) return fail(kErrKey, "block is not a registered full block");
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  const bool on_gpu = s.slot[block_id * s.rows] >= 0;  // where the bytes are
  // Record index per row: pool slots, or host mirror records read in place.
  IndexBuf* ib = nullptr;
  int rc = acquire_index_buf((size_t)s.rows, &ib);
  if (rc != kOk) return rc;
  int32_t* slots = reinterpret_cast<int32_t*>(ib->host);
  for (int r = 0; r < s.rows; ++r)
    slots[r] = on_gpu ? s.slot[block_id * s.rows + r] : (int32_t)(s.row[r].host_off + block_id);
  const int32_t* d_slots = reinterpret_cast<const int32_t*>(ib->dev);
  hipError_t e = hipSuccess;
  const size_t layer_elems = (size_t)s.rows * T * cfg_.kv_heads * cfg_.head_dim;
  for (int l = 0; l < cfg_.num_layers && e == hipSuccess; ++l)
    e = launch_records_to_ref(on_gpu ? pool_[l] : host_dev_[l], d_slots, static_cast<uint16_t*>(key) + l * layer_elems,
                              static_cast<uint16_t*>(value) + l * layer_elems, s.rows, cfg_.kv_heads, (int)T,
                              cfg_.head_dim, stream);
  if (e == hipSuccess) e = hipEventRecord(ib->done, stream);
  ib->pending = true;
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "get_block");
  return kOk;
}

double PagedKV::ram_usage_ratio() const {
  if (ram_budget_ <= 0) return 0.0;
  return (double)cpu_bytes_ / (double)ram_budget_;
}

int PagedKV::load_block(Session& s, int64_t b) {
  const size_t rec = rec_bytes();
  for (int r = 0; r < s.rows; ++r) {
    const size_t k = (size_t)b * s.rows + r;
    if (s.slot[k] >= 0) continue;
    const int sl = alloc_slot();
    if (sl < 0) {
      for (int q = 0; q < r; ++q) {  // leave the block wholly on the host side
        const size_t kq = (size_t)b * s.rows + q;
        free_slot(s.slot[kq]);
        s.slot[kq] = -1;
        if (s.host_valid[kq]) {
          load_pairs_.resize(load_pairs_.size() - 2);
          stats_.load_bytes_copied -= rec * cfg_.num_layers;
        }
      }
      return fail(kErrCapacity, "HBM pool exhausted while loading a block");
    }
    s.slot[k] = sl;
    if (s.host_valid[k]) {
      load_pairs_.push_back(s.row[r].host_off + b);
      load_pairs_.push_back(sl);
      stats_.load_bytes_copied += rec * cfg_.num_layers;
    }
  }
  return kOk;
}

void PagedKV::evict_block(Session& s, int64_t b) {
  const size_t rec = rec_bytes();
  for (int r = 0; r < s.rows; ++r) {
    const size_t k = (size_t)b * s.rows + r;
    const int32_t sl = s.slot[k];
    if (sl < 0) continue;
    if (!s.host_valid[k]) {
      evict_pairs_.push_back(sl);
      evict_pairs_.push_back(s.row[r].host_off + b);
      stats_.evict_bytes_copied += rec * cfg_.num_layers;
      s.host_valid[k] = 1;
    }
    // Recycled only by work queued after this call's copies on the caller's stream; a load
    // of this same call that takes the slot is copied after the evictions.
    free_slot(sl);
    s.slot[k] = -1;
  }
}

int PagedKV::apply_tiers(int sid, const uint8_t* tiers, int64_t n_tiers, int64_t* to_gpu, int64_t* n_gpu,
                         int64_t* to_cpu, int64_t* n_cpu, int64_t* fail_block, hipStream_t stream) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  if (in_step_) return fail(kErrState, "apply_tiers during a decode step");
  Session& s = sessions_[sid];
  const int64_t n_full = s.n_tokens / cfg_.tokens_per_block;
  const int64_t bb = block_bytes_all_layers(sid);
  *n_gpu = 0;
  *n_cpu = 0;
  *fail_block = -1;
  // The copies run on the caller's stream: after the kernels already queued there (which
  // may read the blocks being evicted) and before any later work reuses a freed slot. The
  // caller's next kernels wait for them in any case, and a hand-off through the store's copy
  // stream (two events and a cross-queue wait) added ~30 us to a decode step with an eviction.
  // On a stream other than the last decode step's, the copies also wait for that step's
  // launches, which may still append to a block being evicted.
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  if (int rc0 = order_after_decode(stream); rc0 != kOk) return rc0;
  evict_pairs_.clear();
  load_pairs_.clear();
  // Logical pass, ascending by id as kv_block_store.py:216-226: the move lists, the byte
  // accounting and the RAM-budget check (which stops the pass, moves before it stay).
  std::vector<int64_t> evict, load, first_gpu;  // physical work, done below
  int rc = kOk;
  for (int64_t b = 0; b < n_full; ++b) {
    const int desired = b < n_tiers ? tiers[b] : 2;
    const bool phys_gpu = s.slot[(size_t)b * s.rows] >= 0;
    if (desired == 0 && !s.on_gpu[b]) {
      if (s.placed[b]) {
        cpu_bytes_ -= bb;
        load.push_back(b);
      } else {
        first_gpu.push_back(b);  // a prompt block's first place: HBM
      }
      s.placed[b] = 1;
      s.on_gpu[b] = 1;
      gpu_bytes_ += bb;
      stats_.cpu_to_gpu_bytes += bb;
      stats_.cpu_to_gpu_copies += 1;
      to_gpu[(*n_gpu)++] = b;
    } else if (desired == 0 && !phys_gpu) {
      load.push_back(b);  // placed in HBM while its bytes sat on the host: loaded now
    } else if (desired != 0 && s.on_gpu[b]) {
      if (ram_budget_ >= 0 && cpu_bytes_ + bb > ram_budget_) {
        *fail_block = b;
        rc = fail(kErrBudget, "ram_budget exceeded");
        break;
      }
      if (phys_gpu) evict.push_back(b);
      s.on_gpu[b] = 0;
      cpu_bytes_ += bb;
      gpu_bytes_ -= bb;
      stats_.gpu_to_cpu_bytes += bb;
      stats_.gpu_to_cpu_copies += 1;
      to_cpu[(*n_cpu)++] = b;
    } else if (desired != 0 && !s.placed[b]) {
      // A prompt block taking its first place on the host side (kv_block_store.py:83-99
      // checks the budget the same way when the reference offloads it).
      if (ram_budget_ >= 0 && cpu_bytes_ + bb > ram_budget_) {
        *fail_block = b;
        rc = fail(kErrBudget, "ram_budget exceeded");
        break;
      }
      if (phys_gpu) evict.push_back(b);
      cpu_bytes_ += bb;
      s.placed[b] = 1;
    }
  }
  // Physical pass: evictions first, so that loads may take the slots they free; then the
  // loads; then HBM slots for prompt blocks placed in HBM for the first time, the most recent
  // first, as long as the pool keeps one slot per row for the next open block. A prompt block
  // left without a slot stays logically in HBM with its bytes on the host (read from there)
  // until a later placement loads or evicts it.
  for (int64_t b : evict) evict_block(s, b);
  for (int64_t b : load) {
    const int lrc = load_block(s, b);
    if (lrc != kOk) {
      if (rc == kOk) rc = lrc;
      break;
    }
  }
  for (auto it = first_gpu.rbegin(); rc == kOk && it != first_gpu.rend(); ++it) {
    if ((int64_t)free_slots_.size() < 2 * (int64_t)s.rows) break;
    if (s.slot[(size_t)*it * s.rows] >= 0) continue;
    if (load_block(s, *it) != kOk) break;
  }
  // Evictions first: a load may reuse a slot an eviction of this call freed.
  bool launched = false;
  for (int dir = 0; dir < 2; ++dir) {
    std::vector<int64_t>& pairs = dir == 0 ? evict_pairs_ : load_pairs_;
    if (pairs.empty()) continue;
    PendingTiming t{nullptr, nullptr, dir};  // bytes field tags the direction: 0 to host, 1 to GPU
    // Timing-only events: no system-scope fence (cache writeback and invalidate) at record.
    hipEventCreateWithFlags(&t.start, hipEventDisableSystemFence);
    hipEventCreateWithFlags(&t.stop, hipEventDisableSystemFence);
    hipEventRecord(t.start, stream);
    const int l = cfg_.num_layers;
    const int crc = dir == 0 ? launch_copies(pairs, 0, l, stream) : launch_copies(pairs, l, 0, stream);
    hipEventRecord(t.stop, stream);
    move_timing_.push_back(t);
    if (crc != kOk && rc == kOk) rc = crc;
    launched = true;
  }
  if (launched) {
    // Later work on other streams waits for this event (order_after_moves), recorded now so
    // that no later call touches this stream handle again.
    PGR_HIP(hipEventRecord(moves_done_, stream));
    moves_stream_ = stream;
    moves_queued_ = true;
    moves_waited_.clear();
  }
  return rc;
}

int PagedKV::ensure_workspace(size_t bytes) {
  if (bytes <= ws_bytes_) return kOk;
  PGR_HIP(hipDeviceSynchronize());
  forget_streams();
  if (ws_) PGR_HIP(hipFree(ws_));
  ws_ = nullptr;
  const size_t want = std::max(bytes, ws_bytes_ * 3 / 2);
  PGR_HIP(hipMalloc(&ws_, want));
  ws_bytes_ = want;
  return kOk;
}

int PagedKV::default_workgroups() const {
  // Whole workgroups per CU, all resident in one round: three at head_dim <= 64 (four fit),
  // two at 128 (the register ring allows two).
  const int per_cu = cfg_.head_dim <= 64 ? 3 : 2;
  return per_cu * std::max(1, n_cu_);
}

int PagedKV::begin_step(const int32_t* sids, int n, hipStream_t stream) {
  if (in_step_) return fail(kErrState, "begin_step while a step is open");
  if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  const int64_t T = cfg_.tokens_per_block;
  const int E_max = std::min(kMaxWorkEntries, std::max(kWaves, cfg_.blocks_per_workgroup));
  const int64_t target_wg = cfg_.target_workgroups > 0 ? cfg_.target_workgroups : default_workgroups();
  step_sids_.assign(sids, sids + n);
  step_first_.clear();
  seqs_.clear();
  work_.clear();
  copies_.clear();
  mirror_spans_.clear();
  step_host_ids_.clear();
  step_stats_ = StepStats();
  // Validate and open a block where the new token starts one.
  for (int i = 0; i < n; ++i) {
    const int sid = sids[i];
    if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session in step");
    for (int j = 0; j < i; ++j)
      if (sids[j] == sid) return fail(kErrInvalid, "session listed twice in one step");
    Session& s = sessions_[sid];
    const int64_t p = s.n_tokens;
    if (p / T + 1 >= s.capacity_blocks) return fail(kErrCapacity, "session capacity reached");
    if (p % T == 0) {
      for (int r = 0; r < s.rows; ++r) {
        if (s.slot[(p / T) * s.rows + r] >= 0) continue;
        const int sl = alloc_slot();
        if (sl < 0) return fail(kErrCapacity, "HBM pool exhausted (no slot for the new open block)");
        s.slot[(p / T) * s.rows + r] = sl;
      }
    }
  }
  // Per sequence: the stored blocks holding valid tokens [lo, p) -- resident ones read in
  // place, host runs cut into chunks of staging records. The current token (position p) is
  // not read from the store: the merge kernel takes it from k_new / v_new, and the
  // sequence's first work item appends it to the open block.
  struct Pending {
    int seq;
    BlockEntry e;
    int launch;
  };
  std::vector<Pending> pend;
  std::vector<int32_t> append_slot, append_pos;  // per sequence: record and offset of the current token
  const int64_t chunk_cap = cfg_.staging_slots;
  int64_t mirror_ring_used = 0;          // mirror mode: ring records taken by the spans so far
  std::vector<int32_t> seq_mirror_off;   // per sequence: host record - ring record
  ++step_token_;
  int64_t used_in_chunk = 0;
  int chunk = 0;
  int max_mass = 1;
  for (int i = 0; i < n; ++i) {
    Session& s = sessions_[sids[i]];
    const int64_t p = s.n_tokens;
    const int64_t n_full = p / T;
    step_first_.push_back((int32_t)seqs_.size());
    for (int r = 0; r < s.rows; ++r) {
      const int seq = (int)seqs_.size();
      SeqInfo si{};
      si.lo = s.row[r].lo;
      si.hi = (int32_t)p;
      si.n_mass = (int32_t)n_full;
      const int64_t first_blk = std::min<int64_t>(std::max<int64_t>(si.lo, 0) / T, n_full);
      si.mass_lo = (int32_t)first_blk;
      si.session = i;
      si.step_token = step_token_;
      seqs_.push_back(si);
      append_slot.push_back(s.slot[(p / T) * s.rows + r]);
      append_pos.push_back((int32_t)(p % T));
      max_mass = std::max<int>(max_mass, (int)n_full);
      // The gather list: blocks on the host tier (logical residency, paged_model.py:907-916).
      std::vector<int64_t> host_ids;
      for (int64_t x = first_blk; x < n_full; ++x)
        if (!s.on_gpu[x]) host_ids.push_back(x);
      step_stats_.gather_blocks += (int64_t)host_ids.size();
      int64_t span_lo = -1, span_hi = -1;  // mirror mode: this row's host records to copy
      int64_t b = first_blk;
      while (b < n_full) {
        const int32_t sl = s.slot[b * s.rows + r];
        if (sl >= 0) {
          pend.push_back({seq, BlockEntry{sl, (int32_t)b}, 0});
          step_stats_.resident_tokens += T;
          ++b;
          continue;
        }
        int64_t e = b;
        while (e < n_full && s.slot[e * s.rows + r] < 0) ++e;
        for (int64_t x = b; x < e; ++x)
          if (!s.host_valid[x * s.rows + r]) return fail(kErrState, "host block without data (not imported)");
        if (cfg_.stream_mode != 1) {  // direct and mirror: the kernel reads host record indices
          for (int64_t x = b; x < e; ++x)
            pend.push_back({seq, BlockEntry{(int32_t)(-(s.row[r].host_off + x) - 1), (int32_t)x}, 0});
          if (cfg_.stream_mode == 2) {  // one span per row: its first to last host record
            if (span_lo < 0) span_lo = s.row[r].host_off + b;
            span_hi = s.row[r].host_off + e;
          }
          step_stats_.host_blocks += e - b;
          step_stats_.host_tokens += (e - b) * T;
          b = e;
          continue;
        }
        int64_t cur = b;
        while (cur < e) {
          if (used_in_chunk == chunk_cap) {
            ++chunk;
            used_in_chunk = 0;
          }
          const int64_t take = std::min(e - cur, chunk_cap - used_in_chunk);
          const int64_t stage_rec = (int64_t)(chunk % cfg_.staging_buffers) * chunk_cap + used_in_chunk;
          copies_.push_back(CopyCmd{s.row[r].host_off + cur, stage_rec, take, chunk});
          for (int64_t x = 0; x < take; ++x)
            pend.push_back({seq, BlockEntry{(int32_t)(-(stage_rec + x) - 1), (int32_t)(cur + x)}, chunk});
          used_in_chunk += take;
          cur += take;
        }
        step_stats_.host_blocks += e - b;
        step_stats_.host_tokens += (e - b) * T;
        b = e;
      }
      // The open block, when it already holds valid tokens before the current one.
      if (p % T > 0 && p > si.lo)
        pend.push_back({seq, BlockEntry{s.slot[(p / T) * s.rows + r], (int32_t)(p / T)}, 0});
      step_stats_.resident_tokens += p % T + 1;  // stored part of the open block + the current token
      step_host_ids_.push_back(std::move(host_ids));
      // Mirror mode: the row's span is packed into the ring buffers after the spans before it;
      // its host record h then sits at ring record h - mirror_off.
      int32_t moff = 0;
      if (span_lo >= 0) {
        moff = (int32_t)(span_lo - mirror_ring_used);
        mirror_ring_used += span_hi - span_lo;
        mirror_spans_.push_back({span_lo, span_hi - span_lo});
      }
      seq_mirror_off.push_back(moff);
    }
  }
  const bool any_host = !copies_.empty();
  n_chunks_ = any_host ? chunk + 1 : 0;
  // Cross-layer prefetch (staged mode): when the step's host blocks fit one chunk and there
  // are two or more buffers, layer l reads buffer l % buffers, and decode_layer(l) queues
  // layer l+1's copies right after layer l's attention. The copies then run under the rest
  // of layer l's work (projections, MLP), which leaves the host link idle otherwise. Chunk c
  // of a step without prefetch uses buffer c % buffers. Every step starts on buffer 0, so
  // a step's launches are the same as the last step's when its plan has the same shape.
  prefetch_step_ = n_chunks_ == 1 && cfg_.staging_buffers >= 2;
  prefetched_layer_ = -1;
  cap_forked_ = false;
  std::fill(buf_free_cap_.begin(), buf_free_cap_.end(), 0);
  const int n_launch = std::max(1, n_chunks_);
  // Work items. A launch is cut into whole rounds of target_wg / Hkv work items of nearly
  // equal size: the fewest rounds whose items hold at most E_max entries each, so that
  // every CU streams the same number of bytes and no round runs part-full (a few items past
  // a whole round start a straggler round of their own). A small launch gets at least one
  // entry per wave instead. Each sequence gets work items in proportion to its entries in
  // that launch, by largest remainders so that the items add up exactly. A sequence with
  // nothing stored in scope gets one empty work item: its workgroup runs the merge.
  std::vector<int> seq_wg(seqs_.size(), 0);
  std::vector<int> seq_entries(seqs_.size(), 0);
  for (const Pending& pe : pend) ++seq_entries[pe.seq];
  launch_work_begin_.assign(n_launch, 0);
  launch_work_end_.assign(n_launch, 0);
  std::vector<std::vector<size_t>> by_launch(n_launch);
  for (size_t i = 0; i < pend.size(); ++i) by_launch[pend[i].launch].push_back(i);
  auto new_item = [&](int seq) {
    WorkItem w{};
    w.seq = seq;
    w.partial = seq_wg[seq];
    w.lo = seqs_[seq].lo;
    w.hi = seqs_[seq].hi;
    w.n_mass = seqs_[seq].n_mass;
    w.append_slot = seq_wg[seq] == 0 ? append_slot[seq] : -1;
    w.append_pos = append_pos[seq];
    w.mirror_off = seq_mirror_off[seq];
    ++seq_wg[seq];
    return w;
  };
  for (int L = 0; L < n_launch; ++L) {
    launch_work_begin_[L] = (int)work_.size();
    const auto& idx = by_launch[L];
    const int64_t N = (int64_t)idx.size();
    const int64_t per_round = std::max<int64_t>(1, target_wg / cfg_.kv_heads);
    int64_t items;
    if (N <= per_round * kWaves) {
      items = std::max<int64_t>(1, (N + kWaves - 1) / kWaves);
    } else {
      const int64_t rounds = (N + (int64_t)E_max * per_round - 1) / ((int64_t)E_max * per_round);
      items = rounds * per_round;
    }
    // Items per sequence run: proportional shares, at least ceil(ns / E_max) and at most ns
    // each, the remaining items to the largest remainders.
    std::vector<int64_t> run_ns, run_ws;
    std::vector<double> run_rem;
    for (size_t i = 0; i < idx.size();) {
      size_t e = i;
      while (e < idx.size() && pend[idx[e]].seq == pend[idx[i]].seq) ++e;
      run_ns.push_back((int64_t)(e - i));
      i = e;
    }
    int64_t assigned = 0;
    for (int64_t ns : run_ns) {
      const double q = (double)ns * (double)items / (double)std::max<int64_t>(N, 1);
      int64_t w = std::max<int64_t>((int64_t)q, std::max<int64_t>(1, (ns + E_max - 1) / E_max));
      w = std::min<int64_t>(w, ns);
      run_ws.push_back(w);
      run_rem.push_back(q - (double)w);
      assigned += w;
    }
    std::vector<size_t> order(run_ns.size());
    for (size_t r = 0; r < order.size(); ++r) order[r] = r;
    std::stable_sort(order.begin(), order.end(), [&](size_t x, size_t y) { return run_rem[x] > run_rem[y]; });
    for (size_t k = 0; assigned < items && k < order.size(); ++k)
      if (run_ws[order[k]] < run_ns[order[k]]) {
        ++run_ws[order[k]];
        ++assigned;
      }
    size_t i = 0, run = 0;
    while (i < idx.size()) {
      const int seq = pend[idx[i]].seq;
      const int64_t ns = run_ns[run], ws = run_ws[run];
      ++run;
      for (int64_t k = 0; k < ws; ++k) {
        const int64_t cnt = ns / ws + (k < ns % ws ? 1 : 0);
        WorkItem w = new_item(seq);
        for (int64_t x = 0; x < cnt; ++x) w.entries[w.entry_count++] = pend[idx[i++]].e;
        work_.push_back(w);
      }
    }
    if (L == 0) {
      for (size_t q = 0; q < seqs_.size(); ++q)
        if (seq_entries[q] == 0) work_.push_back(new_item((int)q));
    }
    launch_work_end_[L] = (int)work_.size();
  }
  // Partial slots: sequence q owns slots q * stride .. q * stride + stride - 1, stride = the
  // most work items of any sequence, so that the merge finds a sequence's slots without
  // reading the plan (it issues the loads of its first batch at once, and masks the slots
  // past the sequence's count when that arrives). When that would take more than twice the
  // packed slots (plus 1024), the slots are packed and the merge reads where they start.
  int stride = 1, packed = 0;
  for (size_t q = 0; q < seqs_.size(); ++q) {
    stride = std::max(stride, seq_wg[q]);
    packed += seq_wg[q];
  }
  const bool fixed = (int64_t)seqs_.size() * stride <= 2 * (int64_t)packed + 1024;
  int base = 0;
  for (size_t q = 0; q < seqs_.size(); ++q) {
    seqs_[q].partial_base = fixed ? (int32_t)q * stride : base;
    seqs_[q].partial_count = seq_wg[q];
    base += seq_wg[q];
  }
  for (WorkItem& w : work_) w.partial += seqs_[w.seq].partial_base;
  n_partials_ = fixed ? (int)seqs_.size() * stride : packed;
  partial_stride_ = fixed ? stride : 0;
  mass_stride_ = max_mass;
  step_stats_.copies = (int64_t)copies_.size();
  step_stats_.chunks = n_chunks_;
  step_stats_.launches = n_launch;
  step_stats_.work_items = (int64_t)work_.size();

  // Workspace layout.
  const int S = (int)seqs_.size();
  const int hq = cfg_.query_heads;
  std::vector<int32_t> sess_rows, sess_first;
  for (int i = 0; i < n; ++i) {
    sess_rows.push_back(sessions_[sids[i]].rows);
    sess_first.push_back(step_first_[i]);
  }
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  // Plan: the per-sequence and per-session arrays, the chunks' bounds in the staging pair
  // list, the work items, then the pairs (ahead of the work items, only the bounds array,
  // which holds 32 chunks in its 256 bytes, so the work items stay where they were).
  const size_t o_seqs = carve(sizeof(SeqInfo) * S);
  const size_t o_srows = carve(sizeof(int32_t) * std::max(n, 1));
  const size_t o_sfirst = carve(sizeof(int32_t) * std::max(n, 1));
  const size_t o_cbegin = carve(sizeof(int64_t) * (size_t)(n_chunks_ + 1));
  // Staged mode: (host record, staging record) per record to stream, chunk by chunk.
  stage_pairs_.clear();
  chunk_pair_begin_.assign(n_chunks_ + 1, 0);
  for (const CopyCmd& c : copies_) {
    for (int64_t x = 0; x < c.count; ++x) {
      stage_pairs_.push_back(c.host_rec + x);
      stage_pairs_.push_back(c.stage_rec + x);
    }
    chunk_pair_begin_[c.chunk + 1] = (int64_t)stage_pairs_.size() / 2;
  }
  for (int c = 1; c <= n_chunks_; ++c) chunk_pair_begin_[c] = std::max(chunk_pair_begin_[c], chunk_pair_begin_[c - 1]);
  const size_t o_work = carve(sizeof(WorkItem) * std::max<size_t>(work_.size(), 1));
  const size_t o_spairs = carve(sizeof(int64_t) * std::max<size_t>(stage_pairs_.size(), 2));
  const size_t plan_bytes = off;
  const size_t o_pm = carve(sizeof(float) * (size_t)n_partials_ * hq);
  const size_t o_pl = carve(sizeof(float) * (size_t)n_partials_ * hq);
  const size_t o_pacc = carve(sizeof(float) * (size_t)n_partials_ * hq * cfg_.head_dim);
  const size_t o_mm = carve(sizeof(float) * (size_t)S * hq * mass_stride_);
  const size_t o_ms = carve(sizeof(float) * (size_t)S * hq * mass_stride_);
  const size_t o_mf = carve(sizeof(float) * (size_t)S * hq);
  const size_t o_lf = carve(sizeof(float) * (size_t)S * hq);
  int rc = ensure_workspace(off);
  if (rc != kOk) return rc;
  // Deferred mass for steps with sessions whose pager scores by mass: one [S][Hq][stride]
  // share per layer, cleared by each step's reduction (and zero when allocated).
  mass_deferred_ = false;
  mass_w_dirty_ = false;
  {
    bool want = false;
    for (int i = 0; i < n; ++i) want = want || (sessions_[sids[i]].pager && sessions_[sids[i]].scores_from_mass);
    const size_t layer_floats = (size_t)S * hq * mass_stride_;
    const size_t total = layer_floats * cfg_.num_layers;
    if (want && total <= kMassDeferredMaxFloats) {
      if (total > mass_w_floats_) {
        PGR_HIP(hipDeviceSynchronize());
        forget_streams();
        const size_t grow = std::max(total, mass_w_floats_ * 3 / 2);
        if (mass_w_) PGR_HIP(hipFree(mass_w_));
        mass_w_ = nullptr;
        mass_w_floats_ = 0;
        PGR_HIP(hipMalloc(reinterpret_cast<void**>(&mass_w_), grow * sizeof(float)));
        PGR_HIP(hipMemset(mass_w_, 0, grow * sizeof(float)));
        mass_w_floats_ = grow;
      }
      mass_deferred_ = true;
      mass_layer_floats_ = layer_floats;
    }
  }
  // Pinned plan buffer; wait until the GPU has read it before overwriting it. With several
  // layers per step the first launch reads the plan early in its step, so one buffer holds
  // the host back by little, and a launch signature stays the same from step to step (a
  // captured graph replays). With one layer the first launch is the whole step: the steps
  // alternate between two buffers, so that the host can plan a step while the GPU runs the
  // one before.
  if (cfg_.num_layers == 1) plan_buf_ ^= 1;
  PlanBuf& pb = plan_bufs_[plan_buf_];
  if (pb.pending) {
    pb.pending = false;
    const auto w0 = std::chrono::steady_clock::now();
    if (pb.by_flag) {
      const int rc = wait_plan_flag(pb, plan_buf_);
      if (rc != kOk) return rc;
    } else {
      PGR_HIP(hipEventSynchronize(pb.read));
    }
    step_stats_.plan_wait_ns =
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - w0).count();
  }
  if (plan_bytes > pb.bytes) {
    if (pb.host) PGR_HIP(hipHostFree(pb.host));
    pb.host = nullptr;
    const size_t want = std::max(plan_bytes, pb.bytes * 3 / 2);
    PGR_HIP(hipHostMalloc(&pb.host, want, hipHostMallocDefault));
    PGR_HIP(hipHostGetDevicePointer(&pb.dev, pb.host, 0));
    pb.bytes = want;
  }
  plan_aux_bytes_ = o_work;
  plan_work_off_ = o_work;
  char* h = static_cast<char*>(pb.host);
  std::memcpy(h + o_seqs, seqs_.data(), sizeof(SeqInfo) * S);
  std::memcpy(h + o_work, work_.data(), sizeof(WorkItem) * work_.size());
  std::memcpy(h + o_srows, sess_rows.data(), sizeof(int32_t) * n);
  std::memcpy(h + o_sfirst, sess_first.data(), sizeof(int32_t) * n);
  std::memcpy(h + o_cbegin, chunk_pair_begin_.data(), sizeof(int64_t) * chunk_pair_begin_.size());
  if (!stage_pairs_.empty()) std::memcpy(h + o_spairs, stage_pairs_.data(), sizeof(int64_t) * stage_pairs_.size());
  char* d = static_cast<char*>(ws_);
  // A staging copy queued for a layer that was never decoded may still read the previous
  // step's pair list on the copy stream: the plan is not overwritten before it has run.
  if (stage_copy_pending_) {
    PGR_HIP(hipStreamWaitEvent(stream, stage_copies_done_, 0));
    stage_copy_pending_ = false;
  }
  plan_on_device_ = false;
  if (cfg_.stream_mode == 1) {
    // Staged mode: the staging copies read the pair list before any attention launch runs,
    // so the whole plan goes to the workspace first. plan_bytes is a multiple of 256.
    const int64_t n_vec = (int64_t)(plan_bytes / 16);
    plan_upload_kernel<<<(unsigned)((n_vec + 255) / 256), 256, 0, stream>>>(pb.dev, d, n_vec);
    PGR_HIP(hipGetLastError());
    PGR_HIP(hipEventRecord(plan_uploaded_, stream));
    PGR_HIP(hipEventRecord(pb.read, stream));
    pb.pending = true;
    pb.by_flag = false;
    plan_on_device_ = true;
  }
  // Direct mode: the step's first attention launch reads its work items from the pinned
  // buffer and copies the plan into the workspace for every later kernel (decode_layer).
  d_seqs_ = reinterpret_cast<SeqInfo*>(d + o_seqs);
  d_work_ = reinterpret_cast<WorkItem*>(d + o_work);
  d_sess_rows_ = reinterpret_cast<int32_t*>(d + o_srows);
  d_sess_first_ = reinterpret_cast<int32_t*>(d + o_sfirst);
  d_stage_pairs_ = reinterpret_cast<int64_t*>(d + o_spairs);
  d_chunk_begin_ = reinterpret_cast<int64_t*>(d + o_cbegin);
  d_pm_ = reinterpret_cast<float*>(d + o_pm);
  d_pl_ = reinterpret_cast<float*>(d + o_pl);
  d_pacc_ = reinterpret_cast<float*>(d + o_pacc);
  d_mass_m_ = reinterpret_cast<float*>(d + o_mm);
  d_mass_s_ = reinterpret_cast<float*>(d + o_ms);
  d_mf_ = reinterpret_cast<float*>(d + o_mf);
  d_lf_ = reinterpret_cast<float*>(d + o_lf);
  if (cfg_.stream_mode == 2)
    if (int rc = issue_mirror_copies(stream); rc != kOk) return rc;
  in_step_ = true;
  return kOk;
}

// Mirror mode (end of begin_step). The layers' "mirror filled" words are reset on the step's
// stream once the previous step's copies have finished (a word set late by one of them
// would announce that step's data); this step's copies then start on the copy stream behind
// that point, so after the previous step's launches, which read the mirrors, and after tier
// moves queued on `stream`. Per layer: one DMA copy per row span (its first to last host
// record of the step), then the layer's word, written by the copy stream itself
// (hipStreamWriteValue32, which the runtime executes as a one-workgroup kernel on that
// stream's queue). A launch polling the word holds one lane per workgroup and gives up after
// its bounded wait, so it cannot hold the write up for good. Writing the words from a third
// stream that waits on a per-layer event after the copies measured slower on configuration
// 3 (6.6 against 6.3 ms per token).
// The copy-stream calls run on mirror_issuer_'s thread: the GPU starts the step (its first
// kernels wait for the host to return from begin_step) while they are issued. Everything the
// job reads is fixed after init, apart from the spans, which it takes by value; the GPU-side
// order is the same as when the calls are made here, as every copy waits for mirror_go_.
// They may overlap a graph capture that the caller begins on its own stream after
// begin_step: all of them are asynchronous calls on the store's non-blocking copy stream,
// which a capture in global mode permits on other threads (no implicit synchronization).
int PagedKV::issue_mirror_copies(hipStream_t stream) {
  if (int rc = order_after_decode(stream); rc != kOk) return rc;
  PGR_HIP(mirror_issuer_.wait());  // the last step's job: mirror_done_ is recorded
  if (mirror_pending_) {
    PGR_HIP(hipStreamWaitEvent(stream, mirror_done_, 0));
    mirror_pending_ = false;
  }
  // Each ring buffer holds one layer's share of the step: the rows' spans, packed.
  int64_t need = 0;
  for (const auto& sp : mirror_spans_) need += sp.second;
  if (need > ring_records_) {
    PGR_HIP(hipDeviceSynchronize());
    forget_streams();
    const int64_t grow = std::max(need, ring_records_ * 3 / 2);
    for (void*& b : ring_) {
      if (b) PGR_HIP(hipFree(b));
      b = nullptr;
    }
    ring_records_ = 0;
    for (void*& b : ring_) PGR_HIP(hipMalloc(&b, rec_bytes() * (size_t)grow));
    ring_records_ = grow;
  }
  mirror_flags_reset_kernel<<<1, 256, 0, stream>>>(mirror_flags_, cfg_.num_layers, mirror_spans_.empty() ? 1u : 0u);
  PGR_HIP(hipGetLastError());
  mirror_step_bytes_ = 0;
  if (mirror_spans_.empty()) return kOk;
  PGR_HIP(hipEventRecord(mirror_go_, stream));
  const size_t rec = rec_bytes();
  for (const auto& sp : mirror_spans_) mirror_step_bytes_ += (uint64_t)sp.second * rec;
  mirror_pending_ = true;
  step_closed_ = false;
  const uint32_t token = step_token_;
  const bool timed = timing_;
  mirror_issuer_.submit([this, rec, token, timed, spans = mirror_spans_, ring = ring_]() -> hipError_t {
    const int n_ring = (int)ring.size();
    hipError_t e = hipSetDevice(device_);
    if (e == hipSuccess) e = hipStreamWaitEvent(copy_stream_, mirror_go_, 0);
    for (int l = 0; l < cfg_.num_layers && e == hipSuccess; ++l) {
      // Buffer l % n was last read by layer l - n of this step: its records may be replaced
      // once that layer's merge has published the step's token.
      if (l >= n_ring && !wait_release(l - n_ring, token)) break;
      char* dst = static_cast<char*>(ring[l % n_ring]);
      PendingTiming t{nullptr, nullptr, 0};
      if (timed) {  // events around the layer's copies on the copy stream (measurement only)
        e = hipEventCreateWithFlags(&t.start, hipEventDisableSystemFence);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&t.stop, hipEventDisableSystemFence);
        if (e == hipSuccess) e = hipEventRecord(t.start, copy_stream_);
      }
      int64_t at = 0;
      for (size_t i = 0; i < spans.size() && e == hipSuccess; ++i) {
        e = hipMemcpyHtoDAsync(dst + (size_t)at * rec, static_cast<char*>(host_[l]) + (size_t)spans[i].first * rec,
                               (size_t)spans[i].second * rec, copy_stream_);
        at += spans[i].second;
      }
      if (timed && e == hipSuccess) {
        e = hipEventRecord(t.stop, copy_stream_);
        t.bytes = at * (int64_t)rec;
        std::lock_guard<std::mutex> lk(copy_timing_mu_);
        copy_timing_.push_back(t);
      }
      if (e == hipSuccess) e = hipStreamWriteValue32(copy_stream_, mirror_flags_ + l, 1u, 0);
    }
    const hipError_t e2 = hipEventRecord(mirror_done_, copy_stream_);
    return e != hipSuccess ? e : e2;
  });
  return kOk;
}

bool PagedKV::wait_release(int layer, uint32_t token) {
  auto released = [&] { return (int32_t)(__atomic_load_n(mirror_release_ + layer, __ATOMIC_ACQUIRE) - token) >= 0; };
  if (released()) return true;
  mirror_waiting_ = 1;
  const auto t0 = std::chrono::steady_clock::now();
  bool ok = false;
  for (uint64_t poll = 1;; ++poll) {
    if (released()) {
      ok = true;
      break;
    }
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
    if ((poll & 1023) != 0) continue;
    if (mirror_cancel_) break;
    if (step_closed_) {
      // The step is closed: every launch of it is queued on its decode stream. Once that has
      // drained, a release still missing never comes (a layer that was not decoded).
      const hipError_t q = closed_has_stream_ ? hipStreamQuery(closed_stream_.load()) : hipSuccess;
      if (q != hipErrorNotReady) {
        ok = released();
        break;
      }
    }
    if (std::chrono::steady_clock::now() - t0 > kReleaseWaitLimit) break;
  }
  mirror_waiting_ = 0;
  return ok;
}

void PagedKV::base_launch(PagedLaunch& pl, int layer, const void* q, const void* k_new, const void* v_new, void* out,
                          bool mass, float scale, float softcap, int window) const {
  pl.q = q;
  pl.k_new = k_new;
  pl.v_new = v_new;
  pl.pool = pool_[layer];
  pl.stage = cfg_.stream_mode == 1 ? stage_ : host_dev_[layer];
  if (cfg_.stream_mode == 2) {
    pl.mirror = ring_[layer % ring_.size()];
    pl.mirror_flag = mirror_flags_ + layer;
    pl.release_flag = mirror_release_dev_ + layer;
  }
  pl.seqs = d_seqs_;
  pl.pm = d_pm_;
  pl.pl = d_pl_;
  pl.pacc = d_pacc_;
  pl.mass_m = mass ? d_mass_m_ : nullptr;
  pl.mass_s = mass ? d_mass_s_ : nullptr;
  pl.out = out;
  pl.mf = d_mf_;
  pl.lf = d_lf_;
  pl.hq = cfg_.query_heads;
  pl.hkv = cfg_.kv_heads;
  pl.tokens_per_block = cfg_.tokens_per_block;
  pl.mass_stride = mass_stride_;
  pl.partial_stride = partial_stride_;
  pl.scale = scale;
  pl.softcap = softcap;
  pl.window = window;
}

// Measurement only. The attention launches of decode_layer for every layer, again, with the
// plan already on the device (so every launch reads its work items from the workspace, as
// the step's launches after its first do), reps times back to back between two fence-free
// events: per-launch events add the time between each start marker and its dispatch, about
// 1.6 us on a 13 us launch. The launches rewrite the step's partials and, in each layer, its
// current token (the caller passes each layer's q, k_new and v_new of the step); the merges,
// and so the step's outputs, are not repeated.
int PagedKV::bench_attention(const void* const* q, const void* const* k_new, const void* const* v_new, float scale,
                             float softcap, int reps, hipStream_t stream, double* us_per_launch,
                             int64_t* bytes_per_launch) {
  if (!in_step_ || !plan_on_device_)
    return fail(kErrState, "bench_attention needs an open step whose first layer was decoded");
  if (cfg_.stream_mode != 0) return fail(kErrUnsupported, "bench_attention runs in the direct stream mode only");
  if (reps <= 0 || !q || !k_new || !v_new || !us_per_launch || !bytes_per_launch)
    return fail(kErrInvalid, "bench_attention: reps > 0 and q, k_new, v_new and outputs required");
  for (int layer = 0; layer < cfg_.num_layers; ++layer)
    if (!q[layer] || !k_new[layer] || !v_new[layer]) return fail(kErrInvalid, "bench_attention: a null layer input");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PGR_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap != hipStreamCaptureStatusNone) return fail(kErrState, "bench_attention under stream capture");
  int64_t ent = 0;
  for (const WorkItem& w : work_) ent += w.entry_count;
  hipEvent_t ev[2] = {nullptr, nullptr};
  for (hipEvent_t& e : ev) PGR_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  hipError_t e = hipEventRecord(ev[0], stream);
  int launches = 0;
  for (int r = 0; r < reps && e == hipSuccess; ++r)
    for (int layer = 0; layer < cfg_.num_layers && e == hipSuccess; ++layer) {
      PagedLaunch pl{};
      base_launch(pl, layer, q[layer], k_new[layer], v_new[layer], nullptr, false, scale, softcap, 0);
      pl.work = d_work_;
      pl.n_work = (int)work_.size();
      e = launch_paged(cfg_.dtype, cfg_.head_dim, pl, stream);
      ++launches;
    }
  if (e == hipSuccess) e = hipEventRecord(ev[1], stream);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
  for (hipEvent_t x : ev) (void)hipEventDestroy(x);
  if (e != hipSuccess) return hip_fail(e, "bench_attention");
  *us_per_launch = (double)ms * 1e3 / launches;
  *bytes_per_launch = ent * (int64_t)cfg_.tokens_per_block * 2 * cfg_.head_dim * 2 * cfg_.kv_heads;
  return kOk;
}

int PagedKV::decode_layer(int layer, const void* q, const void* k_new, const void* v_new, void* out,
                          float* mass_accum, int64_t accum_stride, float scale, float softcap, int window,
                          hipStream_t stream) {
  if (!in_step_) return fail(kErrState, "decode_layer outside begin_step/end_step");
  if (layer < 0 || layer >= cfg_.num_layers) return fail(kErrInvalid, "layer out of range");
  // Under stream capture nothing runs now: no cross-stream wait is recorded (the capture
  // starts after the caller's earlier work), and neither the plan buffer (below) nor the
  // decode stream is marked; step_replayed does both for each replay.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PGR_HIP(hipStreamIsCapturing(stream, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (!capturing)
    if (int rc0 = order_after_moves(stream); rc0 != kOk) return rc0;
  const int hq = cfg_.query_heads;
  const int T = cfg_.tokens_per_block;
  const size_t rec = rec_bytes();
  PagedLaunch pl{};
  base_launch(pl, layer, q, k_new, v_new, out, mass_accum != nullptr, scale, softcap, window);
  const int n_launch = (int)launch_work_begin_.size();
  const int nbuf = cfg_.staging_buffers;
  // Side stream: wait until the previous reader of buffer `buf` finished, then stream the
  // host runs of chunk `L` of layer `lay` into it. `shift` moves the plan's records (laid out
  // for buffer 0) to buffer `buf`.
  auto issue_copies = [&](int lay, int L, int buf, int64_t shift) -> int {
    if (capturing) {
      // Everything queued before the graph's launch precedes it: join the capture once, then
      // wait only for this step's readers of the buffer.
      if (!cap_forked_) {
        PGR_HIP(hipEventRecord(cap_fork_, stream));
        PGR_HIP(hipStreamWaitEvent(copy_stream_, cap_fork_, 0));
        cap_forked_ = true;
      }
      if (buf_free_cap_[buf]) PGR_HIP(hipStreamWaitEvent(copy_stream_, buf_free_[buf], 0));
    } else {
      // The pair list is part of the step plan: wait for its upload (which follows every
      // earlier step, replayed ones included) and for the buffer's last reader.
      PGR_HIP(hipStreamWaitEvent(copy_stream_, plan_uploaded_, 0));
      if (buf_free_eager_[buf]) PGR_HIP(hipStreamWaitEvent(copy_stream_, buf_free_[buf], 0));
    }
    stage_copy_kernel<<<kStageCopyWorkgroups, 256, 0, copy_stream_>>>(
        host_dev_[lay], static_cast<char*>(stage_) + shift * (int64_t)rec, d_stage_pairs_, d_chunk_begin_ + L,
        (int64_t)(rec / 16));
    PGR_HIP(hipGetLastError());
    PGR_HIP(hipEventRecord(chunk_ready_[buf], copy_stream_));
    if (!capturing) {
      // A capture is joined back by the launches that wait on chunk_ready_, and a replay ends
      // with its copies; only eager copies may still run when the next step begins.
      PGR_HIP(hipEventRecord(stage_copies_done_, copy_stream_));
      stage_copy_pending_ = true;
    }
    return kOk;
  };
  auto layer_buf = [&](int lay) { return lay % nbuf; };
  auto layer_shift = [&](int lay) { return (int64_t)layer_buf(lay) * cfg_.staging_slots; };
  uint32_t* merge_flag = nullptr;  // set when this call makes the step's first (plan-reading) launch
  uint32_t merge_token = 0;
  for (int L = 0; L < n_launch; ++L) {
    const int buf = prefetch_step_ ? layer_buf(layer) : L % nbuf;
    if (n_chunks_ > 0) {
      if (!(prefetch_step_ && prefetched_layer_ == layer)) {
        const int rc = issue_copies(layer, L, buf, prefetch_step_ ? layer_shift(layer) : 0);
        if (rc != kOk) return rc;
      }
      PGR_HIP(hipStreamWaitEvent(stream, chunk_ready_[buf], 0));
      if (prefetch_step_) pl.stage = static_cast<const char*>(stage_) + layer_shift(layer) * (int64_t)rec;
    }
    pl.work = d_work_ + launch_work_begin_[L];
    pl.n_work = launch_work_end_[L] - launch_work_begin_[L];
    pl.work_out = nullptr;
    pl.aux_src = nullptr;
    pl.aux_dst = nullptr;
    pl.aux_vec = 0;
    const bool first_read = !plan_on_device_;  // direct mode, first decode_layer of the step
    if (first_read) {
      const PlanBuf& pb = plan_bufs_[plan_buf_];
      pl.work = reinterpret_cast<const WorkItem*>(static_cast<const char*>(pb.dev) + plan_work_off_) +
                launch_work_begin_[L];
      pl.work_out = d_work_ + launch_work_begin_[L];
      pl.aux_src = pb.dev;
      pl.aux_dst = ws_;
      pl.aux_vec = (int64_t)(plan_aux_bytes_ / 16);
    }
    PendingTiming t{nullptr, nullptr, 0};
    const bool timed = timing_ && !capturing;  // no event nodes in a captured graph
    if (timed) {
      // Timing-only events recorded on the stream right before and after the launch. Without
      // a system-scope fence at record time they do not write back and invalidate the caches
      // around the launch they stamp. (Events handed to the launch itself read 15 to 18 us on
      // the same launches, varying from process to process.) They come from a pool: creating
      // two events per launch made a timed pass host-bound, and then a launch's interval also
      // held the host's time between recording its start and submitting it.
      PGR_HIP(timing_event(&t.start));
      PGR_HIP(timing_event(&t.stop));
      PGR_HIP(hipEventRecord(t.start, stream));
    }
    PGR_HIP(launch_paged(cfg_.dtype, cfg_.head_dim, pl, stream));
    if (timed) PGR_HIP(hipEventRecord(t.stop, stream));
    if (first_read) {
      // The merge below stores the buffer's token once this launch has finished. Under stream
      // capture nothing runs now and the captured launches carry no token: the caller marks
      // the buffer after each replay of the graph (step_replayed).
      PlanBuf& pb = plan_bufs_[plan_buf_];
      if (!capturing) {
        pb.token = ++plan_token_;
        pb.by_flag = true;
        pb.pending = true;
        pb.stream = stream;
        merge_flag = plan_flags_dev_ + plan_buf_;
        merge_token = pb.token;
      }
      plan_on_device_ = true;
    }
    if (timed) {
      int64_t ent = 0;
      for (int w = launch_work_begin_[L]; w < launch_work_end_[L]; ++w) ent += work_[w].entry_count;
      t.bytes = ent * (int64_t)T * 2 * cfg_.head_dim * 2 * cfg_.kv_heads;  // K+V bytes read, whole blocks
      timing_pending_.push_back(t);
    }
    if (n_chunks_ > 0) {
      PGR_HIP(hipEventRecord(buf_free_[buf], stream));
      buf_free_cap_[buf] = capturing;
      buf_free_eager_[buf] = !capturing;
    }
  }
  prefetched_layer_ = -1;
  if (prefetch_step_ && layer + 1 < cfg_.num_layers) {
    const int rc = issue_copies(layer + 1, 0, layer_buf(layer + 1), layer_shift(layer + 1));
    if (rc != kOk) return rc;
    prefetched_layer_ = layer + 1;
  }
  pl.plan_flag = merge_flag;
  pl.plan_token = merge_token;
  // Deferred mass: the merge writes this layer's block weights, the step's reduction adds
  // them up once (end_step / end_step_place); otherwise a reduction per layer.
  const bool deferred = mass_accum && mass_deferred_;
  if (deferred) {
    pl.mass_w = mass_w_ + (size_t)layer * mass_layer_floats_;
    if (!capturing) mass_w_dirty_ = true;  // a replay marks it (step_replayed)
  }
  PGR_HIP(launch_paged_merge(cfg_.dtype, cfg_.head_dim, pl, (int)seqs_.size(), stream));
  if (mass_accum && !deferred) {
    PGR_HIP(launch_mass_reduce(d_seqs_, d_sess_rows_, d_sess_first_, d_mass_m_, d_mass_s_, d_mf_, d_lf_, mass_accum,
                               (int)accum_stride, hq, mass_stride_, (int)step_sids_.size(), mass_stride_, stream));
  }
  if (mass_accum) {
    mass_accum_last_ = mass_accum;
    mass_stride_last_ = accum_stride;
  }
  if (!capturing) {
    decode_stream_ = stream;
    decode_pending_ = true;
    decode_waited_.clear();
  }
  return kOk;
}

int PagedKV::step_replayed(hipStream_t stream) {
  if (!in_step_) return fail(kErrState, "step_replayed outside begin_step/end_step");
  PlanBuf& pb = plan_bufs_[plan_buf_];
  // The event follows the whole replay; begin_step waits on it before it writes this buffer
  // again (a replayed launch carries no flag token, unlike an eager one). It replaces a flag
  // guard an eager launch of this step may have set, and covers that launch too.
  PGR_HIP(hipEventRecord(pb.read, stream));
  pb.pending = true;
  pb.by_flag = false;
  pb.stream = stream;
  plan_on_device_ = true;
  decode_stream_ = stream;
  decode_pending_ = true;
  decode_waited_.clear();
  // A graph captured with deferred mass writes the step's block weights on every replay.
  if (mass_deferred_ && mass_accum_last_) mass_w_dirty_ = true;
  return kOk;
}

int PagedKV::step_signature(int64_t* out, int64_t cap) const {
  if (!in_step_) return kErrState;
  std::vector<int64_t> v = {
      (int64_t)(uintptr_t)ws_, (int64_t)(uintptr_t)d_seqs_, (int64_t)(uintptr_t)d_work_,
      (int64_t)(uintptr_t)d_sess_rows_, (int64_t)(uintptr_t)d_sess_first_, (int64_t)(uintptr_t)d_pm_,
      (int64_t)(uintptr_t)d_pl_, (int64_t)(uintptr_t)d_pacc_, (int64_t)(uintptr_t)d_mass_m_,
      (int64_t)(uintptr_t)d_mass_s_, (int64_t)(uintptr_t)d_mf_, (int64_t)(uintptr_t)d_lf_,
      (int64_t)cfg_.stream_mode, (int64_t)seqs_.size(), (int64_t)step_sids_.size(), (int64_t)mass_stride_,
      (int64_t)launch_work_begin_.size(), (int64_t)(uintptr_t)plan_bufs_[plan_buf_].dev, (int64_t)plan_on_device_,
      (int64_t)n_chunks_, (int64_t)prefetch_step_, (int64_t)(uintptr_t)d_stage_pairs_,
      (int64_t)(uintptr_t)d_chunk_begin_, (int64_t)mass_deferred_, (int64_t)(uintptr_t)mass_w_,
      (int64_t)mass_layer_floats_, ring_records_, (int64_t)partial_stride_};
  for (void* b : ring_) v.push_back((int64_t)(uintptr_t)b);
  for (size_t L = 0; L < launch_work_begin_.size(); ++L) {
    v.push_back(launch_work_begin_[L]);
    v.push_back(launch_work_end_[L]);
  }
  if (out)
    for (size_t i = 0; i < v.size() && (int64_t)i < cap; ++i) out[i] = v[i];
  return (int)v.size();
}

int PagedKV::finish_step_mass(float* mass_accum, int64_t accum_stride, hipStream_t stream) {
  PGR_HIP(launch_mass_step_reduce(d_seqs_, d_sess_rows_, d_sess_first_, mass_w_, (int64_t)mass_layer_floats_,
                                  cfg_.num_layers, mass_accum, (int)accum_stride, cfg_.query_heads, mass_stride_,
                                  (int)step_sids_.size(), mass_stride_, stream));
  // The next step's merges write the weights this launch clears: work on another stream
  // waits for it (order_after_moves).
  PGR_HIP(hipEventRecord(moves_done_, stream));
  moves_stream_ = stream;
  moves_queued_ = true;
  moves_waited_.clear();
  return kOk;
}

int PagedKV::end_step(int32_t* completed, int* n_completed) {
  if (!in_step_) return fail(kErrState, "end_step without begin_step");
  if (mass_deferred_ && mass_w_dirty_ && mass_accum_last_)
    if (int rc = finish_step_mass(mass_accum_last_, mass_stride_last_, decode_stream_); rc != kOk) return rc;
  return close_step(completed, n_completed);
}

int PagedKV::close_step(int32_t* completed, int* n_completed) {
  const int64_t T = cfg_.tokens_per_block;
  // Host blocks read in place (direct mode) or copied to staging (staged mode) this step, every
  // layer (counted here rather than per launch, so that steps replayed from a captured graph
  // are counted too).
  stats_.stream_bytes += (uint64_t)step_stats_.host_blocks * rec_bytes() * cfg_.num_layers;
  if (cfg_.stream_mode == 2) stats_.stream_copies += (uint64_t)mirror_spans_.size() * cfg_.num_layers;
  if (cfg_.stream_mode == 1) stats_.stream_copies += (uint64_t)copies_.size() * cfg_.num_layers;
  int c = 0;
  for (size_t i = 0; i < step_sids_.size(); ++i) {
    Session& s = sessions_[step_sids_[i]];
    const int64_t p = s.n_tokens;
    s.n_tokens = p + 1;
    if ((p + 1) % T == 0) {
      const int64_t b = p / T;
      s.on_gpu[b] = 1;
      s.placed[b] = 1;
      for (int r = 0; r < s.rows; ++r) s.host_valid[b * s.rows + r] = 0;
      gpu_bytes_ += block_bytes_all_layers(step_sids_[i]);
      if (completed) completed[c] = step_sids_[i];
      ++c;
    }
  }
  if (n_completed) *n_completed = c;
  in_step_ = false;
  if (cfg_.stream_mode == 2) {  // the mirror thread may now tell a missing release from a late one
    closed_has_stream_ = decode_pending_;
    closed_stream_ = decode_stream_;
    step_closed_ = true;
  }
  return kOk;
}

int PagedKV::attach_pager(int sid, PlacementPager* pager, bool scores_from_mass) {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return fail(kErrKey, "unknown session");
  sessions_[sid].pager = pager;
  sessions_[sid].scores_from_mass = scores_from_mass;
  return kOk;
}

int PagedKV::end_step_place(float* mass_accum, int64_t accum_stride, int num_layers, hipStream_t stream,
                            int32_t* completed, int* n_completed, int64_t* counts, int64_t* moves,
                            int64_t moves_cap, double* scores, int64_t scores_cap) {
  if (!in_step_) return fail(kErrState, "end_step_place without begin_step");
  const int64_t T = cfg_.tokens_per_block;
  const std::vector<int32_t> sids = step_sids_;
  const int n = (int)sids.size();
  std::vector<int64_t> n_mass_old(n);
  bool need_mass = false;
  for (int i = 0; i < n; ++i) {
    const Session& s = sessions_[sids[i]];
    n_mass_old[i] = s.n_tokens / T;
    need_mass = need_mass || (s.pager && s.scores_from_mass);
  }
  // Reading the mass and moving records on a stream other than the decode stream waits for
  // the step's launches first.
  if (int rc0 = order_after_decode(stream); rc0 != kOk) return rc0;
  if (need_mass) {
    if (!mass_accum || accum_stride <= 0) return fail(kErrInvalid, "scoring policy needs the mass accumulator");
    const size_t want = (size_t)n * accum_stride;
    if (want > mass_host_floats_) {
      PGR_HIP(hipStreamSynchronize(stream));
      if (mass_host_) PGR_HIP(hipHostFree(mass_host_));
      mass_host_ = nullptr;
      PGR_HIP(hipHostMalloc(reinterpret_cast<void**>(&mass_host_), want * sizeof(float), hipHostMallocDefault));
      mass_host_floats_ = want;
    }
    // The reduction reads the step's plan, which the step's first launch put on the device.
    if (mass_deferred_ && mass_w_dirty_)
      if (int rc = finish_step_mass(mass_accum, accum_stride, stream); rc != kOk) return rc;
    // The reference reads the mass back with .tolist() (a full sync) at this point too.
    PGR_HIP(hipMemcpyAsync(mass_host_, mass_accum, want * sizeof(float), hipMemcpyDeviceToHost, stream));
    PGR_HIP(hipStreamSynchronize(stream));
  }
  std::vector<int32_t> done(n);
  int n_done = 0;
  int rc = close_step(done.data(), &n_done);
  if (rc != kOk) return rc;
  if (completed)
    for (int i = 0; i < n_done; ++i) completed[i] = done[i];
  if (n_completed) *n_completed = n_done;
  int64_t mo = 0, so = 0;
  std::vector<float> fscores;
  std::vector<double> dscores;
  std::vector<uint8_t> tiers;
  for (int i = 0; i < n; ++i) {
    const int sid = sids[i];
    Session& s = sessions_[sid];
    int64_t* c = counts ? counts + 5 * i : nullptr;
    const int64_t n_blocks = s.n_tokens / T;
    const bool added = std::find(done.begin(), done.begin() + n_done, sid) != done.begin() + n_done;
    if (c) {
      c[0] = added ? n_blocks - 1 : -1;
      c[1] = c[2] = c[4] = 0;
      c[3] = -1;
    }
    if (!s.pager || n_blocks == 0) continue;
    // paged_model.py:781-790 and :865-876.
    dscores.clear();
    if (s.scores_from_mass) {
      const float* row = mass_host_ + (size_t)i * accum_stride;
      std::vector<float> averaged(n_mass_old[i]);
      double total = 0.0;
      for (int64_t b = 0; b < n_mass_old[i]; ++b) {
        averaged[b] = row[b] / (float)num_layers;  // fp32 tensor / int
        total += (double)averaged[b];
      }
      if (total > 0.0)
        for (int64_t b = 0; b < n_mass_old[i]; ++b) dscores.push_back((double)averaged[b] / total);
    }
    // Score-free policy, or no positive mass: uniform over the blocks after the step.
    if (dscores.empty()) dscores.assign(n_blocks, 1.0 / (double)n_blocks);
    fscores.assign(dscores.size(), 0.f);
    for (size_t b = 0; b < dscores.size(); ++b) fscores[b] = (float)dscores[b];
    if (scores && so + (int64_t)dscores.size() <= scores_cap)
      std::copy(dscores.begin(), dscores.end(), scores + so);
    so += (int64_t)dscores.size();
    if (c) c[4] = (int64_t)dscores.size();
    if (!s.pager->on_step((uint64_t)(n_blocks - 1), fscores.data(), fscores.size()))
      return fail(kErrState, "attempt to calculate the remainder with a divisor of zero");
    if (added) s.pager->force_rebalance((uint64_t)(n_blocks - 1));
    tiers.assign(s.pager->num_blocks(), 0);
    s.pager->tiers(tiers.data());
    std::vector<int64_t> tg(n_blocks + 1), tc(n_blocks + 1);
    int64_t ng = 0, nc = 0, fb = -1;
    rc = apply_tiers(sid, tiers.data(), (int64_t)tiers.size(), tg.data(), &ng, tc.data(), &nc, &fb, stream);
    if (c) {
      c[1] = ng;
      c[2] = nc;
      c[3] = fb;
    }
    if (moves && mo + ng + nc <= moves_cap) {
      std::copy(tg.begin(), tg.begin() + ng, moves + mo);
      std::copy(tc.begin(), tc.begin() + nc, moves + mo + ng);
    }
    mo += ng + nc;
    if (rc != kOk) return rc;
  }
  return kOk;
}

int PagedKV::session_info(int sid, int64_t* n_tokens, int64_t* n_full, int64_t* gpu_blocks,
                          int64_t* cpu_blocks) const {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return kErrKey;
  const Session& s = sessions_[sid];
  const int64_t nf = s.n_tokens / cfg_.tokens_per_block;
  int64_t g = 0;
  for (int64_t b = 0; b < nf; ++b) g += s.on_gpu[b];
  *n_tokens = s.n_tokens;
  *n_full = nf;
  *gpu_blocks = g;
  *cpu_blocks = nf - g;
  return kOk;
}

int PagedKV::block_ids(int sid, int gpu, int64_t* out, int64_t cap) const {
  if (sid < 0 || sid >= (int)sessions_.size() || !sessions_[sid].live) return kErrKey;
  const Session& s = sessions_[sid];
  const int64_t nf = s.n_tokens / cfg_.tokens_per_block;
  int64_t c = 0;
  for (int64_t b = 0; b < nf; ++b)
    if ((s.on_gpu[b] != 0) == (gpu != 0)) {
      if (c < cap) out[c] = b;
      ++c;
    }
  return (int)c;
}

int PagedKV::step_host_blocks(int seq_index, int64_t* out, int64_t cap) const {
  if (seq_index < 0 || seq_index >= (int)step_host_ids_.size()) return kErrKey;
  const auto& v = step_host_ids_[seq_index];
  for (int64_t i = 0; i < (int64_t)v.size() && i < cap; ++i) out[i] = v[i];
  return (int)v.size();
}

HbmBytes PagedKV::hbm_bytes() const {
  HbmBytes h;
  const int64_t rec = (int64_t)rec_bytes();
  for (void* p : pool_)
    if (p) h.pool += rec * cfg_.pool_slots;
  for (void* p : ring_)
    if (p) h.mirror += rec * ring_records_;
  if (stage_) h.staging = rec * cfg_.staging_slots * cfg_.staging_buffers;
  h.workspace = (int64_t)ws_bytes_ + (int64_t)(mass_w_floats_ * sizeof(float)) +
                (bases_dev_ ? (int64_t)(2 * cfg_.num_layers * sizeof(void*)) : 0) +
                (mirror_flags_ ? (int64_t)(256 * sizeof(uint32_t)) : 0);
  h.total = h.pool + h.mirror + h.staging + h.workspace;
  return h;
}

int64_t PagedKV::resident_gpu_bytes() const { return gpu_bytes_; }
int64_t PagedKV::resident_cpu_bytes() const { return cpu_bytes_; }

StoreStats PagedKV::stats() {
  // Fold finished move timings into the seconds counters.
  std::vector<PendingTiming> keep;
  for (auto& t : move_timing_) {
    if (hipEventQuery(t.stop) == hipSuccess) {
      float ms = 0.f;
      hipEventElapsedTime(&ms, t.start, t.stop);
      if (t.bytes == 1)
        stats_.cpu_to_gpu_sec += ms / 1000.0;
      else
        stats_.gpu_to_cpu_sec += ms / 1000.0;
      hipEventDestroy(t.start);
      hipEventDestroy(t.stop);
    } else {
      keep.push_back(t);
    }
  }
  move_timing_.swap(keep);
  return stats_;
}

int PagedKV::resolve_timing() {
  for (auto& t : timing_pending_) {
    PGR_HIP(hipEventSynchronize(t.stop));
    float ms = 0.f;
    PGR_HIP(hipEventElapsedTime(&ms, t.start, t.stop));
    timing_ms_ += ms;
    timing_launches_ += 1;
    timing_bytes_ += t.bytes;
    timing_events_.push_back(t.start);
    timing_events_.push_back(t.stop);
  }
  timing_pending_.clear();
  return kOk;
}

// An event for launch timing: a resolved one from the pool, or a new one.
hipError_t PagedKV::timing_event(hipEvent_t* ev) {
  if (!timing_events_.empty()) {
    *ev = timing_events_.back();
    timing_events_.pop_back();
    return hipSuccess;
  }
  return hipEventCreateWithFlags(ev, hipEventDisableSystemFence);
}

int PagedKV::kernel_time(double* ms, int64_t* launches, int64_t* bytes) {
  int rc = resolve_timing();
  if (rc != kOk) return rc;
  *ms = timing_ms_;
  *launches = timing_launches_;
  *bytes = timing_bytes_;
  timing_ms_ = 0.0;
  timing_launches_ = 0;
  timing_bytes_ = 0;
  return kOk;
}

int PagedKV::copy_time(double* ms, int64_t* copies, int64_t* bytes) {
  if (in_step_) return fail(kErrState, "copy_time during a decode step");
  PGR_HIP(mirror_issuer_.wait());
  std::lock_guard<std::mutex> lk(copy_timing_mu_);
  double total = 0.0;
  int64_t b = 0;
  for (const PendingTiming& t : copy_timing_) {
    PGR_HIP(hipEventSynchronize(t.stop));
    float one = 0.f;
    PGR_HIP(hipEventElapsedTime(&one, t.start, t.stop));
    total += one;
    b += t.bytes;
  }
  *ms = total;
  *copies = (int64_t)copy_timing_.size();
  *bytes = b;
  for (const PendingTiming& t : copy_timing_) {
    hipEventDestroy(t.start);
    hipEventDestroy(t.stop);
  }
  copy_timing_.clear();
  return kOk;
}

int PagedKV::sync() {
  if (in_step_ && cfg_.stream_mode == 2) {
    // In an open step the mirror job may wait for releases that launches not yet made would
    // publish: wait until it has queued what it can.
    while (mirror_issuer_.busy() && !mirror_waiting_) std::this_thread::yield();
  } else {
    PGR_HIP(mirror_issuer_.wait());
  }
  PGR_HIP(hipStreamSynchronize(copy_stream_));
  PGR_HIP(hipDeviceSynchronize());
  forget_streams();
  return kOk;
}

}  // namespace pgr
