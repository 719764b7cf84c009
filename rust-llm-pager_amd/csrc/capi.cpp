// extern "C" entry points declared in include/pgr.h.
#include "../../include/pgr.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "paged_kv.h"
#include "pager_core.h"
#include "pgr_common.h"
#include "pgr_kernels.h"

// Split-K partials of pgr_attn_step_noalloc: a file-scope device array, one copy per GPU,
// held until the process ends. In host code `scratch` is a host-side stand-in, not a device
// address: the device address is looked up once per device (hipGetSymbolAddress with that
// device current, noalloc_device below) and only that address is used afterwards.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

thread_local std::string g_last_error;

int set_err(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_err(hipError_t e, const char* what) {
  return set_err(pgr::kErrHip, std::string(what) + ": " + hipGetErrorString(e));
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int check_dense(int64_t batch, int64_t hq, int64_t hkv, int64_t tokens, int64_t d, int dtype, float scale) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || tokens < 0 || d <= 0)
    return set_err(pgr::kErrInvalid, "negative or zero dimension");
  if (hq % hkv != 0) return set_err(pgr::kErrInvalid, "num_query_heads must be a multiple of num_kv_heads");
  if (hq / hkv > pgr::kMaxRep)
    return set_err(pgr::kErrUnsupported, "streaming attention's GQA query-head packing supports n_rep up to 16");
  if (!pgr::dense_head_dim_supported((int)d))
    return set_err(pgr::kErrUnsupported, "head_dim must be 8, 16, 32, 64, 128 or 256");
  if (dtype != pgr::kF16 && dtype != pgr::kBF16 && dtype != pgr::kF32)
    return set_err(pgr::kErrInvalid, "dtype must be fp16, bf16 or fp32");
  if (!(scale > 0.f) || !std::isfinite(scale)) return set_err(pgr::kErrInvalid, "scale must be positive and finite");
  if (batch > 65535 || hkv > 65535 || tokens > ((int64_t)1 << 30))
    return set_err(pgr::kErrInvalid, "shape exceeds the launch limits");
  return pgr::kOk;
}

struct DensePlan {
  int wave_tokens = 0, n_split = 0;
  size_t bytes = 0, o_pm = 0, o_pl = 0, o_pacc = 0;
};

DensePlan plan_dense(int64_t batch, int64_t hq, int64_t hkv, int64_t tokens, int64_t d, int mode, int64_t tpb,
                     int dtype) {
  DensePlan p;
  if (tokens <= 0 || batch <= 0) return p;
  const bool mass = mode == PGR_MODE_ACCUMULATE;
  p.wave_tokens =
      pgr::dense_wave_tokens(dtype, (int)d, (int)batch, (int)hkv, (int)tokens, (int)(mass ? tpb : 16), mass);
  const int64_t per_wg = (int64_t)pgr::dense_waves_per_workgroup(dtype, (int)d) * p.wave_tokens;
  p.n_split = (int)((tokens + per_wg - 1) / per_wg);
  const size_t slots = (size_t)batch * hkv * p.n_split;
  const size_t n_rep = (size_t)(hq / hkv);
  size_t off = 0;
  p.o_pm = off;
  off = pgr::align_up(off + slots * n_rep * sizeof(float), 256);
  p.o_pl = off;
  off = pgr::align_up(off + slots * n_rep * sizeof(float), 256);
  p.o_pacc = off;
  if (mode != PGR_MODE_STATS) off = pgr::align_up(off + slots * n_rep * d * sizeof(float), 256);
  p.bytes = off;
  return p;
}

// Launch timing of the operator API's attention kernel (pgr_attn_set_timing): fence-free
// events around each fold launch, resolved by pgr_attn_kernel_time. One process-wide list.
struct DenseTiming {
  hipEvent_t start, stop;
  int64_t bytes;
};
std::mutex g_timing_mu;
bool g_timing_on = false;
std::vector<DenseTiming> g_timing_pending;
std::vector<hipEvent_t> g_timing_free;

hipError_t timing_event(hipEvent_t* ev) {
  if (!g_timing_free.empty()) {
    *ev = g_timing_free.back();
    g_timing_free.pop_back();
    return hipSuccess;
  }
  return hipEventCreateWithFlags(ev, hipEventDisableSystemFence);
}

// The launch arguments of one operator call over its plan and workspace.
pgr::DenseLaunch dense_launch(const DensePlan& p, const void* q, const void* k, const void* v, const int32_t* valid,
                              const int32_t* active, float* m, float* l, float* acc, float* block_mass,
                              int64_t max_blocks, int64_t block_id_offset, int64_t tpb, int64_t batch, int64_t hq,
                              int64_t hkv, int64_t tokens, float scale, float softcap, void* ws) {
  char* w = static_cast<char*>(ws);
  pgr::DenseLaunch L{};
  L.q = q;
  L.k = k;
  L.v = v;
  L.valid = valid;
  L.active = active;
  L.m = m;
  L.l = l;
  L.acc = acc;
  L.block_mass = block_mass;
  L.pm = reinterpret_cast<float*>(w + p.o_pm);
  L.pl = reinterpret_cast<float*>(w + p.o_pl);
  L.pacc = reinterpret_cast<float*>(w + p.o_pacc);
  L.batch = (int)batch;
  L.hq = (int)hq;
  L.hkv = (int)hkv;
  L.tc = (int)tokens;
  L.wave_tokens = p.wave_tokens;
  L.n_split = p.n_split;
  L.tokens_per_block = (int)tpb;
  L.max_blocks = (int)max_blocks;
  L.block_id_offset = (int)block_id_offset;
  L.scale = scale;
  L.softcap = softcap > 0.f ? softcap : 0.f;
  return L;
}

int run_dense(int mode, const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active,
              float* m, float* l, float* acc, float* block_mass, int64_t max_blocks, int64_t block_id_offset,
              int64_t tpb, int64_t batch, int64_t hq, int64_t hkv, int64_t tokens, int64_t d, int dtype, float scale,
              float softcap, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_dense(batch, hq, hkv, tokens, d, dtype, scale);
  if (rc != pgr::kOk) return rc;
  if (mode == PGR_MODE_ACCUMULATE) {
    if (tpb <= 0 || tpb % 16 != 0) return set_err(pgr::kErrUnsupported, "tokens_per_block must be a multiple of 16");
    const int64_t nb = (tokens + tpb - 1) / tpb;
    if (block_id_offset < 0 || block_id_offset + nb > max_blocks)
      return set_err(pgr::kErrInvalid, "block_mass is too small for block_id_offset + this chunk's blocks");
    if (block_mass == nullptr) return set_err(pgr::kErrInvalid, "block_mass is null");
  }
  if (tokens == 0 || batch == 0) return pgr::kOk;  // nothing to fold: the state is unchanged
  if (!q || !k || !m || !l || (mode != PGR_MODE_STATS && (!v || !acc)))
    return set_err(pgr::kErrInvalid, "null tensor pointer");
  const DensePlan p = plan_dense(batch, hq, hkv, tokens, d, mode, tpb, dtype);
  if (ws == nullptr || ws_bytes < p.bytes) return set_err(pgr::kErrCapacity, "workspace too small");
  pgr::DenseLaunch L = dense_launch(p, q, k, v, valid, active, m, l, acc, block_mass, max_blocks, block_id_offset, tpb,
                                    batch, hq, hkv, tokens, scale, softcap, ws);
  std::unique_lock<std::mutex> lk(g_timing_mu);
  const bool timed = g_timing_on;
  if (timed) {
    hipError_t te = timing_event(&L.ev_start);
    if (te == hipSuccess) te = timing_event(&L.ev_stop);
    if (te != hipSuccess) return hip_err(te, "timing event");
  } else {
    lk.unlock();
  }
  hipError_t e = pgr::launch_dense(dtype, mode, (int)d, L, as_stream(stream));
  if (timed) {
    const int64_t elem = dtype == pgr::kF32 ? 4 : 2;
    const int64_t kv = batch * hkv * tokens * d * elem * (mode == PGR_MODE_STATS ? 1 : 2);
    g_timing_pending.push_back({L.ev_start, L.ev_stop, kv});
  }
  if (e != hipSuccess) return hip_err(e, "dense attention launch");
  return pgr::kOk;
}

// Per device, set up on the first call there: the device address of `scratch`, and the
// order of calls that share it. Outside graph capture a call whose stream differs from the
// previous call's makes its stream wait (on the GPU) for an event recorded after the
// previous call's launches, so calls from several streams or threads run one after another
// on the GPU, in the order they were made, instead of racing on the shared array.
constexpr int kMaxDevices = 64;
struct NoAllocDevice {
  std::once_flag once;
  hipError_t err = hipSuccess;
  const char* what = nullptr;
  void* scratch = nullptr;
  std::mutex mu;               // held over a call's launches and event record
  hipEvent_t done = nullptr;   // recorded after the previous call's launches
  hipStream_t last = nullptr;  // that call's stream
  bool have_last = false;
};
NoAllocDevice g_noalloc[kMaxDevices];

int noalloc_device(NoAllocDevice** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_err(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return set_err(pgr::kErrUnsupported, "device index beyond the scratch table");
  NoAllocDevice& d = g_noalloc[dev];
  std::call_once(d.once, [&d] {
    void* p = nullptr;
    d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    d.what = "hipGetSymbolAddress(scratch)";
    d.scratch = p;
    if (d.err == hipSuccess) {
      d.err = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
      d.what = "hipEventCreateWithFlags";
    }
  });
  if (d.err != hipSuccess) return hip_err(d.err, d.what);
  *out = &d;
  return pgr::kOk;
}

// Status for an exception caught at the C boundary (called inside a catch block): none may
// cross into a C caller, not even one thrown while recording the message.
int exception_status() noexcept {
  int code = pgr::kErrInternal;
  const char* what = nullptr;
  try {
    throw;
  } catch (const std::bad_alloc&) {
    code = pgr::kErrCapacity;
  } catch (const std::exception& e) {
    what = e.what();  // the exception lives until the caller's catch block ends
  } catch (...) {
  }
  try {
    if (code == pgr::kErrCapacity)
      g_last_error = "out of host memory";
    else
      g_last_error = std::string("internal error") + (what ? std::string(": ") + what : std::string());
  } catch (...) {
    g_last_error.clear();
  }
  return code;
}

pgr::PagedKV* kv_of(void* h) { return static_cast<pgr::PagedKV*>(h); }

int kv_rc(pgr::PagedKV* kv, int rc) {
  if (rc != pgr::kOk) g_last_error = kv->error();
  return rc;
}

}  // namespace

extern "C" {

int pgr_abi_version(void) { return 10; }

const char* pgr_last_error(void) { return g_last_error.c_str(); }

size_t pgr_attn_workspace_bytes(int64_t batch, int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens,
                                int64_t head_dim, int mode, int64_t tokens_per_block) {
  try {
    if (batch <= 0 || num_kv_heads <= 0 || num_query_heads <= 0 || tokens <= 0 || head_dim <= 0) return 0;
    if (mode == PGR_MODE_ACCUMULATE && (tokens_per_block <= 0 || tokens_per_block % 16 != 0)) return 0;
    // The geometry depends on the element type only at head dims 32/64/128 (16-bit there runs the
    // MFMA kernel, fp32 the generic one): the size covers both.
    const size_t a = plan_dense(batch, num_query_heads, num_kv_heads, tokens, head_dim, mode, tokens_per_block,
                                pgr::kF16).bytes;
    const size_t b = plan_dense(batch, num_query_heads, num_kv_heads, tokens, head_dim, mode, tokens_per_block,
                                pgr::kF32).bytes;
    return a > b ? a : b;
  } catch (...) {
    exception_status();
    return 0;
  }
}

int pgr_attn_step(const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active, float* m,
                  float* l, float* acc, int64_t batch, int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens,
                  int64_t head_dim, int dtype, float scale, float softcap, void* workspace, size_t workspace_bytes,
                  void* stream) {
  try {
    return run_dense(PGR_MODE_FOLD, q, k, v, valid, active, m, l, acc, nullptr, 0, 0, 16, batch, num_query_heads,
                     num_kv_heads, tokens, head_dim, dtype, scale, softcap, workspace, workspace_bytes, stream);
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_bench_step(const void* q, const void* const* k, const void* const* v, int32_t n_chunks, int64_t batch,
                        int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens, int64_t head_dim, int dtype,
                        float scale, void* workspace, size_t workspace_bytes, int32_t reps, double* us_per_launch,
                        int64_t* bytes_per_launch, void* stream) {
  try {
    int rc = check_dense(batch, num_query_heads, num_kv_heads, tokens, head_dim, dtype, scale);
    if (rc != pgr::kOk) return rc;
    if (!q || !k || !v || n_chunks <= 0 || reps <= 0 || !us_per_launch || !bytes_per_launch || tokens <= 0 ||
        batch <= 0)
      return set_err(pgr::kErrInvalid, "pgr_attn_bench_step: inputs, chunks > 0, reps > 0 and outputs required");
    for (int c = 0; c < n_chunks; ++c)
      if (!k[c] || !v[c]) return set_err(pgr::kErrInvalid, "pgr_attn_bench_step: a null chunk");
    const DensePlan p = plan_dense(batch, num_query_heads, num_kv_heads, tokens, head_dim, PGR_MODE_FOLD, 16, dtype);
    if (workspace == nullptr || workspace_bytes < p.bytes) return set_err(pgr::kErrCapacity, "workspace too small");
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) e = hipEventCreateWithFlags(&ev[i], hipEventDisableSystemFence);
    if (e == hipSuccess) e = hipEventRecord(ev[0], as_stream(stream));
    for (int r = 0; r < reps && e == hipSuccess; ++r)
      for (int c = 0; c < n_chunks && e == hipSuccess; ++c) {
        // The fold launch reads no running state (only the merge does), so none is passed.
        pgr::DenseLaunch L = dense_launch(p, q, k[c], v[c], nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0,
                                          16, batch, num_query_heads, num_kv_heads, tokens, scale, 0.f, workspace);
        L.attention_only = true;
        e = pgr::launch_dense(dtype, PGR_MODE_FOLD, (int)head_dim, L, as_stream(stream));
      }
    if (e == hipSuccess) e = hipEventRecord(ev[1], as_stream(stream));
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
    for (hipEvent_t x : ev)
      if (x) (void)hipEventDestroy(x);
    if (e != hipSuccess) return hip_err(e, "pgr_attn_bench_step");
    *us_per_launch = (double)ms * 1e3 / ((double)reps * n_chunks);
    const int64_t elem = dtype == pgr::kF32 ? 4 : 2;
    *bytes_per_launch = batch * num_kv_heads * tokens * head_dim * elem * 2;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_step_noalloc(const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active,
                          float* m, float* l, float* acc, int64_t batch, int64_t num_query_heads,
                          int64_t num_kv_heads, int64_t tokens, int64_t head_dim, int dtype, float scale,
                          float softcap, void* stream) {
  try {
    int rc = check_dense(batch, num_query_heads, num_kv_heads, tokens, head_dim, dtype, scale);
    if (rc != pgr::kOk) return rc;
    if (tokens == 0 || batch == 0) return pgr::kOk;
    // Every partial slot that the merge reads is written by the fold launch before it (a row
    // with active = 0 is skipped by both), so nothing left in `scratch` by an earlier call is
    // read and nothing needs clearing.
    const size_t need =
        plan_dense(batch, num_query_heads, num_kv_heads, tokens, head_dim, PGR_MODE_FOLD, 16, dtype).bytes;
    if (need > kNoAllocScratchBytes)
      return set_err(pgr::kErrCapacity, "pgr_attn_step_noalloc: this chunk needs " + std::to_string(need) +
                                            " bytes of split-K partials, more than the " +
                                            std::to_string(kNoAllocScratchBytes) +
                                            "-byte static scratch; use pgr_attn_step with a workspace");
    NoAllocDevice* dev = nullptr;
    rc = noalloc_device(&dev);
    if (rc != pgr::kOk) return rc;
    const hipStream_t s = as_stream(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &cap);
    if (e != hipSuccess) return hip_err(e, "hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone)  // captured calls: the caller orders the replays
      return run_dense(PGR_MODE_FOLD, q, k, v, valid, active, m, l, acc, nullptr, 0, 0, 16, batch, num_query_heads,
                       num_kv_heads, tokens, head_dim, dtype, scale, softcap, dev->scratch, kNoAllocScratchBytes,
                       stream);
    std::lock_guard<std::mutex> lock(dev->mu);
    if (dev->have_last && dev->last != s) {
      e = hipStreamWaitEvent(s, dev->done, 0);
      if (e != hipSuccess) return hip_err(e, "hipStreamWaitEvent (previous call on another stream)");
    }
    rc = run_dense(PGR_MODE_FOLD, q, k, v, valid, active, m, l, acc, nullptr, 0, 0, 16, batch, num_query_heads,
                   num_kv_heads, tokens, head_dim, dtype, scale, softcap, dev->scratch, kNoAllocScratchBytes, stream);
    if (rc != pgr::kOk) return rc;
    e = hipEventRecord(dev->done, s);
    if (e != hipSuccess) return hip_err(e, "hipEventRecord (call order)");
    dev->last = s;
    dev->have_last = true;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_stats_step(const void* q, const void* k, const int32_t* valid, const int32_t* active, float* m, float* l,
                        int64_t batch, int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens, int64_t head_dim,
                        int dtype, float scale, float softcap, void* workspace, size_t workspace_bytes, void* stream) {
  try {
    return run_dense(PGR_MODE_STATS, q, k, nullptr, valid, active, m, l, nullptr, nullptr, 0, 0, 16, batch,
                     num_query_heads, num_kv_heads, tokens, head_dim, dtype, scale, softcap, workspace, workspace_bytes,
                     stream);
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_accumulate_step(const void* q, const void* k, const void* v, const int32_t* valid, const int32_t* active,
                             const float* m, const float* l, float* acc, float* block_mass, int64_t max_blocks,
                             int64_t block_id_offset, int64_t tokens_per_block, int64_t batch,
                             int64_t num_query_heads, int64_t num_kv_heads, int64_t tokens, int64_t head_dim,
                             int dtype, float scale, float softcap, void* workspace, size_t workspace_bytes,
                             void* stream) {
  try {
    return run_dense(PGR_MODE_ACCUMULATE, q, k, v, valid, active, const_cast<float*>(m), const_cast<float*>(l), acc,
                     block_mass, max_blocks, block_id_offset, tokens_per_block, batch, num_query_heads, num_kv_heads,
                     tokens, head_dim, dtype, scale, softcap, workspace, workspace_bytes, stream);
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_fold_fixed_step(const void* q, const void* k, const void* v, const int32_t* valid, const float* m,
                             const float* l, float* acc, int64_t batch, int64_t num_query_heads, int64_t num_kv_heads,
                             int64_t tokens, int64_t head_dim, int dtype, float scale, float softcap, void* workspace,
                             size_t workspace_bytes, void* stream) {
  try {
    return run_dense(PGR_MODE_FOLD_FIXED, q, k, v, valid, nullptr, const_cast<float*>(m), const_cast<float*>(l), acc,
                     nullptr, 0, 0, 16, batch, num_query_heads, num_kv_heads, tokens, head_dim, dtype, scale, softcap,
                     workspace, workspace_bytes, stream);
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_set_timing(int32_t on) {
  try {
    std::lock_guard<std::mutex> lk(g_timing_mu);
    g_timing_on = on != 0;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_kernel_time(double* ms, int64_t* launches, int64_t* bytes) {
  try {
    if (!ms || !launches || !bytes) return set_err(pgr::kErrInvalid, "null pointer");
    std::lock_guard<std::mutex> lk(g_timing_mu);
    double total = 0.0;
    int64_t n = 0, b = 0;
    for (const DenseTiming& t : g_timing_pending) {
      hipError_t e = hipEventSynchronize(t.stop);
      float one = 0.f;
      if (e == hipSuccess) e = hipEventElapsedTime(&one, t.start, t.stop);
      if (e != hipSuccess) return hip_err(e, "timing event");
      total += one;
      ++n;
      b += t.bytes;
      g_timing_free.push_back(t.start);
      g_timing_free.push_back(t.stop);
    }
    g_timing_pending.clear();
    *ms = total;
    *launches = n;
    *bytes = b;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_bench_stream_read(const void* const* srcs, int32_t n_src, int64_t bytes, int32_t workgroups, int32_t reps,
                          double* us_per_launch, void* stream) {
  try {
    if (!srcs || n_src <= 0 || reps <= 0 || !us_per_launch || bytes <= 0 || bytes % 16 != 0 || workgroups <= 0)
      return set_err(pgr::kErrInvalid, "need buffers, reps > 0 and bytes a positive multiple of 16");
    for (int i = 0; i < n_src; ++i)
      if (!srcs[i] || ((uintptr_t)srcs[i]) % 16 != 0) return set_err(pgr::kErrInvalid, "buffers must be 16-byte aligned");
    std::vector<hipEvent_t> ev(2 * (size_t)reps, nullptr);
    hipError_t e = hipSuccess;
    for (size_t i = 0; i < ev.size() && e == hipSuccess; ++i) e = hipEventCreateWithFlags(&ev[i], hipEventDisableSystemFence);
    for (int r = 0; r < reps && e == hipSuccess; ++r) {
      e = hipEventRecord(ev[2 * r], as_stream(stream));
      if (e == hipSuccess) e = pgr::launch_stream_read(srcs[r % n_src], bytes, workgroups, as_stream(stream));
      if (e == hipSuccess) e = hipEventRecord(ev[2 * r + 1], as_stream(stream));
    }
    double total = 0.0;
    for (int r = 0; r < reps && e == hipSuccess; ++r) {
      float ms = 0.f;
      e = hipEventSynchronize(ev[2 * r + 1]);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]);
      total += ms;
    }
    for (hipEvent_t x : ev)
      if (x) (void)hipEventDestroy(x);
    if (e != hipSuccess) return hip_err(e, "stream read");
    *us_per_launch = total * 1e3 / reps;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_state_init(float* m, float* l, float* acc, int64_t rows, int64_t head_dim, void* stream) {
  try {
    if (rows < 0 || head_dim <= 0) return set_err(pgr::kErrInvalid, "negative or zero dimension");
    if (rows > ((int64_t)1 << 40) / head_dim) return set_err(pgr::kErrInvalid, "state too large");
    if (rows == 0) return pgr::kOk;
    if (!m || !l || !acc) return set_err(pgr::kErrInvalid, "null tensor pointer");
    hipError_t e = pgr::launch_state_init(m, l, acc, rows, head_dim, as_stream(stream));
    if (e != hipSuccess) return hip_err(e, "state init launch");
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_attn_finalize(const float* acc, const float* l, void* out, int64_t rows, int64_t head_dim, int dtype,
                      void* stream) {
  try {
    if (rows < 0 || head_dim <= 0) return set_err(pgr::kErrInvalid, "negative or zero dimension");
    if (dtype != pgr::kF16 && dtype != pgr::kBF16 && dtype != PGR_DTYPE_F32)
      return set_err(pgr::kErrInvalid, "dtype must be fp16, bf16 or fp32");
    if (rows == 0) return pgr::kOk;
    if (!acc || !l || !out) return set_err(pgr::kErrInvalid, "null tensor pointer");
    hipError_t e = pgr::launch_finalize(dtype, acc, l, out, (int)rows, (int)head_dim, as_stream(stream));
    if (e != hipSuccess) return hip_err(e, "finalize launch");
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

// ---- placement -----------------------------------------------------------------------

void* pgr_pager_new(uint64_t vram, uint64_t ram, uint64_t recent, uint64_t rebalance_interval, float promote_margin,
                    float ram_promote_margin, const char* policy) {
  try {
    const std::string name = policy ? policy : "heavy_hitter";
    return new (std::nothrow) pgr::PlacementPager(vram, ram, recent, rebalance_interval, promote_margin,
                                                  ram_promote_margin, pgr::policy_from_name(name));
  } catch (...) {
    exception_status();
    return nullptr;
  }
}

void pgr_pager_free(void* pager) { delete static_cast<pgr::PlacementPager*>(pager); }

int pgr_pager_on_step(void* pager, uint64_t token_idx, uint32_t layer, const float* attention, size_t n) {
  try {
    (void)layer;
    if (!pager || (n && !attention)) return set_err(pgr::kErrInvalid, "null pointer");
    if (n > ((size_t)1 << 31)) return set_err(pgr::kErrInvalid, "attention vector too long");
    if (!static_cast<pgr::PlacementPager*>(pager)->on_step(token_idx, attention, n))
      return set_err(pgr::kErrState, "attempt to calculate the remainder with a divisor of zero");
    return pgr::kOk;
  } catch (...) {
    exception_status();
  }
}

int pgr_pager_force_rebalance(void* pager, uint64_t token_idx) {
  try {
    if (!pager) return set_err(pgr::kErrInvalid, "null pager");
    if (token_idx >= ((uint64_t)1 << 31)) return set_err(pgr::kErrInvalid, "token_idx too large for the block table");
    static_cast<pgr::PlacementPager*>(pager)->force_rebalance(token_idx);
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

size_t pgr_pager_num_blocks(void* pager) { return pager ? static_cast<pgr::PlacementPager*>(pager)->num_blocks() : 0; }

size_t pgr_pager_tiers(void* pager, uint8_t* out, size_t cap) {
  try {
    if (!pager) return 0;
    auto* p = static_cast<pgr::PlacementPager*>(pager);
    const size_t n = p->num_blocks();
    if (out && cap >= n) p->tiers(out);
    return n;
  } catch (...) {
    exception_status();
    return 0;
  }
}

size_t pgr_pager_vram_block_ids(void* pager, uint64_t* out, size_t cap) {
  try {
    if (!pager) return 0;
    auto* p = static_cast<pgr::PlacementPager*>(pager);
    const size_t n = p->vram_count();
    if (out && cap >= n) p->vram_block_ids(out);
    return n;
  } catch (...) {
    exception_status();
    return 0;
  }
}

int pgr_pager_metrics(void* pager, pgr_pager_metrics_t* out) {
  try {
    if (!pager || !out) return set_err(pgr::kErrInvalid, "null pointer");
    const pgr::PagerMetrics& m = static_cast<pgr::PlacementPager*>(pager)->metrics();
    out->tokens = m.tokens;
    out->vram_peak = m.vram_peak;
    out->ram_peak = m.ram_peak;
    out->swap_vram_ram = m.swap_vram_ram;
    out->swap_ram_ssd = m.swap_ram_ssd;
    out->attention_mass_total = m.attention_mass_total;
    out->attention_mass_vram = m.attention_mass_vram;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

// ---- paged KV store -------------------------------------------------------------------

void* pgr_kv_create(const pgr_kv_config_t* c) {
  try {
    if (!c) {
      set_err(pgr::kErrInvalid, "null config");
      return nullptr;
    }
    pgr::PagedKVConfig cfg;
    cfg.num_layers = c->num_layers;
    cfg.kv_heads = c->kv_heads;
    cfg.query_heads = c->query_heads;
    cfg.head_dim = c->head_dim;
    cfg.tokens_per_block = c->tokens_per_block;
    cfg.dtype = c->dtype;
    cfg.pool_slots = c->pool_slots;
    cfg.host_records = c->host_records;
    cfg.staging_slots = c->staging_slots;
    cfg.staging_buffers = c->staging_buffers;
    cfg.blocks_per_workgroup = c->blocks_per_workgroup > 0 ? c->blocks_per_workgroup : 32;
    cfg.target_workgroups = c->target_workgroups > 0 ? c->target_workgroups : 0;
    cfg.stream_mode = c->stream_mode;
    auto* kv = new (std::nothrow) pgr::PagedKV(cfg);
    if (!kv) {
      set_err(pgr::kErrCapacity, "out of host memory");
      return nullptr;
    }
    const int rc = kv->init();
    if (rc != pgr::kOk) {
      g_last_error = kv->error();
      delete kv;
      return nullptr;
    }
    return kv;
  } catch (...) {
    exception_status();
    return nullptr;
  }
}

void pgr_kv_destroy(void* kv) { delete kv_of(kv); }

int pgr_kv_add_session(void* kv, int32_t rows, int64_t capacity_tokens, const int32_t* lo_per_row) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    return kv_rc(kv_of(kv), kv_of(kv)->add_session(rows, capacity_tokens, lo_per_row));
  } catch (...) {
    exception_status();
  }
}

int pgr_kv_remove_session(void* kv, int32_t sid) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    return kv_rc(kv_of(kv), kv_of(kv)->remove_session(sid));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_set_lo(void* kv, int32_t sid, const int32_t* lo_per_row) {
  try {
    if (!kv || !lo_per_row) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->set_lo(sid, lo_per_row));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_reorder_rows(void* kv, int32_t sid, const int32_t* src_rows, int32_t n_rows, void* stream) {
  try {
    if (!kv || !src_rows) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->reorder_rows(sid, src_rows, n_rows, as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_set_length(void* kv, int32_t sid, int64_t n_tokens) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    return kv_rc(kv_of(kv), kv_of(kv)->set_length(sid, n_tokens));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_import(void* kv, int32_t sid, int32_t row, int32_t layer, const void* k, const void* v, int64_t n_src,
                  int64_t n_tokens, void* stream) {
  try {
    if (!kv || !k || !v) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->import_tokens(sid, row, layer, k, v, n_src, n_tokens, as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_export(void* kv, int32_t sid, int32_t row, int32_t layer, void* k, void* v, int64_t n_tokens,
                  void* stream) {
  try {
    if (!kv || !k || !v) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->export_tokens(sid, row, layer, k, v, n_tokens, as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_put_block(void* kv, int32_t sid, int64_t block_id, const void* key, const void* value, void* stream) {
  try {
    if (!kv || !key || !value) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->put_block(sid, block_id, key, value, as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_get_block(void* kv, int32_t sid, int64_t block_id, void* key, void* value, void* stream) {
  try {
    if (!kv || !key || !value) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->get_block(sid, block_id, key, value, as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_apply_tiers(void* kv, int32_t sid, const uint8_t* tiers, int64_t n_tiers, int64_t* to_gpu, int64_t* n_gpu,
                       int64_t* to_cpu, int64_t* n_cpu, int64_t* fail_block, void* stream) {
  try {
    if (!kv || (n_tiers && !tiers) || !to_gpu || !n_gpu || !to_cpu || !n_cpu || !fail_block)
      return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->apply_tiers(sid, tiers, n_tiers, to_gpu, n_gpu, to_cpu, n_cpu, fail_block,
                                                   as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_set_ram_budget(void* kv, int64_t bytes) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    kv_of(kv)->set_ram_budget(bytes);
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_begin_step(void* kv, const int32_t* sids, int32_t n, void* stream) {
  try {
    if (!kv || (n && !sids) || n < 0) return set_err(pgr::kErrInvalid, "null pointer or negative count");
    return kv_rc(kv_of(kv), kv_of(kv)->begin_step(sids, n, as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_decode_layer(void* kv, int32_t layer, const void* q, const void* k_new, const void* v_new, void* out,
                        float* mass_accum, int64_t accum_stride, float scale, float softcap, int32_t window,
                        void* stream) {
  try {
    if (!kv || !q || !k_new || !v_new || !out) return set_err(pgr::kErrInvalid, "null pointer");
    if (!(scale > 0.f) || !std::isfinite(scale)) return set_err(pgr::kErrInvalid, "scale must be positive and finite");
    return kv_rc(kv_of(kv), kv_of(kv)->decode_layer(layer, q, k_new, v_new, out, mass_accum, accum_stride, scale,
                                                    softcap > 0.f ? softcap : 0.f, window > 0 ? window : 0,
                                                    as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_step_signature(void* kv, int64_t* out, int64_t cap) {
  try {
    if (!kv || (cap && !out)) return set_err(pgr::kErrInvalid, "null pointer");
    const int rc = kv_of(kv)->step_signature(out, cap);
    if (rc < 0) return set_err(rc, "step_signature outside a decode step");
    return rc;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_step_replayed(void* kv, void* stream) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    return kv_rc(kv_of(kv), kv_of(kv)->step_replayed(as_stream(stream)));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_end_step(void* kv, int32_t* completed, int32_t* n_completed) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    int c = 0;
    const int rc = kv_of(kv)->end_step(completed, &c);
    if (n_completed) *n_completed = c;
    return kv_rc(kv_of(kv), rc);
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_attach_pager(void* kv, int32_t sid, void* pager, int32_t scores_from_mass) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    return kv_rc(kv_of(kv), kv_of(kv)->attach_pager(sid, static_cast<pgr::PlacementPager*>(pager), scores_from_mass));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_end_step_place(void* kv, float* mass_accum, int64_t accum_stride, int32_t num_layers,
                          int32_t* completed, int32_t* n_completed, int64_t* counts, int64_t* moves,
                          int64_t moves_cap, double* scores, int64_t scores_cap, void* stream) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    if (num_layers <= 0) return set_err(pgr::kErrInvalid, "num_layers must be positive");
    int c = 0;
    const int rc = kv_of(kv)->end_step_place(mass_accum, accum_stride, num_layers, as_stream(stream), completed, &c,
                                             counts, moves, moves_cap, scores, scores_cap);
    if (n_completed) *n_completed = c;
    return kv_rc(kv_of(kv), rc);
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_session_info(void* kv, int32_t sid, int64_t* info) {
  try {
    if (!kv || !info) return set_err(pgr::kErrInvalid, "null pointer");
    const int rc = kv_of(kv)->session_info(sid, &info[0], &info[1], &info[2], &info[3]);
    if (rc != pgr::kOk) return set_err(rc, "unknown session");
    return rc;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_block_ids(void* kv, int32_t sid, int32_t gpu, int64_t* out, int64_t cap) {
  try {
    if (!kv || (cap && !out)) return set_err(pgr::kErrInvalid, "null pointer");
    const int rc = kv_of(kv)->block_ids(sid, gpu, out, cap);
    if (rc < 0) return set_err(rc, "unknown session");
    return rc;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_step_host_blocks(void* kv, int32_t seq, int64_t* out, int64_t cap) {
  try {
    if (!kv || (cap && !out)) return set_err(pgr::kErrInvalid, "null pointer");
    const int rc = kv_of(kv)->step_host_blocks(seq, out, cap);
    if (rc < 0) return set_err(rc, "no such sequence in the last step");
    return rc;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_step_stats(void* kv, pgr_kv_step_stats_t* out) {
  try {
    if (!kv || !out) return set_err(pgr::kErrInvalid, "null pointer");
    const pgr::StepStats& s = kv_of(kv)->step_stats();
    out->resident_tokens = s.resident_tokens;
    out->host_tokens = s.host_tokens;
    out->host_blocks = s.host_blocks;
    out->copies = s.copies;
    out->chunks = s.chunks;
    out->launches = s.launches;
    out->work_items = s.work_items;
    out->gather_blocks = s.gather_blocks;
    out->plan_wait_ns = s.plan_wait_ns;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_stats(void* kv, pgr_kv_stats_t* out) {
  try {
    if (!kv || !out) return set_err(pgr::kErrInvalid, "null pointer");
    const pgr::StoreStats s = kv_of(kv)->stats();
    out->gpu_to_cpu_bytes = s.gpu_to_cpu_bytes;
    out->cpu_to_gpu_bytes = s.cpu_to_gpu_bytes;
    out->gpu_to_cpu_copies = s.gpu_to_cpu_copies;
    out->cpu_to_gpu_copies = s.cpu_to_gpu_copies;
    out->gpu_to_cpu_sec = s.gpu_to_cpu_sec;
    out->cpu_to_gpu_sec = s.cpu_to_gpu_sec;
    out->evict_bytes_copied = s.evict_bytes_copied;
    out->load_bytes_copied = s.load_bytes_copied;
    out->stream_bytes = s.stream_bytes;
    out->stream_copies = s.stream_copies;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_resident_bytes(void* kv, int64_t* gpu, int64_t* cpu) {
  try {
    if (!kv || !gpu || !cpu) return set_err(pgr::kErrInvalid, "null pointer");
    *gpu = kv_of(kv)->resident_gpu_bytes();
    *cpu = kv_of(kv)->resident_cpu_bytes();
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_hbm_bytes(void* kv, int64_t* out) {
  try {
    if (!kv || !out) return set_err(pgr::kErrInvalid, "null pointer");
    const pgr::HbmBytes h = kv_of(kv)->hbm_bytes();
    out[0] = h.pool;
    out[1] = h.mirror;
    out[2] = h.staging;
    out[3] = h.workspace;
    out[4] = h.total;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_block_bytes(void* kv, int32_t sid, int64_t* bytes) {
  try {
    if (!kv || !bytes) return set_err(pgr::kErrInvalid, "null pointer");
    int64_t info[4];
    if (kv_of(kv)->session_info(sid, &info[0], &info[1], &info[2], &info[3]) != pgr::kOk)
      return set_err(pgr::kErrKey, "unknown session");
    *bytes = kv_of(kv)->block_bytes_all_layers(sid);
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_set_timing(void* kv, int32_t on) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    kv_of(kv)->set_timing(on != 0);
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_kernel_time(void* kv, double* ms, int64_t* launches, int64_t* bytes) {
  try {
    if (!kv || !ms || !launches || !bytes) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->kernel_time(ms, launches, bytes));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_bench_attention(void* kv, const void* const* q, const void* const* k_new, const void* const* v_new,
                           float scale, float softcap, int32_t reps, double* us_per_launch, int64_t* bytes_per_launch,
                           void* stream) {
  try {
    if (!kv || !q || !k_new || !v_new || !us_per_launch || !bytes_per_launch)
      return set_err(pgr::kErrInvalid, "null pointer");
    if (!(scale > 0.f) || !std::isfinite(scale)) return set_err(pgr::kErrInvalid, "scale must be positive and finite");
    return kv_rc(kv_of(kv), kv_of(kv)->bench_attention(q, k_new, v_new, scale, softcap > 0.f ? softcap : 0.f, reps,
                                                       as_stream(stream), us_per_launch, bytes_per_launch));
  } catch (...) {
    return exception_status();
  }
}

int pgr_bench_stream_read_back_to_back(const void* const* srcs, int32_t n_src, int64_t bytes, int32_t workgroups,
                                       int32_t reps, double* us_per_launch, void* stream) {
  try {
    if (!srcs || n_src <= 0 || reps <= 0 || !us_per_launch || bytes <= 0 || bytes % 16 != 0 || workgroups <= 0)
      return set_err(pgr::kErrInvalid, "need buffers, reps > 0 and bytes a positive multiple of 16");
    for (int i = 0; i < n_src; ++i)
      if (!srcs[i] || ((uintptr_t)srcs[i]) % 16 != 0) return set_err(pgr::kErrInvalid, "buffers must be 16-byte aligned");
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) e = hipEventCreateWithFlags(&ev[i], hipEventDisableSystemFence);
    if (e == hipSuccess) e = hipEventRecord(ev[0], as_stream(stream));
    for (int r = 0; r < reps && e == hipSuccess; ++r)
      e = pgr::launch_stream_read(srcs[r % n_src], bytes, workgroups, as_stream(stream));
    if (e == hipSuccess) e = hipEventRecord(ev[1], as_stream(stream));
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
    for (hipEvent_t x : ev)
      if (x) (void)hipEventDestroy(x);
    if (e != hipSuccess) return hip_err(e, "stream read");
    *us_per_launch = (double)ms * 1e3 / reps;
    return pgr::kOk;
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_copy_time(void* kv, double* ms, int64_t* copies, int64_t* bytes) {
  try {
    if (!kv || !ms || !copies || !bytes) return set_err(pgr::kErrInvalid, "null pointer");
    return kv_rc(kv_of(kv), kv_of(kv)->copy_time(ms, copies, bytes));
  } catch (...) {
    return exception_status();
  }
}

int pgr_kv_sync(void* kv) {
  try {
    if (!kv) return set_err(pgr::kErrInvalid, "null store");
    return kv_rc(kv_of(kv), kv_of(kv)->sync());
  } catch (...) {
    return exception_status();
  }
}

}  // extern "C"
