// Host-side launchers of the HIP kernels (implemented in attn_kernels.hip, kv_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "pgr_common.h"

namespace pgr {

// V layout inside a record. K is stored row by row, [Hkv][T][D]. V is stored in 16-token tiles,
// [Hkv][T/16][16 * D], and inside a tile in groups of four tokens transposed: element (token r
// of the tile, dim d) sits at vt_index(r, d, D). With DN = D / 16, the run of 4 * DN elements at
// ((r / 4) * 16 + n) * 4 * DN holds tokens 4(r/4)..4(r/4)+3 of dims DN*n .. DN*n + DN - 1, four
// tokens per dim: exactly the V^T operands of the MFMA tiles that decode-kernel lane
// (g = r / 4, n) feeds, so that lane loads one contiguous run (D/2 bytes, the size of its K run)
// and uses it as it arrives. D is a multiple of 16.
__host__ __device__ __forceinline__ int vt_index(int r, int d, int D) {
  const int dn = D / 16;
  return (((r >> 2) * 16 + d / dn) * dn + d % dn) * 4 + (r & 3);
}

// Element offset of V (head h, token t of the block, dim d) from the start of the record's V
// region (T tokens per block).
__host__ __device__ __forceinline__ size_t v_record_index(int h, int t, int d, int T, int D) {
  return ((size_t)h * T + (size_t)(t & ~15)) * D + (size_t)vt_index(t & 15, d, D);
}

struct DenseLaunch {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* valid;
  const int32_t* active;
  float* m;
  float* l;
  float* acc;
  float* block_mass;
  float* pm;
  float* pl;
  float* pacc;
  int batch, hq, hkv, tc;
  int wave_tokens, n_split;
  int tokens_per_block, max_blocks, block_id_offset;
  float scale, softcap;
  // Optional timing events recorded right before and after the attention launch (not the
  // merge): the fold kernel's own duration for measurement.
  hipEvent_t ev_start = nullptr;
  hipEvent_t ev_stop = nullptr;
  // Measurement only: launch the attention kernel and not the merge (m, l, acc untouched).
  bool attention_only = false;
};

// The paged decode kernels of one layer. launch_paged folds work items [work, work + n_work)
// into partial slots (and the work item that carries an append target writes the current
// token's K/V into the pool); launch_paged_merge then combines each sequence's partials
// with the current token (k_new/v_new) into out and the final (mf, lf).
struct PagedLaunch {
  // Merge launch: sequence s's split-K partials are slots s * partial_stride ..
  // s * partial_stride + partial_stride - 1 (the first SeqInfo::partial_count of them
  // written), or, with partial_stride 0, SeqInfo::partial_count slots from partial_base.
  int partial_stride = 0;
  const void* q;
  const void* k_new;
  const void* v_new;
  void* pool;
  const void* stage;
  const WorkItem* work;
  // The step's first launch (direct mode) reads `work` from the pinned plan buffer and copies
  // it to work_out, and the aux_vec 16-byte vectors at aux_src (the rest of the plan) to
  // aux_dst, for the kernels after it. Null / 0 otherwise.
  WorkItem* work_out = nullptr;
  const void* aux_src = nullptr;
  void* aux_dst = nullptr;
  int64_t aux_vec = 0;
  const SeqInfo* seqs;
  float* pm;
  float* pl;
  float* pacc;
  float* mass_m;
  float* mass_s;
  void* out;
  float* mf;
  float* lf;
  int n_work, hq, hkv, tokens_per_block, mass_stride;
  float scale, softcap;
  int window = 0;  // > 0: the layer's own sliding window (positions <= current - window masked)
  // Mirror mode: the layer's HBM mirror of `stage` (the host mirror) and its "filled" word.
  const void* mirror = nullptr;
  const uint32_t* mirror_flag = nullptr;
  // Merge launch only: when set, the merge stores plan_token to *plan_flag (pinned host memory)
  // as it starts, telling the host that the attention launches before it, and so their read of
  // the step's plan buffer, have finished.
  uint32_t* plan_flag = nullptr;
  uint32_t plan_token = 0;
  // Merge launch, mirror mode: the merge stores the step's token (SeqInfo::step_token) to
  // *release_flag (pinned host memory) as it starts: the layer's attention launches, the
  // readers of its ring buffer, have finished.
  uint32_t* release_flag = nullptr;
  // Merge launch, deferred mass: the merge writes s_b * 2^(m_b - m_final) / l_final of every
  // in-scope block of its (sequence, query head) to mass_w[(seq * Hq + head) * mass_stride + b]
  // instead of a mass_reduce launch per layer.
  float* mass_w = nullptr;
};

// Head dims of the MFMA dense kernel (32, 64, 128).
bool head_dim_supported(int d);
// Head dims of the paged decode kernels: 16, 32, 64, 128, 256.
bool paged_head_dim_supported(int d);
// Head dims of the dense operator kernels: 8, 16, 32, 64, 128, 256 (fp16, bf16 or fp32).
bool dense_head_dim_supported(int d);
// Dense launch geometry: the MFMA kernel (4 waves per workgroup, 16-token tiles) takes 16-bit
// q/k/v at head dims 32/64/128; the generic VALU kernel (1 wave, 64-token tiles) the rest.
bool dense_generic(int dtype, int d);
int dense_waves_per_workgroup(int dtype, int d);
int dense_wave_tokens(int dtype, int d, int batch, int hkv, int tc, int tokens_per_block, bool mass);

hipError_t launch_dense(int dtype, int mode, int d, const DenseLaunch& p, hipStream_t stream);
hipError_t launch_finalize(int dtype, const float* acc, const float* l, void* out, int rows, int d,
                           hipStream_t stream);
hipError_t launch_state_init(float* m, float* l, float* acc, int64_t rows, int64_t d, hipStream_t stream);
hipError_t launch_paged(int dtype, int d, const PagedLaunch& p, hipStream_t stream);
hipError_t launch_paged_merge(int dtype, int d, const PagedLaunch& p, int n_seq, hipStream_t stream);
hipError_t launch_mass_reduce(const SeqInfo* seqs, const int32_t* session_rows, const int32_t* session_first,
                              const float* mass_m, const float* mass_s, const float* mf, const float* lf,
                              float* mass_accum, int accum_stride, int hq, int mass_stride, int n_sessions,
                              int max_blocks, hipStream_t stream);
// Deferred mass, once per step: for each session and block, over layers 0..num_layers-1 in
// order, adds the mean over the session's rows and query heads of mass_w[layer] into
// mass_accum, and clears the mass_w entries it reads.
hipError_t launch_mass_step_reduce(const SeqInfo* seqs, const int32_t* session_rows, const int32_t* session_first,
                                   float* mass_w, int64_t layer_floats, int num_layers, float* mass_accum,
                                   int accum_stride, int hq, int mass_stride, int n_sessions, int max_blocks,
                                   hipStream_t stream);

// kv_kernels.hip
// Reference block layout <-> pool records for one layer:
// ref [B, T, Hkv, D] (a layer slice of the [L, B, T, Hkv, D] block) <-> records [B][2][Hkv][T][D].
hipError_t launch_ref_to_records(const void* key, const void* value, void* pool, const int32_t* slots, int rows,
                                 int hkv, int tokens_per_block, int d, hipStream_t stream);
hipError_t launch_records_to_ref(const void* pool, const int32_t* slots, void* key, void* value, int rows, int hkv,
                                 int tokens_per_block, int d, hipStream_t stream);
// Measurement: a plain streaming read of `bytes` (a multiple of 16) with `workgroups` x 256 threads.
hipError_t launch_stream_read(const void* src, int64_t bytes, int workgroups, hipStream_t stream);

}  // namespace pgr
