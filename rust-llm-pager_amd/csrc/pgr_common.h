// Shared definitions for the native decode-attention library (host and device).
#pragma once

#include <cstddef>
#include <cstdint>

namespace pgr {

// Element types of Q/K/V/output. Matches PGR_DTYPE_* in include/pgr.h. fp32 is taken by the
// dense operator API and finalize only; the paged store holds 16-bit K/V.
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

// Status codes. Matches PGR_* in include/pgr.h.
enum Status : int {
  kOk = 0,
  kErrInvalid = -1,      // bad argument (shape, null pointer, range)
  kErrUnsupported = -2,  // valid but unsupported configuration (head_dim, n_rep > 16, ...)
  kErrHip = -3,          // a HIP runtime call failed
  kErrCapacity = -4,     // a fixed-capacity pool or workspace is too small
  kErrState = -5,        // call not valid in the object's current state
  kErrKey = -6,          // unknown block / sequence id
  kErrBudget = -7,       // ram budget would be exceeded
  kErrInternal = -8,     // an internal failure (an exception caught at the C boundary)
};

// Query heads sharing one KV head are packed into the 16 columns of one MFMA tile.
constexpr int kMaxRep = 16;
// Waves per workgroup in the attention kernels.
constexpr int kWaves = 4;
constexpr int kWaveSize = 64;

// One KV block as the paged kernel sees it.
struct BlockEntry {
  int32_t slot;      // >= 0: record index in the layer's HBM pool; < 0: staging record (-slot - 1)
  int32_t block_id;  // logical block id within the sequence; first token = block_id * tokens_per_block
};

// Block entries one workgroup folds at most (4 waves x 8 blocks).
constexpr int kMaxWorkEntries = 32;

// One workgroup's share of a paged decode step (times num_kv_heads via blockIdx.y). Self-
// contained, so a workgroup needs a single (scalar) read before it issues its K/V loads.
struct WorkItem {
  int32_t seq;          // sequence index: row of q / out
  int32_t partial;      // partial-result slot written by this workgroup
  int32_t entry_count;  // number of entries (blocks) it folds
  int32_t lo;           // stored valid tokens [lo, hi) of the sequence
  int32_t hi;
  int32_t n_mass;       // blocks below this id get a mass entry
  int32_t append_slot;  // >= 0 (one work item per sequence): write the current token's K/V to
  int32_t append_pos;   // position append_pos of pool record append_slot
  // Mirror mode: host record r of this sequence sits at record r - mirror_off of the layer's
  // ring buffer (the step's host span of each row is packed there); 0 in the other modes.
  int32_t mirror_off;
  int32_t pad_[3];
  BlockEntry entries[kMaxWorkEntries];
};

// Per-sequence scalars of a paged decode step.
struct SeqInfo {
  int32_t lo;            // first valid token position (left padding / sliding window)
  int32_t hi;            // position of the current token: stored tokens [lo, hi) are read
  int32_t n_mass;        // blocks [0, n_mass) get a mass entry (the full blocks known before this step)
  int32_t mass_lo;       // first block id in scope for mass (blocks below were skipped: mass 0)
  int32_t partial_base;  // first partial slot of this sequence
  int32_t partial_count; // number of partial slots (work items) of this sequence
  int32_t session;       // session index (rows of one session share placement and mass)
  uint32_t step_token;   // the step's number (mirror mode: the merge publishes it per layer)
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace pgr
