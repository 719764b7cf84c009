// KV block-store data movement kernels: reference block layout <-> pool records.
// (The decode token is appended by the fused attention kernel.)
//
// Pool record layout for one (block, sequence row, layer): K [Hkv][T][D] followed by V in
// 16-token tiles of four-token transposed groups (v_record_index, pgr_kernels.h); every
// element is 16-bit (fp16 or bf16) and moved as raw bits.
#include <hip/hip_runtime.h>

#include "pgr_common.h"
#include "pgr_kernels.h"

namespace pgr {
namespace {

// ref [B, T, Hkv, D] -> record of row b at slots[b].
__global__ void ref_to_records_kernel(const uint16_t* key, const uint16_t* value, uint16_t* pool,
                                      const int32_t* slots, int rows, int hkv, int tpb, int d) {
  const size_t per_row = (size_t)tpb * hkv * d;
  const size_t total = per_row * rows;
  const size_t rec = 2 * per_row;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t b = i / per_row;
    size_t r = i - b * per_row;
    const int t = (int)(r / ((size_t)hkv * d));
    r -= (size_t)t * hkv * d;
    const int h = (int)(r / d);
    const int dd = (int)(r - (size_t)h * d);
    uint16_t* kr = pool + (size_t)slots[b] * rec;
    kr[((size_t)h * tpb + t) * d + dd] = key[i];
    kr[per_row + v_record_index(h, t, dd, tpb, d)] = value[i];
  }
}

__global__ void records_to_ref_kernel(const uint16_t* pool, const int32_t* slots, uint16_t* key, uint16_t* value,
                                      int rows, int hkv, int tpb, int d) {
  const size_t per_row = (size_t)tpb * hkv * d;
  const size_t total = per_row * rows;
  const size_t rec = 2 * per_row;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t b = i / per_row;
    size_t r = i - b * per_row;
    const int t = (int)(r / ((size_t)hkv * d));
    r -= (size_t)t * hkv * d;
    const int h = (int)(r / d);
    const int dd = (int)(r - (size_t)h * d);
    const uint16_t* kr = pool + (size_t)slots[b] * rec;
    key[i] = kr[((size_t)h * tpb + t) * d + dd];
    value[i] = kr[per_row + v_record_index(h, t, dd, tpb, d)];
  }
}

unsigned grid_for(size_t total) {
  size_t blocks = (total + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  if (blocks == 0) blocks = 1;
  return (unsigned)blocks;
}

}  // namespace

hipError_t launch_ref_to_records(const void* key, const void* value, void* pool, const int32_t* slots, int rows,
                                 int hkv, int tokens_per_block, int d, hipStream_t stream) {
  const size_t total = (size_t)rows * tokens_per_block * hkv * d;
  if (total == 0) return hipSuccess;
  ref_to_records_kernel<<<grid_for(total), 256, 0, stream>>>(static_cast<const uint16_t*>(key),
                                                             static_cast<const uint16_t*>(value),
                                                             static_cast<uint16_t*>(pool), slots, rows, hkv,
                                                             tokens_per_block, d);
  return hipGetLastError();
}

hipError_t launch_records_to_ref(const void* pool, const int32_t* slots, void* key, void* value, int rows, int hkv,
                                 int tokens_per_block, int d, hipStream_t stream) {
  const size_t total = (size_t)rows * tokens_per_block * hkv * d;
  if (total == 0) return hipSuccess;
  records_to_ref_kernel<<<grid_for(total), 256, 0, stream>>>(static_cast<const uint16_t*>(pool), slots,
                                                             static_cast<uint16_t*>(key),
                                                             static_cast<uint16_t*>(value), rows, hkv,
                                                             tokens_per_block, d);
  return hipGetLastError();
}

}  // namespace pgr
