// Single-token GQA decode attention for CDNA4 (gfx950).
//
// Every kernel here computes, for one batch row and one KV head, the attention of the
// n_rep query heads that share that KV head (heads kv*n_rep .. kv*n_rep+n_rep-1, the
// repeat-interleave grouping of pager_hf/streaming_attention.py:119-123) over a range of
// KV tokens, with fp32 online-softmax state.
//
// MFMA mapping (v_mfma_f32_16x16x16 f16/bf16, fp32 accumulate). A 16-token tile is folded as
//     S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//     O^T[D x 16 heads]     += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
// Lane l = 16*g + n holds S^T rows 4g..4g+3 (four tokens) of column n (query head n).
// That register block is exactly the P^T operand of the second product, and every O^T
// value a lane holds belongs to head n as well, so the softmax state (m, l) and the
// rescale factor are per-lane scalars: no cross-lane traffic inside the tile except the
// max over the four lane groups g. Columns n >= n_rep are zero-query padding and are
// never stored (the reference pads its M tile the same way, streaming_attention.py:55).
//
// Operand layouts (verified on gfx950 with a probe): A[i][k]: lane i + 16*(k/4), element
// k%4; B[k][j]: lane j + 16*(k/4), element k%4; C[i][j]: lane j + 16*(i/4), element i%4.
// The contraction index of S^T (head_dim) is permuted so that lane (g, n) reads one
// contiguous run of D/4 elements of K row n: chunk c, k-slot 4g+i <-> dim (D/4)g + 4c + i.
// V is read as four token rows of D/16 contiguous elements (dims (D/16)n .. +D/16) and
// transposed in registers with v_perm_b32 into the A operand of each of the D/16 M-tiles;
// M-tile j, row r <-> dim (D/16)r + j. In the dense kernel all global loads are 16/8/4-byte
// per lane and one K load instruction covers half of each of the tile's 16 rows. The paged
// kernel reads records whose V is stored transposed in groups of four tokens (PTile), so its
// V operands arrive as 16-byte loads in MFMA order with no permutes.
//
// P is rounded to the K/V element type before the P.V product, as the reference does
// (streaming_attention.py:178, :347, :428).
#include <hip/hip_runtime.h>

#include "pgr_common.h"
#include "pgr_kernels.h"

namespace pgr {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_inff();

struct F16 {
  static __device__ __forceinline__ f32x4 mma(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    f16x2 h = {(_Float16)x, (_Float16)y};
    return __builtin_bit_cast(uint32_t, h);
  }
  static __device__ __forceinline__ uint16_t cvt(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
  static __device__ __forceinline__ float to_f(uint16_t x) { return (float)__builtin_bit_cast(_Float16, x); }
};

struct BF16 {
  static __device__ __forceinline__ f32x4 mma(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0,
                                                     0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    bf16x2 h = {(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, h);
  }
  static __device__ __forceinline__ uint16_t cvt(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
  static __device__ __forceinline__ float to_f(uint16_t x) { return __builtin_bit_cast(float, (uint32_t)x << 16); }
};

__device__ __forceinline__ float wave_max_g(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float wave_sum_g(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Registers of one 16-token tile held by one lane.
template <int D>
struct Tile {
  static_assert(D == 32 || D == 64 || D == 128, "head_dim must be 32, 64 or 128");
  static constexpr int KV4 = D / 32;  // u32x4 of K per lane (D/4 elements)
  static constexpr int VW = D / 32;   // dwords of V per token row per lane (D/16 elements)
  u32x4 k[KV4];
  uint32_t v[4][VW];
};

// K row `row` of the tile at `tile_k` (row stride D elements): elements (D/4)g .. +D/4.
template <int D>
__device__ __forceinline__ void load_k(Tile<D>& t, const uint16_t* tile_k, int row, int g) {
  const u32x4* p = reinterpret_cast<const u32x4*>(tile_k + (size_t)row * D + (D / 4) * g);
#pragma unroll
  for (int i = 0; i < Tile<D>::KV4; ++i) t.k[i] = p[i];
}

// V rows rows[0..3] at `tile_v`: elements (D/16)n .. +D/16 of each.
template <int D>
__device__ __forceinline__ void load_v(Tile<D>& t, const uint16_t* tile_v, const int (&rows)[4], int n) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t* p = tile_v + (size_t)rows[i] * D + (D / 16) * n;
    if constexpr (D == 32) {
      t.v[i][0] = *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (D == 64) {
      u32x2 x = *reinterpret_cast<const u32x2*>(p);
      t.v[i][0] = x.x;
      t.v[i][1] = x.y;
    } else {
      u32x4 x = *reinterpret_cast<const u32x4*>(p);
      t.v[i][0] = x.x;
      t.v[i][1] = x.y;
      t.v[i][2] = x.z;
      t.v[i][3] = x.w;
    }
  }
}

template <int D>
__device__ __forceinline__ void zero_v_row(Tile<D>& t, int i) {
#pragma unroll
  for (int w = 0; w < Tile<D>::VW; ++w) t.v[i][w] = 0u;
}

// K operand (A of S^T) for contraction chunk c: dwords 2c, 2c+1 of the lane's K run.
template <int D>
__device__ __forceinline__ u32x2 k_chunk(const u32x4 (&k)[D / 32], int c) {
  const u32x4 q = k[c >> 1];
  return (c & 1) ? u32x2{q.z, q.w} : u32x2{q.x, q.y};
}

// V^T operand (A of O^T) for M-tile j: element j of each of the four token rows.
template <int D>
__device__ __forceinline__ u32x2 v_tile(const uint32_t (&v)[4][D / 32], int j) {
  const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
  const int w = j >> 1;
  return u32x2{__builtin_amdgcn_perm(v[1][w], v[0][w], sel), __builtin_amdgcn_perm(v[3][w], v[2][w], sel)};
}

// S^T tile of 16 tokens x 16 heads.
template <class Ty, int D>
__device__ __forceinline__ f32x4 qk_tile(const u32x4 (&k)[D / 32], const u32x4 (&q)[D / 32]) {
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < D / 16; ++c) s = Ty::mma(k_chunk<D>(k, c), k_chunk<D>(q, c), s);
  return s;
}

template <class Ty, int D>
__device__ __forceinline__ void pv_tile(f32x4 (&acc)[D / 16], const Tile<D>& t, const float (&p)[4]) {
  const u32x2 pb = {Ty::pack(p[0], p[1]), Ty::pack(p[2], p[3])};
#pragma unroll
  for (int j = 0; j < D / 16; ++j) acc[j] = Ty::mma(v_tile<D>(t.v, j), pb, acc[j]);
}

// Scale + optional softcap of one raw score (streaming_attention.py:158-160).
__device__ __forceinline__ float transform_score(float s, float scale, float softcap) {
  s = s * scale;
  if (softcap > 0.f) s = softcap * tanhf(s / softcap);
  return s;
}

// Dims held by lane (g, n) for O^T M-tile j, element i: (D/4)g + (D/16)i + j.
template <int D>
__device__ __forceinline__ int acc_dim(int g, int i, int j) {
  return (D / 4) * g + (D / 16) * i + j;
}

// Q^T operand for query head (row index `qrow` of a [rows, D] array); zero for padding heads.
template <int D>
__device__ __forceinline__ void load_q(u32x4 (&q)[D / 32], const uint16_t* qptr, bool real, int g) {
#pragma unroll
  for (int i = 0; i < D / 32; ++i) q[i] = u32x4{0u, 0u, 0u, 0u};
  if (real) {
    const u32x4* p = reinterpret_cast<const u32x4*>(qptr + (D / 4) * g);
#pragma unroll
    for (int i = 0; i < D / 32; ++i) q[i] = p[i];
  }
}

template <bool kLog2>
__device__ __forceinline__ float exp_w(float x) {
  if constexpr (kLog2)
    return __builtin_amdgcn_exp2f(x);
  else
    return __expf(x);
}

// ---------------------------------------------------------------------------------------
// Workgroup merge of the four waves' (m, l, acc) and store of one partial slot.
// FOLD: online-softmax partials; FIXED: plain acc sums (m is the caller's fixed max).
template <int D>
struct MergeSmem {
  float m[kWaves][kMaxRep];
  float l[kWaves][kMaxRep];
  float acc[kWaves][kMaxRep][D + 1];
};

// kLog2: (m, scores) are in log2 units and the weights are exp2(m_w - m); otherwise e-based.
template <int D, bool kFold, bool kWithAcc, bool kLog2 = false>
__device__ __forceinline__ void wg_merge_store(MergeSmem<D>& sm, int wave, int g, int n, float m_run, float l_lane,
                                               const f32x4 (&acc)[D / 16], int n_rep, float* pm, float* pl,
                                               float* pacc) {
  const float l_wave = wave_sum_g(l_lane);
  if (g == 0) {
    sm.m[wave][n] = m_run;
    sm.l[wave][n] = l_wave;
  }
  if constexpr (kWithAcc) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.acc[wave][n][acc_dim<D>(g, i, j)] = acc[j][i];
  }
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < n_rep) {
    const int r = tid;
    if constexpr (kFold) {
      float mw = kNegInf;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) mw = fmaxf(mw, sm.m[w][r]);
      float lw = 0.f;
      if (mw != kNegInf) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) lw += sm.l[w][r] * exp_w<kLog2>(sm.m[w][r] - mw);
      }
      pm[r] = mw;
      pl[r] = lw;
    }
  }
  if constexpr (kWithAcc) {
    for (int idx = tid; idx < n_rep * D; idx += kWaves * kWaveSize) {
      const int r = idx / D, d = idx - r * D;
      float a = 0.f;
      if constexpr (kFold) {
        float mw = kNegInf;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mw = fmaxf(mw, sm.m[w][r]);
        if (mw != kNegInf) {
#pragma unroll
          for (int w = 0; w < kWaves; ++w) a += sm.acc[w][r][d] * exp_w<kLog2>(sm.m[w][r] - mw);
        }
      } else {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) a += sm.acc[w][r][d];
      }
      pacc[idx] = a;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Dense chunk kernel: the operator API of pager_hf/streaming_attention.py:452-665.
// k, v: [B, Hkv, Tc, D] contiguous. Grid (n_split, Hkv, B); each wave folds
// `wave_tokens` consecutive tokens, the workgroup covers 4 * wave_tokens.
enum DenseMode : int { kModeFold = 0, kModeStats = 1, kModeAccumulate = 2, kModeFoldFixed = 3 };

struct DenseArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* valid;   // [B, Tc] or null (all valid)
  const int32_t* active;  // [B] or null (all active)
  const float* m_in;      // FIXED modes: final m [B, Hq]
  const float* l_in;      // FIXED modes: final l [B, Hq]
  float* block_mass;      // accumulate: [B, Hq, max_blocks]
  float* pm;              // partials [slot][n_rep]
  float* pl;
  float* pacc;            // [slot][n_rep][D]
  int tc, hq, hkv, n_rep, n_split, wave_tokens;
  int tokens_per_block, max_blocks, block_id_offset;
  float scale, softcap;
};

template <class Ty, int D, int kMode>
__global__ __launch_bounds__(256) void dense_attn_kernel(DenseArgs a) {
  constexpr bool kFold = (kMode == kModeFold || kMode == kModeStats);
  constexpr bool kWithV = (kMode != kModeStats);
  constexpr bool kMass = (kMode == kModeAccumulate);
  __shared__ MergeSmem<D> sm;

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  if (a.active != nullptr && a.active[b] == 0) return;  // whole workgroup: uniform exit
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, n = lane & 15;
  const bool real = n < a.n_rep;
  const int qh = h * a.n_rep + (real ? n : 0);

  const size_t kv_base = ((size_t)b * a.hkv + h) * (size_t)a.tc * D;
  const uint16_t* kp = a.k + kv_base;
  const uint16_t* vp = a.v + kv_base;

  const int t_begin = split * kWaves * a.wave_tokens + wave * a.wave_tokens;
  const int t_end = min(t_begin + a.wave_tokens, a.tc);
  const int tiles = t_begin < t_end ? (t_end - t_begin + 15) / 16 : 0;
  const int tiles_per_block = kMass ? a.tokens_per_block / 16 : 1;

  // Tile ti's K and V (rows past the chunk clamped to its last row, then masked) and which of
  // the lane's four V rows are valid tokens.
  auto fetch = [&](Tile<D>& t, bool (&ok)[4], int ti) {
    const int t0 = t_begin + ti * 16;
    load_k<D>(t, kp, min(t0 + n, a.tc - 1), g);
    int rows[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = t0 + 4 * g + i;
      ok[i] = tok < t_end;
      if (ok[i] && a.valid != nullptr) ok[i] = a.valid[(size_t)b * a.tc + tok] != 0;
      rows[i] = min(tok, a.tc - 1);
    }
    if constexpr (kWithV) load_v<D>(t, vp, rows, n);
  };

  Tile<D> ta, tb;
  bool oka[4], okb[4];
  if (tiles > 0) fetch(ta, oka, 0);  // the first tile's loads go out before the query's

  u32x4 q[D / 32];
  load_q<D>(q, a.q + ((size_t)b * a.hq + qh) * D, real, g);

  float m_run = kNegInf, l_run = 0.f;
  float m_fix = 0.f, l_fix = 1.f;
  if constexpr (!kFold) {
    if (real) {
      m_fix = a.m_in[(size_t)b * a.hq + qh];
      l_fix = a.l_in[(size_t)b * a.hq + qh];
    }
  }
  f32x4 acc[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float blk = 0.f;

  auto process = [&](Tile<D>& t, const bool (&ok)[4], int ti) {
    const int t0 = t_begin + ti * 16;
    if constexpr (kWithV) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!ok[i]) zero_v_row<D>(t, i);
    }
    const f32x4 s4 = qk_tile<Ty, D>(t.k, q);
    float s[4], p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = ok[i] ? transform_score(s4[i], a.scale, a.softcap) : kNegInf;

    if constexpr (kFold) {
      const float tmax = wave_max_g(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
      const float m_new = fmaxf(m_run, tmax);
      const bool empty = (m_new == kNegInf);
      const float alpha = empty ? 0.f : __expf(m_run - m_new);
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = empty ? 0.f : __expf(s[i] - m_new);
      l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
      if constexpr (kWithV) {
#pragma unroll
        for (int j = 0; j < D / 16; ++j) acc[j] *= alpha;
        pv_tile<Ty, D>(acc, t, p);
      }
      m_run = m_new;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = ok[i] ? __expf(s[i] - m_fix) : 0.f;
      pv_tile<Ty, D>(acc, t, p);
      if constexpr (kMass) {
        blk += (p[0] + p[1]) + (p[2] + p[3]);
        if ((ti + 1) % tiles_per_block == 0 || ti + 1 == tiles) {
          const float bs = wave_sum_g(blk);
          if (g == 0 && real) {
            const int j = t0 / a.tokens_per_block;
            a.block_mass[((size_t)b * a.hq + qh) * a.max_blocks + a.block_id_offset + j] = bs / l_fix;
          }
          blk = 0.f;
        }
      }
    }
  };

  // Two tiles per wave in flight: the next tile's loads are issued before the current tile is
  // folded. Unconditional in the loop (a conditional fetch lets the compiler drain the load
  // queue every iteration); the last one or two tiles are folded after it.
  int ti = 0;
  for (; ti + 2 < tiles; ti += 2) {
    fetch(tb, okb, ti + 1);
    process(ta, oka, ti);
    fetch(ta, oka, ti + 2);
    process(tb, okb, ti + 1);
  }
  if (ti + 1 < tiles) {
    fetch(tb, okb, ti + 1);
    process(ta, oka, ti);
    process(tb, okb, ti + 1);
  } else if (ti < tiles) {
    process(ta, oka, ti);
  }

  const size_t slot = ((size_t)b * a.hkv + h) * a.n_split + split;
  wg_merge_store<D, kFold, kWithV>(sm, wave, g, n, m_run, l_run, acc, a.n_rep, a.pm + slot * a.n_rep,
                                   a.pl + slot * a.n_rep, a.pacc + slot * a.n_rep * D);
}

// l of head r from a per-head register array, with r a per-lane value (no dynamic indexing).
template <int N>
__device__ __forceinline__ float l_run_at(const float (&l)[N], int r) {
  float x = 0.f;
#pragma unroll
  for (int q = 0; q < N; ++q)
    if (q == r) x = l[q];
  return x;
}

// ---------------------------------------------------------------------------------------
// Generic dense chunk kernel: the operator API for the cases the MFMA kernel above does not
// take -- fp32 q/k/v (any head dim) and 16-bit head dims 8, 16 and 256. The reference pads
// Q and K with zero columns up to 16 when head_dim < 16 (streaming_attention.py:56-66,
// :125-133) so that tl.dot applies; zero columns add nothing to a dot product, and this
// kernel computes the unpadded dot products directly on the VALU.
//
// One wave per workgroup, grid (n_split, Hkv, B); the wave folds `wave_tokens` consecutive
// tokens in tiles of 64, with the same partial layout and e-based (m, l) as
// dense_attn_kernel, so dense_merge_kernel combines either. Per tile:
//   1. scores: lane t takes token t0 + t and all n_rep query heads (q in LDS);
//   2. softmax: per head, a wave max / sum; P (rounded to the K/V type before P.V, as
//      streaming_attention.py:178 does) goes to LDS;
//   3. P.V: lane (g, c) takes head dims c, c + 64, ... of tokens g, g + G, ... (G = 64 / min(D, 64)),
//      so each V row is read by consecutive lanes; the token groups are summed at the end.
constexpr int kGenTile = 64;

template <class Ty>
struct GenElem {  // 16-bit K/V/q elements
  typedef uint16_t T;
  static __device__ __forceinline__ float ld(const T* p) { return Ty::to_f(*p); }
  static __device__ __forceinline__ float round_p(float p) { return Ty::to_f(Ty::cvt(p)); }
};
struct F32Elem {
  typedef float T;
  static __device__ __forceinline__ float ld(const T* p) { return *p; }
  static __device__ __forceinline__ float round_p(float p) { return p; }
};

__device__ __forceinline__ float wave_max64(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum64(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <class E, int D, int kMode>
__global__ __launch_bounds__(64) void dense_generic_kernel(DenseArgs a) {
  constexpr bool kFold = (kMode == kModeFold || kMode == kModeStats);
  constexpr bool kWithV = (kMode != kModeStats);
  constexpr bool kMass = (kMode == kModeAccumulate);
  constexpr int DL = D < 64 ? D : 64;  // lanes per token group in the P.V pass
  constexpr int G = 64 / DL;           // token groups
  constexpr int DPL = D / DL;          // head dims per lane
  typedef typename E::T T;
  __shared__ float q_s[kMaxRep][D];
  __shared__ float p_s[kMaxRep][kGenTile];    // P rounded for P.V
  __shared__ float praw_s[kMaxRep][kGenTile];  // P unrounded, for the block mass
  __shared__ float alpha_s[kMaxRep];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  if (a.active != nullptr && a.active[b] == 0) return;  // whole workgroup: uniform exit
  const int lane = threadIdx.x;
  const int n_rep = a.n_rep;
  const size_t kv_base = ((size_t)b * a.hkv + h) * (size_t)a.tc * D;
  const T* kp = reinterpret_cast<const T*>(a.k) + kv_base;
  const T* vp = reinterpret_cast<const T*>(a.v) + kv_base;
  const T* qp = reinterpret_cast<const T*>(a.q) + ((size_t)b * a.hq + (size_t)h * n_rep) * D;
  for (int i = lane; i < kMaxRep * D; i += 64) {
    const int r = i / D;
    q_s[r][i - r * D] = r < n_rep ? E::ld(qp + i) : 0.f;
  }
  // Running (m, l) per head: uniform values, kept in registers of every lane.
  float m_run[kMaxRep], l_run[kMaxRep], blk[kMaxRep];
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r) {
    m_run[r] = kNegInf;
    l_run[r] = 0.f;
    blk[r] = 0.f;
    if constexpr (!kFold) {
      if (r < n_rep) {
        m_run[r] = a.m_in[(size_t)b * a.hq + h * n_rep + r];
        l_run[r] = a.l_in[(size_t)b * a.hq + h * n_rep + r];
      }
    }
  }
  float acc[kMaxRep][DPL];
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r)
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[r][j] = 0.f;
  __syncthreads();

  const int t_begin = split * a.wave_tokens;
  const int t_end = min(t_begin + a.wave_tokens, a.tc);
  const int grp = lane / DL, col = lane - grp * DL;
  for (int t0 = t_begin; t0 < t_end; t0 += kGenTile) {
    // 1. Scores of token t0 + lane for every head.
    const int t = t0 + lane;
    bool ok = t < t_end;
    if (ok && a.valid != nullptr) ok = a.valid[(size_t)b * a.tc + t] != 0;
    float s[kMaxRep];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) s[r] = 0.f;
    if (ok) {
      const T* krow = kp + (size_t)t * D;
      for (int d = 0; d < D; ++d) {
        const float kd = E::ld(krow + d);
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r) s[r] += q_s[r][d] * kd;
      }
    }
    // 2. Softmax weights per head.
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
      if (r >= n_rep) continue;  // uniform
      const float x = ok ? transform_score(s[r], a.scale, a.softcap) : kNegInf;
      float p;
      if constexpr (kFold) {
        const float m_new = fmaxf(m_run[r], wave_max64(x));
        const bool empty = m_new == kNegInf;
        const float alpha = empty ? 0.f : __expf(m_run[r] - m_new);
        p = (empty || !ok) ? 0.f : __expf(x - m_new);
        l_run[r] = l_run[r] * alpha + wave_sum64(p);
        m_run[r] = m_new;
        if (lane == 0) alpha_s[r] = alpha;
      } else {
        p = ok ? __expf(x - m_run[r]) : 0.f;
      }
      p_s[r][lane] = E::round_p(p);
      if constexpr (kMass) praw_s[r][lane] = p;
    }
    __syncthreads();
    // 3. P.V over this tile.
    if constexpr (kWithV) {
      if constexpr (kFold) {
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r) {
          if (r >= n_rep) continue;
          const float al = alpha_s[r];
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[r][j] *= al;
        }
      }
      const int n_tok = min(kGenTile, t_end - t0);
      for (int tt = grp; tt < n_tok; tt += G) {
        const T* vrow = vp + (size_t)(t0 + tt) * D;
        float vv[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) vv[j] = E::ld(vrow + col + j * DL);
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r) {
          if (r >= n_rep) continue;
          const float pr = p_s[r][tt];
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[r][j] += pr * vv[j];
        }
      }
    }
    // Block mass (accumulate mode): lane r sums its head's weights token by token, in order,
    // and writes sum / l at the last token of each block (or of the wave's range).
    if constexpr (kMass) {
      if (lane < n_rep) {
        const int r = lane;
        const int n_tok = min(kGenTile, t_end - t0);
        float bs = 0.f;
#pragma unroll
        for (int q = 0; q < kMaxRep; ++q)
          if (q == r) bs = blk[q];
        const int qh = h * n_rep + r;
        for (int tt = 0; tt < n_tok; ++tt) {
          bs += praw_s[r][tt];
          const int tok = t0 + tt;
          if ((tok + 1) % a.tokens_per_block == 0 || tok + 1 == t_end) {
            a.block_mass[((size_t)b * a.hq + qh) * a.max_blocks + a.block_id_offset + tok / a.tokens_per_block] =
                bs / l_run_at(l_run, r);
            bs = 0.f;
          }
        }
#pragma unroll
        for (int q = 0; q < kMaxRep; ++q)
          if (q == r) blk[q] = bs;
      }
    }
    __syncthreads();
  }

  // Partials: token groups summed across lanes (xor over the group bits of the lane id).
  const size_t slot = ((size_t)b * a.hkv + h) * a.n_split + split;
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r) {
    if (r >= n_rep) continue;
    if constexpr (kWithV) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        float x = acc[r][j];
#pragma unroll
        for (int o = DL; o < 64; o <<= 1) x += __shfl_xor(x, o);
        if (grp == 0) a.pacc[(slot * n_rep + r) * D + col + j * DL] = x;
      }
    }
    if constexpr (kFold) {
      if (lane == 0) {
        a.pm[slot * n_rep + r] = m_run[r];
        a.pl[slot * n_rep + r] = l_run[r];
      }
    }
  }
}

// Combine the dense partials into the caller's running state, in place.
// Split-K merge of the operator kernels: one 256-thread workgroup per (batch row, query head).
// Thread (g, c) owns dims 2c, 2c+1 (D/2 columns) and merges the partial slots g, g+G, g+2G, ...
// (G = 512/D groups) online, with kDenseMergeBatch slots' loads in flight before it uses any:
// a running max and sums rescaled under it (e-based units, as the operator state). The groups
// then combine through LDS with the state already in (m, l, acc). Stats mode merges (m, l)
// only; the fixed-max modes add the partial sums as they are. A slot whose split held no valid
// token carries m = -inf and adds nothing; if nothing is valid anywhere the state is left as
// it was.
constexpr int kDenseMergeThreads = 256;
constexpr int kDenseMergeBatch = 8;

template <int kMode>
__global__ __launch_bounds__(kDenseMergeThreads) void dense_merge_kernel(DenseArgs a, float* m, float* l, float* acc,
                                                                         int d) {
  __shared__ float sm_m[kDenseMergeThreads];
  __shared__ float sm_l[kDenseMergeThreads];
  __shared__ float sm_a[2 * kDenseMergeThreads];
  const int row = blockIdx.x;  // b * hq + qh
  const int b = row / a.hq, qh = row - b * a.hq;
  if (a.active != nullptr && a.active[b] == 0) return;  // whole workgroup: uniform exit
  const int h = qh / a.n_rep, r = qh - h * a.n_rep;
  const size_t slot0 = ((size_t)b * a.hkv + h) * a.n_split;
  const int cols = d / 2;                          // d is even (8 .. 256)
  const int groups = kDenseMergeThreads / cols;    // 1 .. 64
  const int g = threadIdx.x / cols, c = threadIdx.x - g * cols;
  constexpr bool kOnline = kMode == kModeFold || kMode == kModeStats;
  constexpr bool kAcc = kMode != kModeStats;
  float mx = kNegInf, ls = 0.f, a0 = 0.f, a1 = 0.f;
  const int n = a.n_split;
  for (int s0 = g; s0 < n; s0 += groups * kDenseMergeBatch) {
    float pmv[kDenseMergeBatch], plv[kDenseMergeBatch], p0[kDenseMergeBatch], p1[kDenseMergeBatch];
#pragma unroll
    for (int j = 0; j < kDenseMergeBatch; ++j) {
      const int sj = s0 + j * groups;
      const size_t slot = (slot0 + (sj < n ? sj : s0)) * a.n_rep + r;  // past the last slot: re-read s0, weight 0
      pmv[j] = kOnline ? (sj < n ? a.pm[slot] : kNegInf) : 0.f;
      plv[j] = kOnline ? a.pl[slot] : 0.f;
      if constexpr (kAcc) {
        const float2 v2 = *reinterpret_cast<const float2*>(a.pacc + slot * d + 2 * c);
        p0[j] = sj < n ? v2.x : 0.f;
        p1[j] = sj < n ? v2.y : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < kDenseMergeBatch; ++j) {
      if constexpr (kOnline) {
        const float mn = fmaxf(mx, pmv[j]);
        if (mn != kNegInf) {
          const float so = __expf(mx - mn), ss = __expf(pmv[j] - mn);
          ls = ls * so + plv[j] * ss;
          if constexpr (kAcc) {
            a0 = a0 * so + p0[j] * ss;
            a1 = a1 * so + p1[j] * ss;
          }
          mx = mn;
        }
      } else {
        a0 += p0[j];
        a1 += p1[j];
      }
    }
  }
  if (c == 0) {
    sm_m[g] = mx;
    sm_l[g] = ls;
  }
  if constexpr (kAcc) {
    sm_a[g * d + 2 * c] = a0;
    sm_a[g * d + 2 * c + 1] = a1;
  }
  __syncthreads();
  if (g != 0) return;
  if constexpr (kOnline) {
    const float m0 = m[row];
    float mf = m0;
    for (int gg = 0; gg < groups; ++gg) mf = fmaxf(mf, sm_m[gg]);
    if (mf == kNegInf) return;  // nothing valid anywhere yet: the state stays as it is
    const float w0 = __expf(m0 - mf);
    float lf = l[row] * w0;
    float x0 = 0.f, x1 = 0.f;
    if constexpr (kAcc) {
      x0 = acc[(size_t)row * d + 2 * c] * w0;
      x1 = acc[(size_t)row * d + 2 * c + 1] * w0;
    }
    for (int gg = 0; gg < groups; ++gg) {
      if (sm_m[gg] == kNegInf) continue;
      const float wg = __expf(sm_m[gg] - mf);
      lf += sm_l[gg] * wg;
      if constexpr (kAcc) {
        x0 += sm_a[gg * d + 2 * c] * wg;
        x1 += sm_a[gg * d + 2 * c + 1] * wg;
      }
    }
    if constexpr (kAcc) {
      acc[(size_t)row * d + 2 * c] = x0;
      acc[(size_t)row * d + 2 * c + 1] = x1;
    }
    if (c == 0) {
      m[row] = mf;
      l[row] = lf;
    }
  } else {
    float x0 = acc[(size_t)row * d + 2 * c], x1 = acc[(size_t)row * d + 2 * c + 1];
    for (int gg = 0; gg < groups; ++gg) {
      x0 += sm_a[gg * d + 2 * c];
      x1 += sm_a[gg * d + 2 * c + 1];
    }
    acc[(size_t)row * d + 2 * c] = x0;
    acc[(size_t)row * d + 2 * c + 1] = x1;
  }
}

template <class Ty>
__global__ void finalize_kernel(const float* acc, const float* l, uint16_t* out, int rows, int d) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * d) return;
  out[i] = Ty::cvt(acc[i] / l[i / d]);
}

__global__ void finalize_f32_kernel(const float* acc, const float* l, float* out, int rows, int d) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * d) return;
  out[i] = acc[i] / l[i / d];
}

// Fresh operator state in one launch: m = -inf, l = 0 for `rows` rows, acc = 0 for rows * d.
__global__ void state_init_kernel(float* m, float* l, float* acc, int64_t rows, int64_t n_acc) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_acc; i += stride) {
    acc[i] = 0.f;
    if (i < rows) {
      m[i] = kNegInf;
      l[i] = 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Paged kernel: the fused decode path. Blocks are read in place from the layer's HBM
// pool, from the mapped pinned host mirror, or from a staging buffer filled by
// host-to-device copies; record layout per (block, sequence): K [Hkv][T][D] then
// V [Hkv][T][D]. Grid (n_work, Hkv).
//
// Each wave streams the blocks w, w+4, ... of its work item through a ring of NB register
// tiles (NB-1 tiles of loads in flight while one is folded). Everything that selects a
// tile (entry, slot, block id, tile index) is wave-uniform and lives in SGPRs; a lane's
// part of a tile is a fixed byte offset, so every load is one `buffer_load` with the
// tile's offsets in SGPRs.
//
// Scores are kept in log2 units (x = s * scale * log2 e, p = 2^(x - m)). The running max m
// is refreshed lazily: a tile rescales (m, l, acc) only when one of its scores exceeds m
// by more than kLazyRescale, so p <= 2^kLazyRescale and most tiles skip the cross-lane max
// and the acc rescale. The final (m, l, acc) describe the same softmax exactly; P is still
// rounded to the K/V type before P.V (streaming_attention.py:178).
struct PagedArgs {
  const uint16_t* q;      // [S, Hq, D]
  const uint16_t* k_new;  // [S, Hkv, D]: the current token (appended here, attended in the merge)
  const uint16_t* v_new;
  uint16_t* pool;         // layer pool base
  const uint16_t* stage;  // staging base
  const WorkItem* work;
  WorkItem* work_out;     // first launch of a step: device copy of the plan (see PagedLaunch)
  const void* aux_src;
  void* aux_dst;
  int64_t aux_vec;
  const SeqInfo* seqs;
  float* pm;              // [slot][Hq], log2 units
  float* pl;
  float* pacc;            // [slot][Hq][D]
  float* mass_m;          // [S][Hq][mass_stride], log2 units (null: no mass)
  float* mass_s;
  uint16_t* out;          // [S, Hq, D]
  float* mf;              // [S, Hq]: final max (log2 units) and sum, for the mass pass
  float* lf;
  int hq, hkv, n_rep, tokens_per_block, mass_stride;
  float scale, softcap;
  int window;             // > 0: the layer's sliding window (see PagedLaunch)
  const uint16_t* mirror;       // mirror mode: the layer's ring buffer (host records, packed), or null
  const uint32_t* mirror_flag;  // set once this layer's copies into `mirror` have landed
  uint32_t* plan_flag;    // merge: pinned word for plan_token (see PagedLaunch), or null
  uint32_t plan_token;
  uint32_t* release_flag; // merge, mirror mode: pinned word for the step token (see PagedLaunch)
  float* mass_w;          // merge, deferred mass: this layer's [S][Hq][mass_stride] weights
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyRescale = 8.0f;
constexpr float kMInit = -1.0e30f;  // running max before any valid score (finite: 2^(-inf - kMInit) = 0)


// Registers of one 16-token tile in the decode kernel, both read as D/2 contiguous bytes per
// lane: K row n, dims (D/4)g .. (D/4)g + D/4 - 1 (the chunks of the S^T products), and V in
// the record's transposed layout (v_record_index, pgr_kernels.h): tokens 4g..4g+3 of dims
// (D/16)n .. (D/16)n + D/16 - 1, four tokens per dim, which are the A operands of the D/16
// O^T products as they stand (M-tile j = dwords 2j, 2j + 1). A lane's run is D/32 16-byte
// vectors, or one 8-byte vector at head dim 16.
template <int D>
struct LaneRun {
  using T = u32x4;
  static constexpr int N = D / 32;
};
template <>
struct LaneRun<16> {
  using T = u32x2;
  static constexpr int N = 1;
};
template <int D>
using RunVec = typename LaneRun<D>::T;

template <int D>
struct PTile {
  RunVec<D> k[LaneRun<D>::N];
  RunVec<D> v[LaneRun<D>::N];
};

// Dwords 2c, 2c + 1 of a lane's run: the MFMA operand of contraction chunk c (K, q) or of
// M-tile c (V).
template <int D>
__device__ __forceinline__ u32x2 run_chunk(const RunVec<D> (&r)[LaneRun<D>::N], int c) {
  if constexpr (D == 16) {
    return r[0];
  } else {
    const u32x4 q = r[c >> 1];
    return (c & 1) ? u32x2{q.z, q.w} : u32x2{q.x, q.y};
  }
}

// S^T tile of 16 tokens x 16 heads from the lane's K and q runs.
template <class Ty, int D>
__device__ __forceinline__ f32x4 qk_run(const RunVec<D> (&k)[LaneRun<D>::N], const RunVec<D> (&q)[LaneRun<D>::N]) {
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < D / 16; ++c) s = Ty::mma(run_chunk<D>(k, c), run_chunk<D>(q, c), s);
  return s;
}

// Query head row at `qptr`, the lane's run of it (dims (D/4)g .. +D/4); zero for padding heads.
template <int D>
__device__ __forceinline__ void load_q_run(RunVec<D> (&q)[LaneRun<D>::N], const uint16_t* qptr, bool real, int g) {
#pragma unroll
  for (int i = 0; i < LaneRun<D>::N; ++i) q[i] = RunVec<D>{};
  if (real) {
    const RunVec<D>* p = reinterpret_cast<const RunVec<D>*>(qptr + (D / 4) * g);
#pragma unroll
    for (int i = 0; i < LaneRun<D>::N; ++i) q[i] = p[i];
  }
}

constexpr int kBufferFlags = 0x00020000;  // dword 3 of a raw buffer resource on gfx9

// One tile through a buffer resource: `r` covers one KV head of one record, `sk` / `sv` are the
// tile's K and V byte offsets (wave-uniform, in SGPRs), `k_lane` / `v_lane` the lane's offsets
// in them. Each load instruction covers every other 16 bytes of the tile's K (or V) bytes, the
// next instruction the rest. A resource with no records makes every load return zeros without
// a memory access.
template <int D>
__device__ __forceinline__ void load_tile_rs(PTile<D>& t, __amdgpu_buffer_rsrc_t r, uint32_t sk, uint32_t sv,
                                             uint32_t k_lane, uint32_t v_lane) {
  if constexpr (D == 16) {
    t.k[0] = __builtin_amdgcn_raw_buffer_load_b64(r, k_lane, sk, 0);
    t.v[0] = __builtin_amdgcn_raw_buffer_load_b64(r, v_lane, sv, 0);
  } else {
#pragma unroll
    for (int i = 0; i < D / 32; ++i) t.k[i] = __builtin_amdgcn_raw_buffer_load_b128(r, k_lane + 16u * i, sk, 0);
#pragma unroll
    for (int i = 0; i < D / 32; ++i) t.v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, v_lane + 16u * i, sv, 0);
  }
}

// O^T[D x 16 heads] += V^T . P^T with the transposed V tile.
template <class Ty, int D>
__device__ __forceinline__ void pv_tile_t(f32x4 (&acc)[D / 16], const PTile<D>& t, const float (&p)[4]) {
  const u32x2 pb = {Ty::pack(p[0], p[1]), Ty::pack(p[2], p[3])};
#pragma unroll
  for (int j = 0; j < D / 16; ++j) acc[j] = Ty::mma(run_chunk<D>(t.v, j), pb, acc[j]);
}

struct TileMeta {
  int t0;        // first token position of the tile
  int block_id;
  int last;      // last tile of its block
};

// Mirror mode: most reads of a layer's "mirror filled" word before a workgroup reads the host
// in place instead (s_sleep 127 between reads: ~8k cycles each, ~20 ms in all).
constexpr int kMirrorPolls = 6000;

template <int D>
struct PagedRing {
  // Register tiles per wave. At head dim 256 a tile is 64 VGPRs of K and V per lane (next to
  // 64 of accumulators and 32 of q), so two.
  static constexpr int NB = D == 256 ? 2 : 3;
};

// The three pointers the first loads depend on come as separate leading arguments: the build
// preloads leading kernel arguments into SGPRs, so a workgroup issues its work-item load
// without first loading the argument block (one dependent memory hop less at start-up).
template <class Ty, int D, bool kMass>
__global__ __launch_bounds__(256) void paged_attn_kernel(const WorkItem* __restrict__ work, uint16_t* pool,
                                                         const uint16_t* stage, PagedArgs a) {
  constexpr int NB = PagedRing<D>::NB;
  constexpr int kWaveEntries = kMaxWorkEntries / kWaves;  // entries one wave folds at most
  __shared__ MergeSmem<D> sm;
  __shared__ float mass_sm[kMass ? kWaves : 1][kWaveEntries][2][kMaxRep];
  const WorkItem* wi = work + blockIdx.x;
  const int h = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, n = lane & 15;
  const bool real = n < a.n_rep;
  const int qh = h * a.n_rep + (real ? n : 0);
  const int T = a.tokens_per_block;
  const int tpb = T >> 4;  // tiles per block
  const size_t rec = (size_t)2 * a.hkv * T * D;  // elements per record
  const size_t head_off = (size_t)h * T * D;
  const size_t v_off = (size_t)a.hkv * T * D;
  const int seq = wi->seq, hi = wi->hi, n_mass = wi->n_mass;
  // A layer with its own sliding window masks the stored positions <= hi - window as well
  // (hi is the current token's position); its blocks are read all the same.
  const int lo = a.window > 0 ? max(wi->lo, hi - a.window + 1) : wi->lo;
  const int count = wi->entry_count, partial = wi->partial;
  const int append_slot = wi->append_slot, append_pos = wi->append_pos;
  const uint32_t k_lane = (uint32_t)(n * D + (D / 4) * g) * 2u;
  const uint32_t v_lane = (uint32_t)lane * (D / 2);  // lane (g, n) = 16 g + n: its transposed V run

  if (a.work_out != nullptr) {
    // First launch of a step: `work` is the pinned plan buffer. This workgroup's work item
    // (head 0 only) and its share of the rest of the plan go to the device copy that every
    // later kernel of the step reads. Issued first, beside the scalar loads of the work item
    // that the first fetch waits for anyway.
    static_assert(sizeof(WorkItem) % 16 == 0, "work items copy as 16-byte vectors");
    constexpr int kItemVec = (int)(sizeof(WorkItem) / 16);
    if (h == 0 && (int)threadIdx.x < kItemVec)
      reinterpret_cast<u32x4*>(a.work_out + blockIdx.x)[threadIdx.x] = reinterpret_cast<const u32x4*>(wi)[threadIdx.x];
    const int64_t stride = (int64_t)gridDim.x * gridDim.y * blockDim.x;
    for (int64_t v = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; v < a.aux_vec;
         v += stride)
      static_cast<u32x4*>(a.aux_dst)[v] = static_cast<const u32x4*>(a.aux_src)[v];
  }

  // The work item's blocks hold count * tpb tiles, flat index x = entry * tpb + tile in
  // block. With per-block mass (kMass) wave w folds whole blocks: entries w, w+4, w+8, ...
  // (a block's mass is then one wave's). Otherwise it folds tiles x = w, w+4, w+8, ..., so
  // that the four waves' tile counts differ by at most one and no wave holds the workgroup
  // up by a whole block. The cursor (fe, ftb) names the next fetch's entry and tile in
  // block; the entry being fetched and the next one sit in SGPRs, and the one after is read
  // (a scalar load) as a fetch is issued, a fetch or a block ahead of its use. Entries past
  // entry_count are never read by a fetch (the slots exist in every work item).
  int fe = kMass ? 0 : wave / tpb, ftb = kMass ? 0 : wave - (wave / tpb) * tpb;
  const int step_e = kWaves / tpb, step_tb = kWaves - step_e * tpb;  // x += kWaves (no kMass)
  auto advance = [&](int& e, int& tb) {
    tb += step_tb;
    e += step_e;
    if (tb >= tpb) {
      tb -= tpb;
      ++e;
    }
  };
  auto entry_at = [&](int e) { return wi->entries[e < kMaxWorkEntries ? e : kMaxWorkEntries - 1]; };
  int ne = fe, ntb = ftb;  // the fetch after the next one
  if (!kMass) advance(ne, ntb);
  BlockEntry ecur = kMass ? wi->entries[wave] : entry_at(fe);
  BlockEntry enxt = kMass ? wi->entries[wave + kWaves] : entry_at(ne);

  // Mirror mode: host records come from the layer's HBM mirror, filled by DMA on the store's
  // copy stream, which sets the word after the layer's copies. One lane per workgroup polls
  // the word past the caches, sleeping between reads, for at most kMirrorPolls reads (~20 ms);
  // if it is still clear then, the workgroup reads the host in place (same data). The copies
  // do not depend on this launch, so the wait ends with them. A host record's data never
  // change while its session holds it, and the mirror is refilled only after the launches
  // of the step before have finished.
  const uint16_t* host_src = stage;
  int host_shift = 0;  // ring buffer record = host record - host_shift
  if (a.mirror_flag != nullptr) {
    __shared__ uint32_t mirror_ready;
    if (threadIdx.x == 0) {
      uint32_t f = __hip_atomic_load(a.mirror_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      for (int i = 0; f == 0u && i < kMirrorPolls; ++i) {
        __builtin_amdgcn_s_sleep(127);
        f = __hip_atomic_load(a.mirror_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      // The ring buffer held another layer's records when this launch started, and a cache
      // may still hold lines of them: a system-scope acquire (cache invalidate) orders the
      // workgroup's reads after the DMA copy that the word announces.
      if (f != 0u) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
      mirror_ready = f;
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(mirror_ready) != 0u) {
      host_src = a.mirror;
      host_shift = wi->mirror_off;
    }
  }

  RunVec<D> q[LaneRun<D>::N];  // loaded behind the first tile (below)

  // Score transform: x = mult * s' with s' = s (no softcap) or cap * tanh(s * scale / cap).
  const bool capped = a.softcap > 0.f;
  const float mult = capped ? kLog2e : a.scale * kLog2e;
  const float cap_in = capped ? a.scale / a.softcap : 0.f;

  float m_run = kMInit, m_thr = kMInit, l_run = 0.f, blk = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int my_blocks = count > wave ? (count - wave + kWaves - 1) / kWaves : 0;
  const int tiles = kMass ? my_blocks * tpb : (count * tpb > wave ? (count * tpb - wave + kWaves - 1) / kWaves : 0);

  // Next tile to fetch: the wave's nf-th. Every fetch in the loop is unconditional, so the
  // load counter stays in order; a fetch past the wave's last tile goes through an empty
  // buffer resource and returns at once with zeros.
  int nf = 0;
  auto fetch = [&](PTile<D>& t, TileMeta& mt) {
    const int slot = ecur.slot, bid = ecur.block_id;
    const uint16_t* rb =
        slot >= 0 ? pool + (size_t)slot * rec : host_src + (size_t)((-slot - 1) - host_shift) * rec;
    // A tile with no token in [lo, hi) (below a layer's own sliding window, or past the
    // current token in the open block) is fully masked: its loads go through an empty
    // resource and return zeros without a memory access, as past the wave's last tile.
    const int tt0 = bid * T + ftb * 16;
    const bool read = nf < tiles && tt0 + 16 > lo && tt0 < hi;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)(rb + head_off), (short)0, read ? 0x7fffffff : 0, kBufferFlags);
    const uint32_t sk = (uint32_t)(ftb * 16 * D * 2);
    load_tile_rs<D>(t, r, sk, sk + (uint32_t)(v_off * 2), k_lane, v_lane);
    mt.t0 = tt0;
    mt.block_id = bid;
    mt.last = (ftb == tpb - 1) ? fe : -1;
    ++nf;
    if constexpr (kMass) {
      if (++ftb == tpb) {
        ftb = 0;
        ++fe;
        ecur = enxt;
        if (fe + 1 < kWaveEntries) enxt = wi->entries[wave + (fe + 1) * kWaves];
      }
    } else {
      fe = ne;
      ftb = ntb;
      ecur = enxt;
      advance(ne, ntb);
      enxt = entry_at(ne);
    }
  };

  auto fold = [&](PTile<D>& t, const TileMeta& mt) {
    f32x4 s4 = qk_run<Ty, D>(t.k, q);
    if (capped) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s4[i] = a.softcap * tanhf(s4[i] * cap_in);
    }
    if (mt.t0 < lo || mt.t0 + 16 > hi) {  // tile straddles the valid range: mask per token
      // Token 4g + i of the lane's V operands is 16-bit half (i & 1) of dwords x / z (i < 2)
      // or y / w (i >= 2): a masked token's V is zeroed, so stale record bytes never reach P.V.
      uint32_t mx = 0xffffffffu, my = 0xffffffffu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = mt.t0 + 4 * g + i;
        if (tok < lo || tok >= hi) {
          s4[i] = kNegInf;
          const uint32_t keep = (i & 1) ? 0x0000ffffu : 0xffff0000u;
          if (i < 2)
            mx &= keep;
          else
            my &= keep;
        }
      }
      if constexpr (D == 16) {
        t.v[0] &= u32x2{mx, my};
      } else {
#pragma unroll
        for (int w = 0; w < D / 32; ++w) t.v[w] &= u32x4{mx, my, mx, my};
      }
    }
    const float lmax = fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3])) * mult;
    if (__builtin_amdgcn_ballot_w64(lmax > m_thr) != 0) {
      const float m_new = fmaxf(m_run, wave_max_g(lmax));
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      blk *= alpha;
#pragma unroll
      for (int j = 0; j < D / 16; ++j) acc[j] *= alpha;
      m_run = m_new;
      m_thr = m_new + kLazyRescale;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s4[i], mult, -m_run));
    const float psum = (p[0] + p[1]) + (p[2] + p[3]);
    l_run += psum;
    pv_tile_t<Ty, D>(acc, t, p);
    if constexpr (kMass) {
      blk += psum;
      if (mt.last >= 0) {  // block complete: (m_b, s_b) of this block to LDS, stored after the loop
        const float bs = wave_sum_g(blk);
        if (g == 0) {
          mass_sm[wave][mt.last][0][n] = m_run;
          mass_sm[wave][mt.last][1][n] = bs;
        }
        blk = 0.f;
      }
    }
  };

  if (tiles > 0) {
    PTile<D> buf[NB];
    TileMeta meta[NB];
    // Tile 0, then q, then the rest of the prologue: q is needed by the first fold, and
    // waiting for it here (which also waits for tile 0, as loads return in order) keeps
    // the loop's wait counts independent of it while tiles 1 .. NB-2 stay in flight.
    fetch(buf[0], meta[0]);
    load_q_run<D>(q, a.q + ((size_t)seq * a.hq + qh) * D, real, g);
#pragma unroll
    for (int j = 1; j < NB - 1; ++j) fetch(buf[j], meta[j]);
#pragma unroll
    for (int i = 0; i < LaneRun<D>::N; ++i) asm volatile("" ::"v"(q[i]));
    for (int ti = 0; ti < tiles; ti += NB) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        fetch(buf[(j + NB - 1) % NB], meta[(j + NB - 1) % NB]);
        if (ti + j < tiles) fold(buf[j], meta[j]);
      }
    }
  }
  if constexpr (kMass) {
    if (g == 0 && real) {
      for (int e = 0; e < my_blocks; ++e) {
        const int bid = wi->entries[wave + e * kWaves].block_id;
        if (bid < n_mass) {
          const size_t mi = ((size_t)seq * a.hq + qh) * a.mass_stride + bid;
          a.mass_m[mi] = mass_sm[wave][e][0][n];
          a.mass_s[mi] = mass_sm[wave][e][1][n];
        }
      }
    }
  }

  // Append (one work item per sequence): the current token's K/V of this head into its
  // block record. No workgroup of this launch reads that position (work covers [lo, hi)).
  if (append_slot >= 0 && threadIdx.x < D) {
    const size_t src = ((size_t)seq * a.hkv + h) * D + threadIdx.x;
    uint16_t* rec_base = pool + (size_t)append_slot * rec;
    rec_base[head_off + (size_t)append_pos * D + threadIdx.x] = a.k_new[src];
    rec_base[v_off + v_record_index(h, append_pos, threadIdx.x, T, D)] = a.v_new[src];
  }

  const size_t slot = (size_t)partial;
  const float m_out = m_run == kMInit ? kNegInf : m_run;
  wg_merge_store<D, true, true, true>(sm, wave, g, n, m_out, l_run, acc, a.n_rep, a.pm + slot * a.hq + h * a.n_rep,
                                      a.pl + slot * a.hq + h * a.n_rep, a.pacc + (slot * a.hq + h * a.n_rep) * D);
}

// ---------------------------------------------------------------------------------------
// Split-K merge: one workgroup per (sequence, query head). Thread (g, c) owns output dims
// 2c, 2c+1 and merges the partial slots g, g+G, g+2G, ... online (running max, rescaled
// sums), G = 512 / D thread groups; the groups are then combined through LDS together with
// the current token (score q.k_new, weight 2^(x - m), P rounded like every other P), and the
// output and the final (m, l) for the mass pass are written. The kernel is latency-bound:
// each thread issues a whole batch of partial loads before using any of them (a load past
// the last partial re-reads it and is weighted 0).
constexpr int kMergeBatch = 16;

// The leading arguments are preloaded into SGPRs (as in paged_attn_kernel): the partial loads
// of the first batch depend on nothing else, and go out before the plan's SeqInfo arrives.
template <class Ty, int D>
__global__ __launch_bounds__(256) void paged_merge_kernel(const SeqInfo* __restrict__ seqs, const float* pm0,
                                                          const float* pl0, const float* pacc0,
                                                          int partial_stride, int hq, int n_rep, int hkv,
                                                          PagedArgs a) {
  constexpr int kLanes = D / 2;          // threads per partial group (two dims each)
  constexpr int G = 256 / kLanes;        // partial groups
  constexpr int kU = kMergeBatch;
  constexpr int kRed = kLanes < kWaveSize ? kLanes : kWaveSize;  // lanes of group 0 per wave
  __shared__ float m_s[G], l_s[G];
  __shared__ float acc_s[G][D];
  __shared__ float dot_s[kLanes / kRed];
  const int seq = blockIdx.x, qh = blockIdx.y;
  const int tid = threadIdx.x;
  const int c = tid % kLanes, grp = tid / kLanes;
  const SeqInfo* si = seqs + seq;
  const size_t stride_a = (size_t)hq * D;
  const float *pm, *pl, *pa;  // this (sequence, head)'s first slot
  auto set_base = [&](int base) {
    pm = pm0 + (size_t)base * hq + qh;
    pl = pl0 + (size_t)base * hq + qh;
    pa = pacc0 + ((size_t)base * hq + qh) * D + 2 * c;
  };
  // A batch: slots p0, p0 + G, ... (kU of them), clamped to limit - 1, every load issued
  // before any is used. A slot at or past P (not written this step, or re-read) gets weight
  // 0 in the fold: its m is -inf and its l and acc are zeroed, not multiplied, since an
  // unwritten slot may hold anything.
  auto load_batch = [&](int p0, int limit, float (&xm)[kU], float (&xl)[kU], float2 (&xa)[kU]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int p = min(p0 + G * u, limit - 1);
      xm[u] = pm[(size_t)p * hq];
      xl[u] = pl[(size_t)p * hq];
      xa[u] = *reinterpret_cast<const float2*>(pa + (size_t)p * stride_a);
    }
  };
  float xm0[kU], xl0[kU];
  float2 xa0[kU];
  if (partial_stride > 0) {
    // Sequence s owns slots s * partial_stride .. + partial_stride - 1: the first batch
    // depends on the preloaded arguments only, and its loads go out before the plan's
    // SeqInfo (P, the flags' token) and the current token's operands are read.
    set_base(seq * partial_stride);
    load_batch(grp, partial_stride, xm0, xl0, xa0);
  } else {
    // Packed slots (a step whose sequences' work-item counts differ too much for fixed
    // ranges): the first slot and the count come from the sequence's SeqInfo.
    set_base(si->partial_base);
    load_batch(grp, si->partial_count, xm0, xl0, xa0);
  }

  const int P = si->partial_count;  // P >= 1: every sequence has a work item
  const int h = qh / n_rep;
  const size_t kv_row = ((size_t)seq * hkv + h) * D;
  if (seq == 0 && qh == 0 && tid == 0) {
    // The attention launches before this merge have finished: tell the host that the step's
    // plan buffer is free (a system-scope vector store into pinned host memory).
    if (a.plan_flag != nullptr)
      __hip_atomic_store(a.plan_flag, a.plan_token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    // Mirror mode: the layer's attention launch has finished reading its ring buffer; the
    // host may queue the next copies into it once this word holds the step's token.
    if (a.release_flag != nullptr)
      __hip_atomic_store(a.release_flag, si->step_token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }

  // Group 0 also computes the current token's score (its loads overlap the partial loads).
  uint32_t qd = 0, kd = 0, vd = 0;
  if (grp == 0) {
    qd = *reinterpret_cast<const uint32_t*>(a.q + ((size_t)seq * hq + qh) * D + 2 * c);
    kd = *reinterpret_cast<const uint32_t*>(a.k_new + kv_row + 2 * c);
    vd = *reinterpret_cast<const uint32_t*>(a.v_new + kv_row + 2 * c);
  }

  float m = kNegInf, l = 0.f;
  float2 acc = float2{0.f, 0.f};
  auto fold_batch = [&](int p0, float (&xm)[kU], float (&xl)[kU], float2 (&xa)[kU]) {
    float bmax = kNegInf;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (p0 + G * u >= P) {
        xm[u] = kNegInf;
        xl[u] = 0.f;
        xa[u] = float2{0.f, 0.f};
      }
      bmax = fmaxf(bmax, xm[u]);
    }
    const float m_new = fmaxf(m, bmax);
    const float mm = m_new == kNegInf ? 0.f : m_new;  // nothing valid yet: every weight is 0
    const float alpha = __builtin_amdgcn_exp2f(m - mm);
    l *= alpha;
    acc.x *= alpha;
    acc.y *= alpha;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const float w = __builtin_amdgcn_exp2f(xm[u] - mm);
      l += xl[u] * w;
      acc.x += xa[u].x * w;
      acc.y += xa[u].y * w;
    }
    m = m_new;
  };
  fold_batch(grp, xm0, xl0, xa0);
  for (int p0 = grp + G * kU; p0 < P; p0 += G * kU) {  // P > G * kU slots: later batches clamp to P
    float xm[kU], xl[kU];
    float2 xa[kU];
    load_batch(p0, P, xm, xl, xa);
    fold_batch(p0, xm, xl, xa);
  }
  // q . k_new: group 0's two-dim products, summed over its lanes in each wave (every lane
  // takes part in the shuffles; group 0 is aligned to kRed lanes), then over its waves.
  float dot = 0.f;
  if (grp == 0)
    dot = Ty::to_f((uint16_t)(qd & 0xffffu)) * Ty::to_f((uint16_t)(kd & 0xffffu)) +
          Ty::to_f((uint16_t)(qd >> 16)) * Ty::to_f((uint16_t)(kd >> 16));
#pragma unroll
  for (int o = kRed / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
  if (grp == 0 && c % kRed == 0) dot_s[c / kRed] = dot;
  if (c == 0) {
    m_s[grp] = m;
    l_s[grp] = l;
  }
  acc_s[grp][2 * c] = acc.x;
  acc_s[grp][2 * c + 1] = acc.y;
  __syncthreads();
  __shared__ float fin_s[2];  // final (m, l) of this (sequence, head), for the block weights
  if (grp == 0) {
    dot = dot_s[0];
#pragma unroll
    for (int w = 1; w < kLanes / kRed; ++w) dot += dot_s[w];
    float x_cur;
    if (a.softcap > 0.f)
      x_cur = a.softcap * tanhf(dot * (a.scale / a.softcap)) * kLog2e;
    else
      x_cur = dot * (a.scale * kLog2e);
    float mf = x_cur;  // the current token is always valid: mf is finite
#pragma unroll
    for (int g2 = 0; g2 < G; ++g2) mf = fmaxf(mf, m_s[g2]);
    const float pc = __builtin_amdgcn_exp2f(x_cur - mf);
    const float pcr = Ty::to_f(Ty::cvt(pc));  // P rounded to the K/V type before P.V
    float lf = pc;
    float o0 = pcr * Ty::to_f((uint16_t)(vd & 0xffffu));
    float o1 = pcr * Ty::to_f((uint16_t)(vd >> 16));
#pragma unroll
    for (int g2 = 0; g2 < G; ++g2) {
      const float w = __builtin_amdgcn_exp2f(m_s[g2] - mf);  // empty group: m = -inf, w = 0
      lf += l_s[g2] * w;
      o0 += acc_s[g2][2 * c] * w;
      o1 += acc_s[g2][2 * c + 1] * w;
    }
    const uint32_t packed = (uint32_t)Ty::cvt(o0 / lf) | ((uint32_t)Ty::cvt(o1 / lf) << 16);
    *reinterpret_cast<uint32_t*>(a.out + ((size_t)seq * hq + qh) * D + 2 * c) = packed;
    if (c == 0) {
      a.mf[(size_t)seq * hq + qh] = mf;
      a.lf[(size_t)seq * hq + qh] = lf;
      fin_s[0] = mf;
      fin_s[1] = lf;
    }
  }
  if (a.mass_w == nullptr) return;
  // Deferred mass: the weight of every in-scope block of this (sequence, head) under the
  // final (m, l), s_b * 2^(m_b - m_f) / l_f (l_f > 0: the current token always counts), by
  // all threads. Blocks below mass_lo keep the 0 the last step's reduction left.
  __syncthreads();
  const float mfin = fin_s[0], lfin = fin_s[1];
  const size_t row = (size_t)seq * hq + qh;
  const int n_mass = si->n_mass;
  for (int b = si->mass_lo + tid; b < n_mass; b += 256) {
    const size_t mi = row * a.mass_stride + b;
    a.mass_w[mi] = a.mass_s[mi] * __builtin_amdgcn_exp2f(a.mass_m[mi] - mfin) / lfin;
  }
}

// Per (session, block): mean over the session's rows and all query heads of
// s_b * 2^(m_b - m_final) / l_final (log2 units), added into the session's mass accumulator
// (paged_model.py:1041-1048 per layer).
// Per-block attention mass of each session, averaged over its rows and query heads and added
// to mass_accum (one layer's share). Block b of row r, head h contributes
// s_b * 2^(m_b - m_final) / l_final. Workgroup: 64 blocks x 4 head groups; each thread sums
// its heads h = g, g + 4, ... (loads unrolled so they overlap), then the four groups are
// added through LDS in a fixed order, so the result does not depend on scheduling.
constexpr int kMassBlocksPerWG = 64;
constexpr int kMassHeadGroups = 4;

__global__ __launch_bounds__(256) void mass_reduce_kernel(const SeqInfo* seqs, const int32_t* session_rows,
                                                          const int32_t* session_first, const float* mass_m,
                                                          const float* mass_s, const float* mf, const float* lf,
                                                          float* mass_accum, int accum_stride, int hq, int mass_stride,
                                                          int n_sessions, int max_blocks) {
  __shared__ float part[kMassHeadGroups][kMassBlocksPerWG];
  const int sess = blockIdx.y;
  const int bl = threadIdx.x % kMassBlocksPerWG, hg = threadIdx.x / kMassBlocksPerWG;
  const int blk = blockIdx.x * kMassBlocksPerWG + bl;
  const int first = session_first[sess], rows = session_rows[sess];
  const int n_mass = seqs[first].n_mass;
  const bool live = blk < n_mass && blk < max_blocks;
  float total = 0.f;
  if (live) {
    for (int r = 0; r < rows; ++r) {
      if (blk < seqs[first + r].mass_lo) continue;  // out of scope for this row: mass 0
      const size_t row0 = (size_t)(first + r) * hq;
#pragma unroll 4
      for (int qh = hg; qh < hq; qh += kMassHeadGroups) {
        const size_t row = row0 + qh;
        const float l = lf[row];
        const size_t mi = row * mass_stride + blk;
        if (l > 0.f) total += mass_s[mi] * __builtin_amdgcn_exp2f(mass_m[mi] - mf[row]) / l;
      }
    }
  }
  part[hg][bl] = total;
  __syncthreads();
  if (hg == 0 && live) {
    const float sum = ((part[0][bl] + part[1][bl]) + part[2][bl]) + part[3][bl];
    mass_accum[(size_t)sess * accum_stride + blk] += sum / (float)(rows * hq);
  }
}

// Deferred mass, once per step (see launch_mass_step_reduce). Workgroup: 16 blocks x 16 head
// groups. For a pass of up to 32 layers every thread adds up its heads (h = g, g + 16, ...) of
// its block per layer in LDS, 8 layers x 4 heads of loads in flight at a time, and clears what
// it read; then one thread per (layer, block) adds the 16 groups in a fixed order, and one
// thread per block adds the layers up in layer order, so the result does not depend on
// scheduling.
constexpr int kStepMassBlocks = 16;
constexpr int kStepMassGroups = 16;
constexpr int kStepMassLayers = 32;  // layers per pass through LDS
constexpr int kStepMassUnrollL = 8;  // layers whose loads one thread has in flight together
constexpr int kStepMassUnrollH = 4;  // heads per group and layer loaded together (hq <= 64)

__global__ __launch_bounds__(256) void mass_step_reduce_kernel(const SeqInfo* seqs, const int32_t* session_rows,
                                                               const int32_t* session_first, float* mass_w,
                                                               int64_t layer_floats, int num_layers,
                                                               float* mass_accum, int accum_stride, int hq,
                                                               int mass_stride, int max_blocks) {
  __shared__ float part[kStepMassLayers][kStepMassGroups][kStepMassBlocks];
  __shared__ float layer_sum[kStepMassLayers][kStepMassBlocks];
  const int sess = blockIdx.y;
  const int bl = threadIdx.x % kStepMassBlocks, hg = threadIdx.x / kStepMassBlocks;
  const int blk = blockIdx.x * kStepMassBlocks + bl;
  const int first = session_first[sess], rows = session_rows[sess];
  const int n_mass = seqs[first].n_mass;
  const bool live = blk < n_mass && blk < max_blocks;
  const float denom = (float)(rows * hq);
  float acc = 0.f;
  if (hg == 0 && live) acc = mass_accum[(size_t)sess * accum_stride + blk];
  for (int l0 = 0; l0 < num_layers; l0 += kStepMassLayers) {
    const int nl = min(kStepMassLayers, num_layers - l0);
    for (int li = 0; li < nl; ++li) part[li][hg][bl] = 0.f;
    for (int r = 0; live && r < rows; ++r) {
      if (blk < seqs[first + r].mass_lo) continue;  // out of scope for this row: mass 0
      float* wr = mass_w + (size_t)l0 * layer_floats + ((size_t)(first + r) * hq + hg) * mass_stride + blk;
      for (int qh0 = hg; qh0 < hq; qh0 += kStepMassGroups * kStepMassUnrollH) {
        for (int li0 = 0; li0 < nl; li0 += kStepMassUnrollL) {
          float x[kStepMassUnrollL][kStepMassUnrollH];
#pragma unroll
          for (int u = 0; u < kStepMassUnrollL; ++u)
#pragma unroll
            for (int k = 0; k < kStepMassUnrollH; ++k) {
              const bool in = li0 + u < nl && qh0 + k * kStepMassGroups < hq;
              const size_t at = (size_t)(li0 + u) * layer_floats +
                                (size_t)(qh0 - hg + k * kStepMassGroups) * mass_stride;
              x[u][k] = in ? wr[at] : 0.f;
            }
#pragma unroll
          for (int u = 0; u < kStepMassUnrollL; ++u)
#pragma unroll
            for (int k = 0; k < kStepMassUnrollH; ++k) {
              if (li0 + u < nl && qh0 + k * kStepMassGroups < hq) {
                wr[(size_t)(li0 + u) * layer_floats + (size_t)(qh0 - hg + k * kStepMassGroups) * mass_stride] = 0.f;
                part[li0 + u][hg][bl] += x[u][k];  // heads in ascending order
              }
            }
        }
      }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < nl * kStepMassBlocks; t += blockDim.x) {
      const int li = t / kStepMassBlocks, b = t % kStepMassBlocks;
      float sum = 0.f;
#pragma unroll
      for (int g = 0; g < kStepMassGroups; ++g) sum += part[li][g][b];
      layer_sum[li][b] = sum;
    }
    __syncthreads();
    if (hg == 0 && live)
      for (int li = 0; li < nl; ++li) acc += layer_sum[li][bl] / denom;
    __syncthreads();
  }
  if (hg == 0 && live) mass_accum[(size_t)sess * accum_stride + blk] = acc;
}

hipError_t launch_dense_merge(const DenseArgs& a, int mode, int batch, int d, float* m, float* l, float* acc,
                              hipStream_t stream) {
  dim3 mgrid(batch * a.hq);
  switch (mode) {
    case kModeFold:
      dense_merge_kernel<kModeFold><<<mgrid, kDenseMergeThreads, 0, stream>>>(a, m, l, acc, d);
      break;
    case kModeStats:
      dense_merge_kernel<kModeStats><<<mgrid, kDenseMergeThreads, 0, stream>>>(a, m, l, acc, d);
      break;
    default:
      dense_merge_kernel<kModeAccumulate><<<mgrid, kDenseMergeThreads, 0, stream>>>(a, m, l, acc, d);
      break;
  }
  return hipGetLastError();
}

template <class Ty, int D>
hipError_t launch_dense_t(const DenseArgs& a, int mode, int batch, hipStream_t stream) {
  dim3 grid(a.n_split, a.hkv, batch);
  switch (mode) {
    case kModeFold:
      dense_attn_kernel<Ty, D, kModeFold><<<grid, 256, 0, stream>>>(a);
      break;
    case kModeStats:
      dense_attn_kernel<Ty, D, kModeStats><<<grid, 256, 0, stream>>>(a);
      break;
    case kModeAccumulate:
      dense_attn_kernel<Ty, D, kModeAccumulate><<<grid, 256, 0, stream>>>(a);
      break;
    default:
      dense_attn_kernel<Ty, D, kModeFoldFixed><<<grid, 256, 0, stream>>>(a);
      break;
  }
  return hipGetLastError();
}

template <class Ty>
hipError_t launch_dense_ty(const DenseArgs& a, int mode, int batch, int d, hipStream_t stream) {
  switch (d) {
    case 32:
      return launch_dense_t<Ty, 32>(a, mode, batch, stream);
    case 64:
      return launch_dense_t<Ty, 64>(a, mode, batch, stream);
    default:
      return launch_dense_t<Ty, 128>(a, mode, batch, stream);
  }
}

template <class E, int D>
hipError_t launch_generic_t(const DenseArgs& a, int mode, int batch, hipStream_t stream) {
  dim3 grid(a.n_split, a.hkv, batch);
  switch (mode) {
    case kModeFold:
      dense_generic_kernel<E, D, kModeFold><<<grid, 64, 0, stream>>>(a);
      break;
    case kModeStats:
      dense_generic_kernel<E, D, kModeStats><<<grid, 64, 0, stream>>>(a);
      break;
    case kModeAccumulate:
      dense_generic_kernel<E, D, kModeAccumulate><<<grid, 64, 0, stream>>>(a);
      break;
    default:
      dense_generic_kernel<E, D, kModeFoldFixed><<<grid, 64, 0, stream>>>(a);
      break;
  }
  return hipGetLastError();
}

// 16-bit q/k/v at the head dims the MFMA kernel does not take.
template <class Ty>
hipError_t launch_generic_16(const DenseArgs& a, int mode, int batch, int d, hipStream_t stream) {
  switch (d) {
    case 8:
      return launch_generic_t<GenElem<Ty>, 8>(a, mode, batch, stream);
    case 16:
      return launch_generic_t<GenElem<Ty>, 16>(a, mode, batch, stream);
    default:
      return launch_generic_t<GenElem<Ty>, 256>(a, mode, batch, stream);
  }
}

hipError_t launch_generic_32(const DenseArgs& a, int mode, int batch, int d, hipStream_t stream) {
  switch (d) {
    case 8:
      return launch_generic_t<F32Elem, 8>(a, mode, batch, stream);
    case 16:
      return launch_generic_t<F32Elem, 16>(a, mode, batch, stream);
    case 32:
      return launch_generic_t<F32Elem, 32>(a, mode, batch, stream);
    case 64:
      return launch_generic_t<F32Elem, 64>(a, mode, batch, stream);
    case 128:
      return launch_generic_t<F32Elem, 128>(a, mode, batch, stream);
    default:
      return launch_generic_t<F32Elem, 256>(a, mode, batch, stream);
  }
}

template <class Ty, int D>
hipError_t launch_paged_t(const PagedArgs& a, int n_work, bool mass, hipStream_t stream) {
  dim3 grid(n_work, a.hkv);
  if (mass) {
    paged_attn_kernel<Ty, D, true><<<grid, 256, 0, stream>>>(a.work, a.pool, a.stage, a);
  } else {
    paged_attn_kernel<Ty, D, false><<<grid, 256, 0, stream>>>(a.work, a.pool, a.stage, a);
  }
  return hipGetLastError();
}

template <class Ty>
hipError_t launch_paged_d(const PagedArgs& a, int d, int n_work, bool mass, hipStream_t stream) {
  switch (d) {
    case 16:
      return launch_paged_t<Ty, 16>(a, n_work, mass, stream);
    case 32:
      return launch_paged_t<Ty, 32>(a, n_work, mass, stream);
    case 64:
      return launch_paged_t<Ty, 64>(a, n_work, mass, stream);
    case 128:
      return launch_paged_t<Ty, 128>(a, n_work, mass, stream);
    default:
      return launch_paged_t<Ty, 256>(a, n_work, mass, stream);
  }
}

template <class Ty>
void launch_merge_d(const PagedArgs& a, int stride, int d, dim3 grid, hipStream_t stream) {
  switch (d) {
    case 16:
      paged_merge_kernel<Ty, 16><<<grid, 256, 0, stream>>>(a.seqs, a.pm, a.pl, a.pacc, stride, a.hq, a.n_rep, a.hkv, a);
      break;
    case 32:
      paged_merge_kernel<Ty, 32><<<grid, 256, 0, stream>>>(a.seqs, a.pm, a.pl, a.pacc, stride, a.hq, a.n_rep, a.hkv, a);
      break;
    case 64:
      paged_merge_kernel<Ty, 64><<<grid, 256, 0, stream>>>(a.seqs, a.pm, a.pl, a.pacc, stride, a.hq, a.n_rep, a.hkv, a);
      break;
    case 128:
      paged_merge_kernel<Ty, 128><<<grid, 256, 0, stream>>>(a.seqs, a.pm, a.pl, a.pacc, stride, a.hq, a.n_rep, a.hkv, a);
      break;
    default:
      paged_merge_kernel<Ty, 256><<<grid, 256, 0, stream>>>(a.seqs, a.pm, a.pl, a.pacc, stride, a.hq, a.n_rep, a.hkv, a);
  }
}

}  // namespace

bool head_dim_supported(int d) { return d == 32 || d == 64 || d == 128; }

bool paged_head_dim_supported(int d) { return d == 16 || head_dim_supported(d) || d == 256; }

bool dense_head_dim_supported(int d) { return d == 8 || d == 16 || head_dim_supported(d) || d == 256; }

bool dense_generic(int dtype, int d) { return dtype == kF32 || !head_dim_supported(d); }

int dense_waves_per_workgroup(int dtype, int d) { return dense_generic(dtype, d) ? 1 : kWaves; }

int dense_wave_tokens(int dtype, int d, int batch, int hkv, int tc, int tokens_per_block, bool mass) {
  // Aim for about 2048 waves over the grid (8 per CU; 1024 one-wave workgroups for the
  // generic kernel), each folding at least one tile (16 tokens in the MFMA kernel, 64 in the
  // generic one).
  const bool gen = dense_generic(dtype, d);
  const long tile = gen ? kGenTile : 16;
  const long target = gen ? 1024 : 2048;
  const long tiles = (tc + tile - 1) / tile;
  const long rows = (long)batch * hkv;
  long per_wave = (tiles * rows + target - 1) / target;
  if (per_wave < 1) per_wave = 1;
  long tokens = per_wave * tile;
  if (mass) {
    const long tpb = tokens_per_block;
    tokens = (tokens + tpb - 1) / tpb * tpb;
  }
  return (int)tokens;
}

hipError_t launch_dense(int dtype, int mode, int d, const DenseLaunch& p, hipStream_t stream) {
  DenseArgs a;
  a.q = static_cast<const uint16_t*>(p.q);
  a.k = static_cast<const uint16_t*>(p.k);
  a.v = static_cast<const uint16_t*>(p.v);
  a.valid = p.valid;
  a.active = p.active;
  a.m_in = p.m;
  a.l_in = p.l;
  a.block_mass = p.block_mass;
  a.pm = p.pm;
  a.pl = p.pl;
  a.pacc = p.pacc;
  a.tc = p.tc;
  a.hq = p.hq;
  a.hkv = p.hkv;
  a.n_rep = p.hq / p.hkv;
  a.wave_tokens = p.wave_tokens;
  a.n_split = p.n_split;
  a.tokens_per_block = p.tokens_per_block;
  a.max_blocks = p.max_blocks;
  a.block_id_offset = p.block_id_offset;
  a.scale = p.scale;
  a.softcap = p.softcap;
  hipError_t e;
  if (p.ev_start != nullptr && (e = hipEventRecord(p.ev_start, stream)) != hipSuccess) return e;
  if (dtype == kF32)
    e = launch_generic_32(a, mode, p.batch, d, stream);
  else if (!head_dim_supported(d))
    e = dtype == kF16 ? launch_generic_16<F16>(a, mode, p.batch, d, stream)
                      : launch_generic_16<BF16>(a, mode, p.batch, d, stream);
  else
    e = dtype == kF16 ? launch_dense_ty<F16>(a, mode, p.batch, d, stream)
                      : launch_dense_ty<BF16>(a, mode, p.batch, d, stream);
  if (e != hipSuccess) return e;
  if (p.ev_stop != nullptr && (e = hipEventRecord(p.ev_stop, stream)) != hipSuccess) return e;
  if (p.attention_only) return hipSuccess;
  return launch_dense_merge(a, mode, p.batch, d, p.m, p.l, p.acc, stream);
}

hipError_t launch_finalize(int dtype, const float* acc, const float* l, void* out, int rows, int d,
                           hipStream_t stream) {
  const size_t total = (size_t)rows * d;
  if (total == 0) return hipSuccess;
  const int threads = 256;
  const unsigned blocks = (unsigned)((total + threads - 1) / threads);
  if (dtype == kF16)
    finalize_kernel<F16><<<blocks, threads, 0, stream>>>(acc, l, static_cast<uint16_t*>(out), rows, d);
  else if (dtype == kBF16)
    finalize_kernel<BF16><<<blocks, threads, 0, stream>>>(acc, l, static_cast<uint16_t*>(out), rows, d);
  else
    finalize_f32_kernel<<<blocks, threads, 0, stream>>>(acc, l, static_cast<float*>(out), rows, d);
  return hipGetLastError();
}

hipError_t launch_state_init(float* m, float* l, float* acc, int64_t rows, int64_t d, hipStream_t stream) {
  const int64_t n_acc = rows * d;  // >= rows: d >= 1
  if (n_acc == 0) return hipSuccess;
  const int threads = 256;
  const int64_t want = (n_acc + threads - 1) / threads;
  const unsigned blocks = (unsigned)(want < 4096 ? want : 4096);
  state_init_kernel<<<blocks, threads, 0, stream>>>(m, l, acc, rows, n_acc);
  return hipGetLastError();
}

hipError_t launch_paged(int dtype, int d, const PagedLaunch& p, hipStream_t stream) {
  if (p.n_work == 0) return hipSuccess;
  PagedArgs a{};
  a.q = static_cast<const uint16_t*>(p.q);
  a.k_new = static_cast<const uint16_t*>(p.k_new);
  a.v_new = static_cast<const uint16_t*>(p.v_new);
  a.pool = static_cast<uint16_t*>(p.pool);
  a.stage = static_cast<const uint16_t*>(p.stage);
  a.work = p.work;
  a.work_out = p.work_out;
  a.aux_src = p.aux_src;
  a.aux_dst = p.aux_dst;
  a.aux_vec = p.aux_vec;
  a.seqs = p.seqs;
  a.pm = p.pm;
  a.pl = p.pl;
  a.pacc = p.pacc;
  a.mass_m = p.mass_m;
  a.mass_s = p.mass_s;
  a.out = static_cast<uint16_t*>(p.out);
  a.mf = p.mf;
  a.lf = p.lf;
  a.hq = p.hq;
  a.hkv = p.hkv;
  a.n_rep = p.hq / p.hkv;
  a.tokens_per_block = p.tokens_per_block;
  a.mass_stride = p.mass_stride;
  a.scale = p.scale;
  a.softcap = p.softcap;
  a.window = p.window;
  a.mirror = static_cast<const uint16_t*>(p.mirror);
  a.mirror_flag = p.mirror_flag;
  const bool mass = p.mass_m != nullptr;
  return dtype == kF16 ? launch_paged_d<F16>(a, d, p.n_work, mass, stream)
                       : launch_paged_d<BF16>(a, d, p.n_work, mass, stream);
}

hipError_t launch_paged_merge(int dtype, int d, const PagedLaunch& p, int n_seq, hipStream_t stream) {
  if (n_seq == 0) return hipSuccess;
  PagedArgs a{};
  a.q = static_cast<const uint16_t*>(p.q);
  a.k_new = static_cast<const uint16_t*>(p.k_new);
  a.v_new = static_cast<const uint16_t*>(p.v_new);
  a.seqs = p.seqs;
  a.pm = p.pm;
  a.pl = p.pl;
  a.pacc = p.pacc;
  a.out = static_cast<uint16_t*>(p.out);
  a.mf = p.mf;
  a.lf = p.lf;
  a.hq = p.hq;
  a.hkv = p.hkv;
  a.n_rep = p.hq / p.hkv;
  a.scale = p.scale;
  a.softcap = p.softcap;
  a.plan_flag = p.plan_flag;
  a.plan_token = p.plan_token;
  a.release_flag = p.release_flag;
  a.mass_w = p.mass_w;
  a.mass_m = p.mass_m;
  a.mass_s = p.mass_s;
  a.mass_stride = p.mass_stride;
  dim3 grid(n_seq, p.hq);
  if (dtype == kF16)
    launch_merge_d<F16>(a, p.partial_stride, d, grid, stream);
  else
    launch_merge_d<BF16>(a, p.partial_stride, d, grid, stream);
  return hipGetLastError();
}

hipError_t launch_mass_reduce(const SeqInfo* seqs, const int32_t* session_rows, const int32_t* session_first,
                              const float* mass_m, const float* mass_s, const float* mf, const float* lf,
                              float* mass_accum, int accum_stride, int hq, int mass_stride, int n_sessions,
                              int max_blocks, hipStream_t stream) {
  if (n_sessions == 0 || max_blocks == 0) return hipSuccess;
  dim3 grid((max_blocks + kMassBlocksPerWG - 1) / kMassBlocksPerWG, n_sessions);
  mass_reduce_kernel<<<grid, 256, 0, stream>>>(seqs, session_rows, session_first, mass_m, mass_s, mf, lf, mass_accum,
                                               accum_stride, hq, mass_stride, n_sessions, max_blocks);
  return hipGetLastError();
}

hipError_t launch_mass_step_reduce(const SeqInfo* seqs, const int32_t* session_rows, const int32_t* session_first,
                                   float* mass_w, int64_t layer_floats, int num_layers, float* mass_accum,
                                   int accum_stride, int hq, int mass_stride, int n_sessions, int max_blocks,
                                   hipStream_t stream) {
  if (n_sessions == 0 || max_blocks == 0 || num_layers == 0) return hipSuccess;
  dim3 grid((max_blocks + kStepMassBlocks - 1) / kStepMassBlocks, n_sessions);
  mass_step_reduce_kernel<<<grid, kStepMassBlocks * kStepMassGroups, 0, stream>>>(seqs, session_rows, session_first, mass_w, layer_floats,
                                                    num_layers, mass_accum, accum_stride, hq, mass_stride,
                                                    max_blocks);
  return hipGetLastError();
}

}  // namespace pgr
