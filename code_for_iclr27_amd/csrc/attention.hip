// Attention over the packed ragged KV layout: one query block per (request, KV head) segment,
// the drop-in for the flash_attn_varlen_func call of src/lazy_recall/attention.py:15-35.
//
// Segment s (= request b * kv_heads + KV head h) owns key rows [cu[s], cu[s+1]) of the packed
// K/V buffers and `length` queries for each of its G = query_heads / kv_heads query heads. Its
// L*G query rows are numbered row = i*G + g (query i, group g). Causal masking is aligned to the
// end of the segment, as flash-attention's varlen causal mode: query i sees keys j <= i + n - L
// (n = the segment's key count); for decode (L = 1) that is every key. A row with no visible key
// outputs zeros. Softmax scale `scale`, accumulation in f32, output rounded to the input type.
//
// Work split (flash decoding): a workgroup of four waves owns R query rows of one segment and
// one block of keys; each wave takes 12-16 KB of its K rows (wave_keys) and issues every load
// (queries, K rows, V slices) before the first use, so one memory round trip covers the wave.
// QK^T runs on v_mfma_f32_16x16x32 (the R rows padded to 16, K rows straight into the B operand,
// 16 B per lane); each wave forms its own max and exp-sum in registers, stages p in LDS and
// accumulates P*V on the VALU with each lane holding 8 elements of a V row (D/8 lanes per row).
// The four wave states merge in LDS. A segment whose keys need more than one block writes
// (max, sum, unnormalised output) partials, and a second launch merges them (one workgroup per
// segment and tile). The launch boundary orders the two: a device-scope fence per workgroup
// instead (a ticket taken by the last block) costs an L2 writeback and invalidate on every
// workgroup's XCD, and measured 4-6x slower at the cfg2 decode shape.

#include <algorithm>
#include <mutex>
#include <string>

#include "lr_common.hpp"

namespace lr {
namespace {

typedef __bf16 attn_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 attn_f16x8 __attribute__((ext_vector_type(8)));
typedef float attn_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned attn_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = 64 * kAttnWaves;
// Keys per wave: 12 KB of K rows (and as many V bytes) for d64/d128, 16 KB for d256 (a whole
// number of 16-key MFMA blocks); small enough for three waves per SIMD. A call whose blocks of
// that size would not give every CU two workgroups (batch-1 decode: cfg1 has 96) takes one
// 16-key MFMA block per wave instead, so that its single round of loads spreads over the chip.
constexpr int wave_keys(int dim) { return dim == 256 ? 32 : 6144 / dim; }
constexpr int kSmallWaveKeys = 16;
constexpr int64_t kFewBlocks = 512;
// Partial blocks each merging thread loads at once: four, or twelve where a thread folds more
// than four blocks (batch-1 decode: cfg1's 36 blocks per unit take one round of loads instead
// of three; measured 14.9 against 15.3 us per layer, and no better for cfg2's 12 blocks).
constexpr int kMergeUnroll = 4;
constexpr int kMergeUnrollWide = 12;
constexpr float kAttnLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

template <typename T> struct AttnVec;
template <> struct AttnVec<__bf16> {
  using x8 = attn_bf16x8;
  static __device__ __forceinline__ attn_f32x4 mfma(x8 a, x8 b, attn_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct AttnVec<_Float16> {
  using x8 = attn_f16x8;
  static __device__ __forceinline__ attn_f32x4 mfma(x8 a, x8 b, attn_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

struct AttnArgs {
  const void* queries;      // element strides below; the last dimension is contiguous
  int64_t q_batch, q_head, q_query;
  const void* keys;         // [key_rows, D]
  const void* values;       // [key_rows, D]
  int64_t key_rows;
  const int32_t* cu;        // [segments + 1]
  int64_t kv_heads, groups, length;
  int64_t tiles;            // query-row tiles per segment: ceil(L*G / R)
  int64_t splits;           // key chunks per (segment, tile) in the grid
  float scale;
  void* out;                // [B, L, kv_heads * G, D]
  float* part_o;            // [units * splits, R, D]
  float* part_ml;           // [units * splits, R, 2]
  const void* pending_keys;    // NULL, or [segments, D]: a row after each segment's cached rows
  const void* pending_values;  // with pending_keys
};

template <typename T>
__device__ __forceinline__ void unpack8(attn_u32x4 raw, float (&v)[8]) {
  if constexpr (std::is_same<T, __bf16>::value) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __builtin_bit_cast(float, raw[e] << 16);
      v[2 * e + 1] = __builtin_bit_cast(float, raw[e] & 0xffff0000u);
    }
  } else {
    const attn_f16x8 h = __builtin_bit_cast(attn_f16x8, raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(h[e]);
  }
}

template <typename T>
__device__ __forceinline__ attn_u32x4 pack8(const float (&v)[8]) {
  typename AttnVec<T>::x8 h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = static_cast<T>(v[e]);  // round to nearest even
  return __builtin_bit_cast(attn_u32x4, h);
}

__device__ __forceinline__ attn_u32x4 load16(const void* p) {
  return *(const __attribute__((address_space(1))) attn_u32x4*)p;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
  return v;
}

// Output row `row` of segment `seg` (query i = row / G, query head h*G + row % G).
template <typename T, int D>
__device__ __forceinline__ T* output_row(const AttnArgs& a, int64_t seg, int64_t row) {
  const int64_t b = seg / a.kv_heads, h = seg - b * a.kv_heads;
  const int64_t i = row / a.groups, g = row - i * a.groups;
  const int64_t heads = a.kv_heads * a.groups;
  return static_cast<T*>(a.out) + ((b * a.length + i) * heads + h * a.groups + g) * D;
}

// A (max, exp-sum, unnormalised output slice) softmax state; merge_into folds another in.
struct MergeState {
  float m, l, o[8];
};

__device__ __forceinline__ void merge_into(MergeState& s, float m, float l, const float (&o)[8]) {
  if (m == kNegInf) return;
  const float mx = fmaxf(s.m, m);
  const float ws = s.m == kNegInf ? 0.f : __builtin_amdgcn_exp2f((s.m - mx) * kAttnLog2e);
  const float wo = __builtin_amdgcn_exp2f((m - mx) * kAttnLog2e);
  s.l = __builtin_fmaf(wo, l, s.l * ws);
#pragma unroll
  for (int e = 0; e < 8; ++e) s.o[e] = __builtin_fmaf(wo, o[e], s.o[e] * ws);
  s.m = mx;
}

template <typename T, int D, int R, int CH>
__global__ __launch_bounds__(kAttnThreads, D == 256 ? 2 : 3) void packed_attention_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "head dim");
  static_assert(R == 4 || R == 8, "rows per tile");
  constexpr int KS = D / 32;          // MFMA k-steps over the head dimension
  constexpr int LPK = D / 8;          // lanes per V row in the P*V phase
  constexpr int KPI = 64 / LPK;       // V rows per wave-wide load
  static_assert(CH % 16 == 0, "whole MFMA key blocks");
  constexpr int NB = CH / 16;         // 16-key MFMA blocks per wave
  constexpr int VL = CH / KPI;        // V loads (16 B) per lane
  constexpr int ITEMS = R * LPK;      // (row, 8-element slice) items of one output tile
  static_assert(ITEMS <= kAttnThreads, "one merge item per thread");
  using Vec = AttnVec<T>;
  using X8 = typename Vec::x8;
  __shared__ __align__(16) float probs[kAttnWaves][CH][R];
  __shared__ __align__(16) float wave_o[kAttnWaves][R][D];
  __shared__ float wave_ml[kAttnWaves][R][2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t unit = blockIdx.x / a.splits, split = blockIdx.x - unit * a.splits;
  const int64_t seg = unit / a.tiles, tile = unit - seg * a.tiles;
  const int64_t rows = a.length * a.groups;
  const int64_t row0 = tile * R;
  const int64_t rows_here = rows - row0 < R ? rows - row0 : R;

  // Segment bounds, clamped into the key buffer. A pending row (the decode step's own token,
  // not yet appended) is key `cached` of the segment, after its cached rows.
  int64_t key0 = a.cu[seg], n = static_cast<int64_t>(a.cu[seg + 1]) - key0;
  key0 = key0 < 0 ? 0 : (key0 > a.key_rows ? a.key_rows : key0);
  n = n < 0 ? 0 : (n > a.key_rows - key0 ? a.key_rows - key0 : n);
  const int64_t cached = n;
  if (a.pending_keys != nullptr) ++n;
  const int64_t shift = n - a.length;  // query i sees keys j <= i + shift
  const int64_t last_query = (row0 + rows_here - 1) / a.groups;
  int64_t key_end = last_query + shift + 1;
  key_end = key_end < 0 ? 0 : (key_end > n ? n : key_end);
  constexpr int64_t kBlockKeys = kAttnWaves * CH;
  int64_t needed = (key_end + kBlockKeys - 1) / kBlockKeys;
  needed = needed > a.splits ? a.splits : needed;  // keys past splits * block keys are not read

  if (needed == 0) {  // no visible key for any row of this tile: zeros
    if (split != 0) return;
    for (int item = tid; item < ITEMS; item += kAttnThreads) {
      const int r = item / LPK, c = item - r * LPK;
      if (r < rows_here)
        *reinterpret_cast<attn_u32x4*>(output_row<T, D>(a, seg, row0 + r) + 8 * c) =
            attn_u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  if (split >= needed) return;  // uniform across the workgroup

  const int64_t kb = split * kBlockKeys + wave * CH;
  const int64_t ke = kb + CH < key_end ? kb + CH : key_end;
  const int nk = kb < ke ? static_cast<int>(ke - kb) : 0;
  const int m = lane & 15, j = lane >> 4;
  const int kg = lane / LPK, c = lane - kg * LPK;

  float row_max[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
  float row_sum[4] = {0.f, 0.f, 0.f, 0.f};
  float acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;

  if (nk > 0) {
    const T* kbase = static_cast<const T*>(a.keys) + (key0 + kb) * D;
    const T* vbase = static_cast<const T*>(a.values) + (key0 + kb) * D;
    // row of wave key `key` (< nk): a cached row, or the segment's pending row
    const int64_t cached_here = cached - kb;
    auto key_row = [&](const T* base, const void* pending, int key) -> const T* {
      return key < cached_here ? base + static_cast<int64_t>(key) * D
                               : static_cast<const T*>(pending) + seg * D;
    };
    // Every load of the wave is issued before the first use: queries (A operand, row m = lane
    // & 15, k chunk j = lane >> 4), K rows (B operand, key m of each 16-key block), V slices.
    X8 qop[KS];
    {
      const bool row_ok = m < rows_here;
      const int64_t row = row0 + (row_ok ? m : 0);
      const int64_t b = seg / a.kv_heads, h = seg - b * a.kv_heads;
      const int64_t i = row / a.groups, g = row - i * a.groups;
      const T* q = static_cast<const T*>(a.queries) + b * a.q_batch +
                   (h * a.groups + g) * a.q_head + i * a.q_query + 8 * j;
      // Unconditional loads from a valid row (padding lanes read row0's) and a select after
      // them: a load under a branch is waited for inside the branch.
      attn_u32x4 raw[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) raw[ks] = load16(q + 32 * ks);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qop[ks] = __builtin_bit_cast(X8, row_ok ? raw[ks] : attn_u32x4{0u, 0u, 0u, 0u});
    }
    attn_u32x4 kraw[NB][KS];
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      int key = blk * 16 + m;
      key = key < nk ? key : nk - 1;  // clamped in-range row; its score is masked below
      const T* kp = key_row(kbase, a.pending_keys, key) + 8 * j;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kraw[blk][ks] = load16(kp + 32 * ks);
    }
    attn_u32x4 vraw[VL];
#pragma unroll
    for (int u = 0; u < VL; ++u) {
      int key = kg + u * KPI;
      key = key < nk ? key : nk - 1;
      vraw[u] = load16(key_row(vbase, a.pending_values, key) + 8 * c);
    }

    // QK^T. D layout: lane holds key 16 * blk + (lane & 15) for rows 4j + r.
    int64_t limit[4];  // causal limit of this lane's rows, relative to kb (keys <= limit seen)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = row0 + 4 * j + r;
      limit[r] = (4 * j + r < rows_here) ? row / a.groups + shift - kb : -1;
    }
    float s[NB][4];
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      attn_f32x4 dot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) dot = Vec::mfma(qop[ks], __builtin_bit_cast(X8, kraw[blk][ks]), dot);
      const int key = blk * 16 + m;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[blk][r] = (key < nk && key <= limit[r]) ? dot[r] * a.scale : kNegInf;
        row_max[r] = fmaxf(row_max[r], s[blk][r]);
      }
    }
    // Row max and exp-sum over the 16 lanes that share rows 4j .. 4j + 3.
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int offset = 1; offset < 16; offset <<= 1)
        row_max[r] = fmaxf(row_max[r], __shfl_xor(row_max[r], offset));
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      attn_f32x4 p;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = s[blk][r] == kNegInf ? 0.f
                                    : __builtin_amdgcn_exp2f((s[blk][r] - row_max[r]) * kAttnLog2e);
        row_sum[r] += p[r];
      }
      if (4 * j < R) *reinterpret_cast<attn_f32x4*>(&probs[wave][blk * 16 + m][4 * j]) = p;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int offset = 1; offset < 16; offset <<= 1) row_sum[r] += __shfl_xor(row_sum[r], offset);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // P*V on the prefetched V slices; keys past nk carry p = 0 from a clamped row, skipped.
#pragma unroll
    for (int u = 0; u < VL; ++u) {
      const int key = kg + u * KPI;
      if (key >= nk) break;
      float v[8];
      unpack8<T>(vraw[u], v);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float p = probs[wave][key][r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(p, v[e], acc[r][e]);
      }
    }
    // Sum the KPI lane groups (lanes c, c + LPK, ... hold the same elements).
#pragma unroll
    for (int offset = LPK; offset < 64; offset <<= 1)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] += __shfl_xor(acc[r][e], offset);
  }

  // Wave states to LDS: rows r = 4j + i are held by lanes 16j .. 16j + 15.
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r % KPI != kg) continue;
    float* wo = &wave_o[wave][r][8 * c];
    *reinterpret_cast<attn_f32x4*>(wo) = attn_f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
    *reinterpret_cast<attn_f32x4*>(wo + 4) = attn_f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
  }
  if (m == 0 && 4 * j < R) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wave_ml[wave][4 * j + r][0] = row_max[r];
      wave_ml[wave][4 * j + r][1] = row_sum[r];
    }
  }
  __syncthreads();

  // Merge the waves: thread t < ITEMS owns row r = t / LPK, elements 8 * (t % LPK) ...
  const int r_item = tid / LPK, c_item = tid - r_item * LPK;
  MergeState st{kNegInf, 0.f, {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}};
  if (tid < ITEMS) {
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      float o[8];
      const float* wo = &wave_o[w][r_item][8 * c_item];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = wo[e];
      merge_into(st, wave_ml[w][r_item][0], wave_ml[w][r_item][1], o);
    }
  }
  if (needed == 1) {  // the only block of keys: normalise and write
    if (tid < ITEMS && r_item < rows_here) {
      const float inv = st.l > 0.f ? 1.0f / st.l : 0.f;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = st.o[e] * inv;
      *reinterpret_cast<attn_u32x4*>(output_row<T, D>(a, seg, row0 + r_item) + 8 * c_item) =
          pack8<T>(o);
    }
    return;
  }

  // ---- Partial state of this block; attention_merge_kernel combines the blocks.
  const int64_t slot = (unit * a.splits + split) * R;
  if (tid < ITEMS) {
    float* po = a.part_o + (slot + r_item) * D + 8 * c_item;
    *reinterpret_cast<attn_f32x4*>(po) = attn_f32x4{st.o[0], st.o[1], st.o[2], st.o[3]};
    *reinterpret_cast<attn_f32x4*>(po + 4) = attn_f32x4{st.o[4], st.o[5], st.o[6], st.o[7]};
    if (c_item == 0) {
      a.part_ml[(slot + r_item) * 2] = st.m;
      a.part_ml[(slot + r_item) * 2 + 1] = st.l;
    }
  }
}

// Second launch: one workgroup per (segment, tile) whose keys spanned more than one block merges
// the blocks' partial states. Thread (part, item) folds blocks part, part + PARTS, ... (in that
// order, whatever U) with the loads of U blocks in flight at once; the PARTS states then meet
// in LDS.
template <typename T, int D, int R, int CH, int U>
__global__ __launch_bounds__(kAttnThreads) void attention_merge_kernel(AttnArgs a) {
  constexpr int LPK = D / 8;
  constexpr int ITEMS = R * LPK;
  constexpr int PARTS = kAttnThreads / ITEMS;
  constexpr int64_t kBlockKeys = kAttnWaves * CH;
  __shared__ __align__(16) float merge_o[kAttnThreads][8];
  __shared__ float merge_ml[kAttnThreads][2];
  const int tid = threadIdx.x;
  const int64_t unit = blockIdx.x;
  const int64_t seg = unit / a.tiles, tile = unit - seg * a.tiles;
  const int64_t rows = a.length * a.groups;
  const int64_t row0 = tile * R;
  const int64_t rows_here = rows - row0 < R ? rows - row0 : R;
  int64_t key0 = a.cu[seg], n = static_cast<int64_t>(a.cu[seg + 1]) - key0;
  key0 = key0 < 0 ? 0 : (key0 > a.key_rows ? a.key_rows : key0);
  n = n < 0 ? 0 : (n > a.key_rows - key0 ? a.key_rows - key0 : n);
  if (a.pending_keys != nullptr) ++n;  // the pending row, as in the first launch
  const int64_t last_query = (row0 + rows_here - 1) / a.groups;
  int64_t key_end = last_query + n - a.length + 1;
  key_end = key_end < 0 ? 0 : (key_end > n ? n : key_end);
  int64_t needed = (key_end + kBlockKeys - 1) / kBlockKeys;
  needed = needed > a.splits ? a.splits : needed;
  if (needed <= 1) return;  // the first launch wrote this tile's output

  const int part = tid / ITEMS, item = tid - part * ITEMS;
  const int r = item / LPK, cc = item - r * LPK;
  const int64_t first = unit * a.splits * R;
  MergeState total{kNegInf, 0.f, {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}};
  for (int64_t k0 = part; k0 < needed; k0 += PARTS * U) {
    float mk[U], lk[U];
    attn_f32x4 lo[U], hi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t k = k0 + u * PARTS;
      const bool live = k < needed;
      k = live ? k : k0;
      const int64_t at = first + k * R + r;
      mk[u] = live ? a.part_ml[at * 2] : kNegInf;
      lk[u] = a.part_ml[at * 2 + 1];
      lo[u] = *reinterpret_cast<const attn_f32x4*>(a.part_o + at * D + 8 * cc);
      hi[u] = *reinterpret_cast<const attn_f32x4*>(a.part_o + at * D + 8 * cc + 4);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float o[8] = {lo[u][0], lo[u][1], lo[u][2], lo[u][3],
                          hi[u][0], hi[u][1], hi[u][2], hi[u][3]};
      merge_into(total, mk[u], lk[u], o);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) merge_o[tid][e] = total.o[e];
  merge_ml[tid][0] = total.m;
  merge_ml[tid][1] = total.l;
  __syncthreads();
  if (part != 0 || r >= rows_here) return;
  for (int p = 1; p < PARTS; ++p) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = merge_o[p * ITEMS + item][e];
    merge_into(total, merge_ml[p * ITEMS + item][0], merge_ml[p * ITEMS + item][1], o);
  }
  const float inv = total.l > 0.f ? 1.0f / total.l : 0.f;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = total.o[e] * inv;
  *reinterpret_cast<attn_u32x4*>(output_row<T, D>(a, seg, row0 + r) + 8 * cc) = pack8<T>(o);
}

struct AttnPlan {
  int rows_per_tile, wave_keys;
  int64_t tiles, splits, chunk, units;
};

AttnPlan plan_attention(int64_t segments, int64_t groups, int64_t length, int64_t max_keys,
                        int64_t dim) {
  AttnPlan p{};
  const int64_t rows = length * groups;
  p.rows_per_tile = rows <= 4 ? 4 : 8;
  p.tiles = ceil_div(rows, p.rows_per_tile);
  p.units = segments * p.tiles;
  // Keys one workgroup covers: four waves of wave_keys keys each.
  p.wave_keys = wave_keys(static_cast<int>(dim));
  p.chunk = kAttnWaves * p.wave_keys;
  p.splits = std::max<int64_t>(1, ceil_div(max_keys, p.chunk));
  if (p.units * p.splits < kFewBlocks && p.splits > 1) {
    p.wave_keys = kSmallWaveKeys;
    p.chunk = kAttnWaves * p.wave_keys;
    p.splits = ceil_div(max_keys, p.chunk);
  }
  return p;
}

size_t workspace_bytes(const AttnPlan& p, int64_t dim) {
  if (p.splits == 1) return 0;
  const int64_t slots = p.units * p.splits * p.rows_per_tile;
  return static_cast<size_t>(slots) * static_cast<size_t>(dim + 2) * 4;
}

template <typename T, int D, int R, int CH>
int launch_attention(const AttnArgs& args, int64_t blocks, hipStream_t stream) {
  hipLaunchKernelGGL((packed_attention_kernel<T, D, R, CH>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kAttnThreads), 0, stream, args);
  if (int status = check_launch("packed_attention")) return status;
  if (args.splits == 1) return LR_OK;
  // blocks each merging thread folds: PARTS = threads / (R * D / 8) threads share a row slice
  const int64_t per_part = ceil_div(args.splits, int64_t{kAttnThreads / (R * D / 8)});
  if (per_part > kMergeUnroll)
    hipLaunchKernelGGL((attention_merge_kernel<T, D, R, CH, kMergeUnrollWide>),
                       dim3(static_cast<unsigned>(blocks / args.splits)), dim3(kAttnThreads), 0,
                       stream, args);
  else
    hipLaunchKernelGGL((attention_merge_kernel<T, D, R, CH, kMergeUnroll>),
                       dim3(static_cast<unsigned>(blocks / args.splits)), dim3(kAttnThreads), 0,
                       stream, args);
  return check_launch("packed_attention merge");
}

template <typename T, int D, int R>
int launch_keys(const AttnArgs& args, int keys_per_wave, int64_t blocks, hipStream_t stream) {
  return keys_per_wave == kSmallWaveKeys
             ? launch_attention<T, D, R, kSmallWaveKeys>(args, blocks, stream)
             : launch_attention<T, D, R, wave_keys(D)>(args, blocks, stream);
}

template <typename T, int D>
int launch_rows(const AttnArgs& args, const AttnPlan& plan, int64_t blocks, hipStream_t stream) {
  return plan.rows_per_tile == 4 ? launch_keys<T, D, 4>(args, plan.wave_keys, blocks, stream)
                                 : launch_keys<T, D, 8>(args, plan.wave_keys, blocks, stream);
}

template <typename T>
int launch_dim(const AttnArgs& args, int64_t dim, const AttnPlan& plan, int64_t blocks,
               hipStream_t stream) {
  switch (dim) {
    case 64: return launch_rows<T, 64>(args, plan, blocks, stream);
    case 128: return launch_rows<T, 128>(args, plan, blocks, stream);
    default: return launch_rows<T, 256>(args, plan, blocks, stream);
  }
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" size_t lr_packed_attention_workspace_bytes(int64_t segments, int64_t groups,
                                                      int64_t length, int64_t max_keys,
                                                      int64_t dim) {
  if (segments <= 0 || groups <= 0 || length <= 0 || max_keys < 0 || dim <= 0) return 0;
  return workspace_bytes(plan_attention(segments, groups, length, max_keys, dim), dim);
}

namespace lr {
namespace {

// The checks and launches shared by lr_packed_attention and lr_packed_attention_noalloc.
// `scratch_limit` is nonzero for the allocation-free variant: its workspace is the library's
// fixed per-device array of that size, and a call that needs more is refused with its own
// message before anything is enqueued.
int packed_attention(const void* queries, int64_t q_batch_stride, int64_t q_head_stride,
                     int64_t q_query_stride, const void* keys, const void* values,
                     int64_t key_rows, const int32_t* cu_seqlens_k, int64_t batch,
                     int64_t kv_heads, int64_t groups, int64_t length, int64_t dim, int dtype,
                     int64_t max_keys, float scale, void* out, void* workspace,
                     size_t workspace_size, size_t scratch_limit, void* stream,
                     const void* pending_keys = nullptr, const void* pending_values = nullptr) {
  LR_REQUIRE(dtype == LR_DTYPE_BF16 || dtype == LR_DTYPE_F16,
             "FlashAttention only supports fp16 and bf16 data type");
  LR_REQUIRE((pending_keys == nullptr) == (pending_values == nullptr),
             "Pending keys and values go together");
  LR_REQUIRE(pending_keys == nullptr || length == 1, "Pending rows need one query per segment");
  LR_REQUIRE(dim == 64 || dim == 128 || dim == 256, "Head dimension must be 64, 128 or 256");
  LR_REQUIRE(batch > 0 && kv_heads > 0 && groups > 0 && length > 0, "Empty attention dimensions");
  LR_REQUIRE(key_rows >= 0 && max_keys >= 0, "Invalid key lengths");
  LR_REQUIRE(queries && out && cu_seqlens_k && (key_rows == 0 || (keys && values)),
             "Invalid attention buffers");
  const uintptr_t alignment = reinterpret_cast<uintptr_t>(queries) |
                              reinterpret_cast<uintptr_t>(keys) |
                              reinterpret_cast<uintptr_t>(values) |
                              reinterpret_cast<uintptr_t>(out) |
                              reinterpret_cast<uintptr_t>(pending_keys) |
                              reinterpret_cast<uintptr_t>(pending_values) |
                              static_cast<uintptr_t>((q_batch_stride | q_head_stride |
                                                      q_query_stride) * 2);
  LR_REQUIRE(alignment % 16 == 0, "Attention operands must be 16-byte aligned");
  const int64_t segments = batch * kv_heads;
  if (pending_keys != nullptr) ++max_keys;  // every segment's pending row
  const AttnPlan plan = plan_attention(segments, groups, length, max_keys, dim);
  const size_t needed = workspace_bytes(plan, dim);
  if (scratch_limit) {
    LR_REQUIRE(needed <= scratch_limit,
               "Attention needs " + std::to_string(needed) +
                   " bytes of scratch; the allocation-free entry point holds at most " +
                   std::to_string(scratch_limit) + " bytes per device");
  }
  LR_REQUIRE(workspace_size >= needed && (needed == 0 || workspace != nullptr),
             "Attention workspace too small");
  LR_REQUIRE(needed == 0 || reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
             "Attention workspace must be 256-byte aligned");
  const int64_t blocks = plan.units * plan.splits;
  LR_REQUIRE(blocks < (int64_t{1} << 31), "Attention grid too large");

  AttnArgs args{};
  args.queries = queries;
  args.q_batch = q_batch_stride;
  args.q_head = q_head_stride;
  args.q_query = q_query_stride;
  args.keys = keys;
  args.values = values;
  args.key_rows = key_rows;
  args.cu = cu_seqlens_k;
  args.kv_heads = kv_heads;
  args.groups = groups;
  args.length = length;
  args.tiles = plan.tiles;
  args.splits = plan.splits;
  args.scale = scale;
  args.out = out;
  args.pending_keys = pending_keys;
  args.pending_values = pending_values;
  if (needed) {
    args.part_ml = static_cast<float*>(workspace);
    args.part_o = args.part_ml + plan.units * plan.splits * plan.rows_per_tile * 2;
  }
  const hipStream_t s = as_stream(stream);
  return dtype == LR_DTYPE_BF16
             ? launch_dim<__bf16>(args, dim, plan, blocks, s)
             : launch_dim<_Float16>(args, dim, plan, blocks, s);
}

// Workspace of the allocation-free entry point: one fixed array per device, held from the
// library's load onto that device until the process ends. Host code never passes `scratch`
// itself to a kernel (on the host the name is only a stand-in for the symbol); it passes the
// device address hipGetSymbolAddress gives, looked up once per device.
constexpr size_t kAttentionScratchBytes = size_t{16} << 20;
__device__ __align__(256) unsigned char scratch[kAttentionScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

// The device address of `scratch` on the device that owns `stream` (the current device for the
// null stream). The first call on a device makes that device current for the lookup and then
// restores the caller's device.
int scratch_address(hipStream_t stream, void** address) {
  int device = 0;
  if (stream != nullptr) {
    LR_HIP_TRY(hipStreamGetDevice(stream, &device));
  } else {
    LR_HIP_TRY(hipGetDevice(&device));
  }
  LR_REQUIRE(device >= 0 && device < kMaxDevices, "Device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    int current = 0;
    LR_HIP_TRY(hipGetDevice(&current));
    if (current != device) LR_HIP_TRY(hipSetDevice(device));
    void* found = nullptr;
    const hipError_t status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    if (current != device) LR_HIP_TRY(hipSetDevice(current));
    if (status != hipSuccess || found == nullptr) {
      (void)hipGetLastError();
      set_error(std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(status));
      return LR_ERR_HIP;
    }
    g_scratch_address[device] = found;
  }
  *address = g_scratch_address[device];
  return LR_OK;
}

}  // namespace
}  // namespace lr

extern "C" int lr_packed_attention(const void* queries, int64_t q_batch_stride,
                                   int64_t q_head_stride, int64_t q_query_stride,
                                   const void* keys, const void* values, int64_t key_rows,
                                   const int32_t* cu_seqlens_k, int64_t batch, int64_t kv_heads,
                                   int64_t groups, int64_t length, int64_t dim, int dtype,
                                   int64_t max_keys, float scale, void* out, void* workspace,
                                   size_t workspace_size, void* stream) {
  clear_error();
  return packed_attention(queries, q_batch_stride, q_head_stride, q_query_stride, keys, values,
                          key_rows, cu_seqlens_k, batch, kv_heads, groups, length, dim, dtype,
                          max_keys, scale, out, workspace, workspace_size, 0, stream);
}

extern "C" size_t lr_packed_attention_pending_workspace_bytes(int64_t segments, int64_t groups,
                                                              int64_t max_keys, int64_t dim) {
  return lr_packed_attention_workspace_bytes(segments, groups, 1, max_keys + 1, dim);
}

extern "C" int lr_packed_attention_pending(const void* queries, int64_t q_batch_stride,
                                           int64_t q_head_stride, int64_t q_query_stride,
                                           const void* keys, const void* values,
                                           int64_t key_rows, const int32_t* cu_seqlens_k,
                                           int64_t batch, int64_t kv_heads, int64_t groups,
                                           int64_t dim, int dtype, int64_t max_keys, float scale,
                                           const void* pending_keys, const void* pending_values,
                                           void* out, void* workspace, size_t workspace_size,
                                           void* stream) {
  clear_error();
  LR_REQUIRE(pending_keys != nullptr && pending_values != nullptr, "Invalid attention buffers");
  return packed_attention(queries, q_batch_stride, q_head_stride, q_query_stride, keys, values,
                          key_rows, cu_seqlens_k, batch, kv_heads, groups, 1, dim, dtype,
                          max_keys, scale, out, workspace, workspace_size, 0, stream,
                          pending_keys, pending_values);
}

extern "C" size_t lr_packed_attention_scratch_bytes(void) { return kAttentionScratchBytes; }

extern "C" int lr_packed_attention_noalloc(const void* queries, int64_t q_batch_stride,
                                           int64_t q_head_stride, int64_t q_query_stride,
                                           const void* keys, const void* values,
                                           int64_t key_rows, const int32_t* cu_seqlens_k,
                                           int64_t batch, int64_t kv_heads, int64_t groups,
                                           int64_t length, int64_t dim, int dtype,
                                           int64_t max_keys, float scale, void* out,
                                           void* stream) {
  clear_error();
  // The size check comes first and needs no HIP call; a call that needs no partial states
  // (every segment within one key block) does not touch the scratch array at all.
  const int64_t segments =
      batch > 0 && kv_heads > 0 && batch <= (int64_t{1} << 31) / kv_heads ? batch * kv_heads : 0;
  const size_t needed = lr_packed_attention_workspace_bytes(segments, groups, length, max_keys, dim);
  LR_REQUIRE(needed <= kAttentionScratchBytes,
             "Attention needs " + std::to_string(needed) +
                 " bytes of scratch; the allocation-free entry point holds at most " +
                 std::to_string(kAttentionScratchBytes) + " bytes per device");
  void* workspace = nullptr;
  if (needed) {
    if (int status = scratch_address(as_stream(stream), &workspace)) return status;
  }
  return packed_attention(queries, q_batch_stride, q_head_stride, q_query_stride, keys, values,
                          key_rows, cu_seqlens_k, batch, kv_heads, groups, length, dim, dtype,
                          max_keys, scale, out, workspace, needed ? kAttentionScratchBytes : 0,
                          kAttentionScratchBytes, stream);
}
