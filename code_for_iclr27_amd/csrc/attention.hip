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
// Work split (flash-decoding): a one-wave workgroup owns R query rows of one segment and one
// chunk of at most `chunk` keys. QK^T runs on v_mfma_f32_16x16x32 (the R rows padded to 16,
// K rows read straight into the B operand, 16 B per lane), the chunk's scores go to LDS, the wave
// forms its own max and exp-sum, then accumulates P*V on the VALU with each lane holding 8
// elements of a V row (16 B loads, D/8 lanes per row). A segment whose keys need more than one
// chunk writes (max, sum, unnormalised output) partials; the last of its workgroups to finish
// (a ticket counter, no waiting) merges them and writes the output. Every ticket is reset to zero
// by the workgroup that consumed it, so a zeroed workspace stays valid across calls.

#include <algorithm>

#include "lr_common.hpp"

namespace lr {
namespace {

typedef __bf16 attn_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 attn_f16x8 __attribute__((ext_vector_type(8)));
typedef float attn_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned attn_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kAttnThreads = 64;
constexpr int kAttnMaxChunk = 256;  // keys per workgroup (LDS holds kAttnMaxChunk x R scores)
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
  int64_t chunk;            // keys per chunk (multiple of 16, <= kAttnMaxChunk)
  float scale;
  void* out;                // [B, L, kv_heads * G, D]
  float* part_o;            // [units * splits, R, D]
  float* part_ml;           // [units * splits, R, 2]
  uint32_t* tickets;        // [units]
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

template <typename T, int D, int R>
__global__ __launch_bounds__(kAttnThreads) void packed_attention_kernel(AttnArgs a) {
  static_assert(D % 32 == 0 && D >= 64 && D <= 512, "head dim must be a multiple of 32");
  static_assert(R == 4 || R == 8, "rows per tile");
  constexpr int KS = D / 32;       // MFMA k-steps over the head dimension
  constexpr int LPK = D / 8;       // lanes per V row in the P*V phase
  constexpr int KPI = 64 / LPK;    // V rows per wave-wide load
  using Vec = AttnVec<T>;
  using X8 = typename Vec::x8;
  __shared__ __align__(16) float scores[kAttnMaxChunk][R];

  const int lane = threadIdx.x;
  const int64_t unit = blockIdx.x / a.splits, split = blockIdx.x - unit * a.splits;
  const int64_t seg = unit / a.tiles, tile = unit - seg * a.tiles;
  const int64_t rows = a.length * a.groups;
  const int64_t row0 = tile * R;
  const int64_t rows_here = rows - row0 < R ? rows - row0 : R;

  // Segment bounds, clamped into the key buffer.
  int64_t key0 = a.cu[seg], n = static_cast<int64_t>(a.cu[seg + 1]) - key0;
  key0 = key0 < 0 ? 0 : (key0 > a.key_rows ? a.key_rows : key0);
  n = n < 0 ? 0 : (n > a.key_rows - key0 ? a.key_rows - key0 : n);
  const int64_t shift = n - a.length;  // query i sees keys j <= i + shift
  const int64_t last_query = (row0 + rows_here - 1) / a.groups;
  int64_t key_end = last_query + shift + 1;
  key_end = key_end < 0 ? 0 : (key_end > n ? n : key_end);
  int64_t needed = (key_end + a.chunk - 1) / a.chunk;
  needed = needed > a.splits ? a.splits : needed;  // keys past splits * chunk are not read

  if (needed == 0) {  // no visible key for any row of this tile: zeros
    if (split != 0) return;
    for (int item = lane; item < R * LPK; item += kAttnThreads) {
      const int r = item / LPK, c = item - r * LPK;
      if (r < rows_here)
        *reinterpret_cast<attn_u32x4*>(output_row<T, D>(a, seg, row0 + r) + 8 * c) =
            attn_u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  if (split >= needed) return;

  const int64_t kb = split * a.chunk;
  const int64_t ke = kb + a.chunk < key_end ? kb + a.chunk : key_end;
  const int nk = static_cast<int>(ke - kb);
  const T* kbase = static_cast<const T*>(a.keys) + (key0 + kb) * D;
  const T* vbase = static_cast<const T*>(a.values) + (key0 + kb) * D;

  // ---- QK^T: A = query rows (row m = lane & 15), B = 16 key rows; k chunk j = lane >> 4.
  const int m = lane & 15, j = lane >> 4;
  X8 qop[KS];
  {
    const bool row_ok = m < rows_here;
    const int64_t row = row0 + (row_ok ? m : 0);
    const int64_t b = seg / a.kv_heads, h = seg - b * a.kv_heads;
    const int64_t i = row / a.groups, g = row - i * a.groups;
    const T* q = static_cast<const T*>(a.queries) + b * a.q_batch + (h * a.groups + g) * a.q_head +
                 i * a.q_query + 8 * j;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const attn_u32x4 raw = row_ok ? load16(q + 32 * ks) : attn_u32x4{0u, 0u, 0u, 0u};
      qop[ks] = __builtin_bit_cast(X8, raw);
    }
  }
  // This lane's output rows are 4 * j + r; their causal limits (keys at or below are visible).
  int64_t limit[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = row0 + 4 * j + r;
    limit[r] = (4 * j + r < rows_here) ? row / a.groups + shift - kb : -1;
  }
  const int blocks = (nk + 15) >> 4;
  for (int blk = 0; blk < blocks; blk += 2) {
    attn_u32x4 kraw[2][KS];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      int key = (blk + u) * 16 + m;
      key = key < nk ? key : nk - 1;  // clamped in-range row; its score is masked below
      const T* kp = kbase + static_cast<int64_t>(key) * D + 8 * j;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kraw[u][ks] = load16(kp + 32 * ks);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (blk + u >= blocks) break;
      attn_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc = Vec::mfma(qop[ks], __builtin_bit_cast(X8, kraw[u][ks]), acc);
      const int key = (blk + u) * 16 + m;  // D layout: lane holds key (lane & 15), rows 4j + r
      if (4 * j < R && key < nk) {
        attn_f32x4 s;
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = key <= limit[r] ? acc[r] * a.scale : kNegInf;
        *reinterpret_cast<attn_f32x4*>(&scores[key][4 * j]) = s;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- Per-row max and exp-sum over this chunk (lane owns keys lane, lane + 64, ...).
  float row_max[R], row_sum[R];
#pragma unroll
  for (int r = 0; r < R; ++r) row_max[r] = kNegInf;
  for (int key = lane; key < nk; key += kAttnThreads) {
#pragma unroll
    for (int r = 0; r < R; ++r) row_max[r] = fmaxf(row_max[r], scores[key][r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    row_max[r] = wave_max(row_max[r]);
    row_sum[r] = 0.f;
  }
  for (int key = lane; key < nk; key += kAttnThreads) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float s = scores[key][r];
      const float p = s == kNegInf ? 0.f : __builtin_amdgcn_exp2f((s - row_max[r]) * kAttnLog2e);
      scores[key][r] = p;
      row_sum[r] += p;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) row_sum[r] = wave_sum(row_sum[r]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- P*V: lane group kg = lane / LPK takes keys kg, kg + KPI, ...; lane owns 8 elements.
  const int kg = lane / LPK, c = lane - kg * LPK;
  float acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  constexpr int kUnroll = 4;
  for (int base = kg; base < nk; base += kUnroll * KPI) {
    attn_u32x4 vraw[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int key = base + u * KPI;
      key = key < nk ? key : nk - 1;
      vraw[u] = load16(vbase + static_cast<int64_t>(key) * D + 8 * c);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int key = base + u * KPI;
      if (key >= nk) break;
      float v[8];
      unpack8<T>(vraw[u], v);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float p = scores[key][r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(p, v[e], acc[r][e]);
      }
    }
  }
  // Sum the KPI lane groups (lanes c, c + LPK, ... hold the same elements).
#pragma unroll
  for (int offset = LPK; offset < 64; offset <<= 1)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] += __shfl_xor(acc[r][e], offset);

  if (needed == 1) {  // the only chunk: normalise and write
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r % KPI != kg || r >= rows_here) continue;
      const float inv = row_sum[r] > 0.f ? 1.0f / row_sum[r] : 0.f;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = acc[r][e] * inv;
      *reinterpret_cast<attn_u32x4*>(output_row<T, D>(a, seg, row0 + r) + 8 * c) = pack8<T>(o);
    }
    return;
  }

  // ---- Partials, then the last workgroup of this (segment, tile) merges them.
  const int64_t slot = (unit * a.splits + split) * R;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r % KPI != kg) continue;
    float* po = a.part_o + (slot + r) * D + 8 * c;
    *reinterpret_cast<attn_f32x4*>(po) = attn_f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
    *reinterpret_cast<attn_f32x4*>(po + 4) = attn_f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
  }
  if (lane < R) {
    float mx = 0.f, sm = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r == lane) { mx = row_max[r]; sm = row_sum[r]; }
    a.part_ml[(slot + lane) * 2] = mx;
    a.part_ml[(slot + lane) * 2 + 1] = sm;
  }
  __threadfence();  // partials visible device-wide before the ticket is taken
  uint32_t ticket = 0;
  if (lane == 0) ticket = atomicAdd(&a.tickets[unit], 1u);
  ticket = __shfl(ticket, 0);
  if (ticket != static_cast<uint32_t>(needed - 1)) return;
  __threadfence();
  if (lane == 0) a.tickets[unit] = 0u;  // consumed: the workspace is ready for the next call

  const int64_t first = unit * a.splits * R;
  for (int item = lane; item < R * LPK; item += kAttnThreads) {
    const int r = item / LPK, cc = item - r * LPK;
    if (r >= rows_here) continue;
    float mx = kNegInf;
    for (int64_t k = 0; k < needed; ++k) mx = fmaxf(mx, a.part_ml[(first + k * R + r) * 2]);
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float total = 0.f;
    if (mx != kNegInf) {
      for (int64_t k = 0; k < needed; ++k) {
        const float mk = a.part_ml[(first + k * R + r) * 2];
        if (mk == kNegInf) continue;
        const float w = __builtin_amdgcn_exp2f((mk - mx) * kAttnLog2e);
        total = __builtin_fmaf(w, a.part_ml[(first + k * R + r) * 2 + 1], total);
        const float* po = a.part_o + (first + k * R + r) * D + 8 * cc;
        const attn_f32x4 lo = *reinterpret_cast<const attn_f32x4*>(po);
        const attn_f32x4 hi = *reinterpret_cast<const attn_f32x4*>(po + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = __builtin_fmaf(w, lo[e], o[e]);
          o[4 + e] = __builtin_fmaf(w, hi[e], o[4 + e]);
        }
      }
    }
    const float inv = total > 0.f ? 1.0f / total : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
    *reinterpret_cast<attn_u32x4*>(output_row<T, D>(a, seg, row0 + r) + 8 * cc) = pack8<T>(o);
  }
}

struct AttnPlan {
  int rows_per_tile;
  int64_t tiles, splits, chunk, units;
};

AttnPlan plan_attention(int64_t segments, int64_t groups, int64_t length, int64_t max_keys) {
  AttnPlan p{};
  const int64_t rows = length * groups;
  p.rows_per_tile = rows <= 4 ? 4 : 8;
  p.tiles = ceil_div(rows, p.rows_per_tile);
  p.units = segments * p.tiles;
  // Enough workgroups to fill the chip (about 8 waves per CU), in chunks of 64..256 keys.
  constexpr int64_t kTargetWaves = 2048;
  int64_t chunk = kAttnMaxChunk;
  while (chunk > 64 && p.units * ceil_div(std::max<int64_t>(max_keys, 1), chunk) < kTargetWaves)
    chunk /= 2;
  p.chunk = chunk;
  p.splits = std::max<int64_t>(1, ceil_div(max_keys, chunk));
  return p;
}

size_t workspace_bytes(const AttnPlan& p, int64_t dim) {
  if (p.splits == 1) return 0;
  const int64_t slots = p.units * p.splits * p.rows_per_tile;
  const size_t tickets = static_cast<size_t>(ceil_div(p.units * 4, 256) * 256);
  return tickets + static_cast<size_t>(slots) * static_cast<size_t>(dim + 2) * 4;
}

template <typename T, int D, int R>
int launch_attention(const AttnArgs& args, int64_t blocks, hipStream_t stream) {
  hipLaunchKernelGGL((packed_attention_kernel<T, D, R>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kAttnThreads), 0, stream, args);
  return check_launch("packed_attention");
}

template <typename T, int D>
int launch_rows(const AttnArgs& args, int rows_per_tile, int64_t blocks, hipStream_t stream) {
  return rows_per_tile == 4 ? launch_attention<T, D, 4>(args, blocks, stream)
                            : launch_attention<T, D, 8>(args, blocks, stream);
}

template <typename T>
int launch_dim(const AttnArgs& args, int64_t dim, int rows_per_tile, int64_t blocks,
               hipStream_t stream) {
  switch (dim) {
    case 64: return launch_rows<T, 64>(args, rows_per_tile, blocks, stream);
    case 128: return launch_rows<T, 128>(args, rows_per_tile, blocks, stream);
    default: return launch_rows<T, 256>(args, rows_per_tile, blocks, stream);
  }
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" size_t lr_packed_attention_workspace_bytes(int64_t segments, int64_t groups,
                                                      int64_t length, int64_t max_keys,
                                                      int64_t dim) {
  if (segments <= 0 || groups <= 0 || length <= 0 || max_keys < 0 || dim <= 0) return 0;
  return workspace_bytes(plan_attention(segments, groups, length, max_keys), dim);
}

extern "C" int lr_packed_attention(const void* queries, int64_t q_batch_stride,
                                   int64_t q_head_stride, int64_t q_query_stride,
                                   const void* keys, const void* values, int64_t key_rows,
                                   const int32_t* cu_seqlens_k, int64_t batch, int64_t kv_heads,
                                   int64_t groups, int64_t length, int64_t dim, int dtype,
                                   int64_t max_keys, float scale, void* out, void* workspace,
                                   size_t workspace_size, void* stream) {
  clear_error();
  LR_REQUIRE(dtype == LR_DTYPE_BF16 || dtype == LR_DTYPE_F16,
             "FlashAttention only supports fp16 and bf16 data type");
  LR_REQUIRE(dim == 64 || dim == 128 || dim == 256, "Head dimension must be 64, 128 or 256");
  LR_REQUIRE(batch > 0 && kv_heads > 0 && groups > 0 && length > 0, "Empty attention dimensions");
  LR_REQUIRE(key_rows >= 0 && max_keys >= 0, "Invalid key lengths");
  LR_REQUIRE(queries && out && cu_seqlens_k && (key_rows == 0 || (keys && values)),
             "Invalid attention buffers");
  const uintptr_t alignment = reinterpret_cast<uintptr_t>(queries) |
                              reinterpret_cast<uintptr_t>(keys) |
                              reinterpret_cast<uintptr_t>(values) |
                              reinterpret_cast<uintptr_t>(out) |
                              static_cast<uintptr_t>((q_batch_stride | q_head_stride |
                                                      q_query_stride) * 2);
  LR_REQUIRE(alignment % 16 == 0, "Attention operands must be 16-byte aligned");
  const int64_t segments = batch * kv_heads;
  const AttnPlan plan = plan_attention(segments, groups, length, max_keys);
  const size_t needed = workspace_bytes(plan, dim);
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
  args.chunk = plan.chunk;
  args.scale = scale;
  args.out = out;
  if (needed) {
    char* base = static_cast<char*>(workspace);
    args.tickets = reinterpret_cast<uint32_t*>(base);
    const size_t tickets = static_cast<size_t>(ceil_div(plan.units * 4, 256) * 256);
    args.part_ml = reinterpret_cast<float*>(base + tickets);
    args.part_o = args.part_ml + plan.units * plan.splits * plan.rows_per_tile * 2;
  }
  const hipStream_t s = as_stream(stream);
  return dtype == LR_DTYPE_BF16
             ? launch_dim<__bf16>(args, dim, plan.rows_per_tile, blocks, s)
             : launch_dim<_Float16>(args, dim, plan.rows_per_tile, blocks, s);
}
