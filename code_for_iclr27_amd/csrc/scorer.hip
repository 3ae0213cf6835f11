// Fused temporal decision-risk scorer for all (layer, KV head) segments of an audit.
//
// Reference semantics (per head, src/lazy_recall/scoring.py:152-195 and csrc/scoring.cu:32-128):
//   pv[g,t]   = grad[g,:] . V[t,:]                                   (f32)
//   z[w,g,t]  = bf16(bf16(Q[w,g,:] . K[t,:]) * scale), -inf where kpos[t] > qpos[w]
//   p[w,g,t]  = exp(z - max_t z) / sum_t exp(z - max_t z)
//   op[w,g]   = sum_t p * pv[g,t]
//   drop[w,t] = sum_g p/max(1-p, eps) * (pv[g,t] - op[w,g])
//   score[t]  = f32(max(risk64(min_w drop), risk64(max_w drop)))     (f64 Bernoulli risk)
// The reference materialises z and p for every (query, group, key) in HBM. Here neither ever
// leaves the chip:
//   1. projected_values_kernel: pv for every key of every segment (VALU, reads V once).
//   2. row_stats_kernel: for each (g, w) row, an online pass over all keys: Q.K^T on MFMA
//      (v_mfma_f32_32x32x16_bf16), the bf16 double rounding, running max / sum / pv-sum.
//      Writes 16 bytes of statistics per row.
//   3. column_scores_kernel: each 128-key tile keeps its K operand in registers, streams every
//      (query tile, group) Q tile through LDS, recomputes Q.K^T on MFMA, forms p from the row
//      statistics, accumulates the drop over groups and the min/max over queries in registers,
//      and finishes with the f64 risk. One score per candidate is the only HBM write.
// Operand layout for every MFMA here: A = 32 keys x 16 k, B = 16 k x 32 queries; lane
// (col = lane % 32, half = lane / 32) supplies key/query `col` at k = half*D/2 + 8*ks + [0,8)
// in k-step ks, so each lane reads one contiguous half row. The accumulator element r of a
// lane is (key 8*(r/4) + 4*half + r%4, query col).
#include <cmath>

#include "lr_common.hpp"

namespace lr {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxGroups = 16;
constexpr int kMaxQueryTiles = 256;  // window <= 8192
constexpr int kTileKeys = 128;       // candidate keys per column-pass workgroup

struct Segment {
  const __bf16* keys;
  const __bf16* values;
  const float* key_positions;
  const __bf16* queries;
  const float* gradient;
  int64_t length, first, last, out_offset, stats_offset, pv_offset;
};

__device__ __forceinline__ Segment load_segment(const int64_t* table, int64_t s) {
  const int64_t* w = table + s * LR_SEG_WORDS;
  Segment g;
  g.keys = reinterpret_cast<const __bf16*>(w[0]);
  g.values = reinterpret_cast<const __bf16*>(w[1]);
  g.key_positions = reinterpret_cast<const float*>(w[2]);
  g.queries = reinterpret_cast<const __bf16*>(w[3]);
  g.gradient = reinterpret_cast<const float*>(w[4]);
  g.length = w[5];
  g.first = w[6];
  g.last = w[7];
  g.out_offset = w[8];
  g.stats_offset = w[9];
  g.pv_offset = w[10];
  return g;
}

__device__ __forceinline__ float bf16_round(float x) {
  return static_cast<float>(static_cast<__bf16>(x));
}

// The logit exactly as the reference forms it: GEMM output rounded to bf16, scaled in f32,
// rounded to bf16 again (scoring.py:184 then csrc/scoring.cu:44-45).
__device__ __forceinline__ float logit_value(float acc, float scale) {
  return bf16_round(bf16_round(acc) * scale);
}

__device__ __forceinline__ int acc_key(int r, int half) { return 8 * (r >> 2) + 4 * half + (r & 3); }

__device__ __forceinline__ f32x16 mfma_tile_zero() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ double softplus64(double v) { return v > 20.0 ? v : log1p(exp(v)); }

__device__ __forceinline__ double risk64(double margin, double probability, double base_softplus,
                                         float drop) {
  const double compared = margin - static_cast<double>(drop);
  return fmax(0.0, probability * (margin - compared) - base_softplus + softplus64(compared));
}

// ---------------------------------------------------------------------------------------
// 1. Projected values pv[g, t] = grad[g] . V[t] for every key of every segment. A lane group
// of D/8 lanes reads one V row with 16-byte loads (fully coalesced); each lane forms its
// 8-column partial dot product per group and the group reduces across its lanes.
template <int D>
__global__ __launch_bounds__(256) void projected_values_kernel(const int64_t* __restrict__ table,
                                                               int64_t groups,
                                                               float* __restrict__ pv,
                                                               int* __restrict__ nonfinite) {
  constexpr int LPR = D / 8;         // lanes per row
  constexpr int RPB = 256 / LPR;     // rows per block step
  __shared__ float grad[kMaxGroups * D];
  const Segment seg = load_segment(table, blockIdx.y);
  if (nonfinite != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *nonfinite = 0;
  for (int64_t i = threadIdx.x; i < groups * D; i += 256) grad[i] = seg.gradient[i];
  __syncthreads();
  const int lane = threadIdx.x % LPR;
  const int64_t row_slot = threadIdx.x / LPR;
  float* out = pv + seg.pv_offset;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * RPB + row_slot; t < seg.length;
       t += static_cast<int64_t>(gridDim.x) * RPB) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(seg.values + t * D + 8 * lane);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = static_cast<float>(v[e]);
    for (int64_t g = 0; g < groups; ++g) {
      const float* w = grad + g * D + 8 * lane;
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(w[e], x[e], acc);
#pragma unroll
      for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, LPR);
      if (lane == 0) out[g * seg.length + t] = acc;
    }
  }
}

// Stages a 32-row bf16 tile (rows src_row0.., D wide, rows >= valid_rows zero) into LDS with
// a 16-byte pad per row. All 256 threads participate.
template <int D>
struct TileStager {
  static constexpr int kChunks = 32 * D / 8;  // 16-byte chunks per tile
  static constexpr int kPerThread = (kChunks + 255) / 256;
  uint4 data[kPerThread];

  __device__ __forceinline__ void load(const __bf16* base, int64_t valid_rows) {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c / (D / 8), part = c % (D / 8);
      data[i] = make_uint4(0, 0, 0, 0);
      if (c < kChunks && row < valid_rows)
        data[i] = *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(row) * D + 8 * part);
    }
  }
  __device__ __forceinline__ void store(__bf16* lds) const {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c / (D / 8), part = c % (D / 8);
      if (c < kChunks) *reinterpret_cast<uint4*>(lds + row * (D + 8) + 8 * part) = data[i];
    }
  }
};

// ---------------------------------------------------------------------------------------
// 2. Row statistics. One wave per (group, 32-query tile) task, four tasks per workgroup; the
// workgroup streams all key tiles of its segment through LDS (double buffered).
// Output per row (g, w): {-m*log2(e), S, eps*S, op} with m the masked row max, S the sum of
// exp(z - m) and op = sum exp(z - m) * pv / S; {NaN x4} for a fully masked row.
template <int D>
__global__ __launch_bounds__(256) void row_stats_kernel(
    const int64_t* __restrict__ table, int64_t groups, int64_t window, int64_t query_stride,
    const int64_t* __restrict__ query_positions, float scale, float epsilon,
    int64_t wg_per_segment, const float* __restrict__ pv, float4* __restrict__ stats) {
  constexpr int KS = D / 16;
  constexpr int ROW = D + 8;
  __shared__ __bf16 k_lds[2][32 * ROW];
  __shared__ float pv_lds[2][kMaxGroups * 32];
  __shared__ float kpos_lds[2][32];
  __shared__ float kmax_lds[2];

  const int64_t s = blockIdx.x / wg_per_segment;
  const int64_t wg = blockIdx.x % wg_per_segment;
  const Segment seg = load_segment(table, s);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = lane >> 5, col = lane & 31;
  const int64_t qtiles = (window + 31) / 32;
  const int64_t task = wg * 4 + wave;
  const bool active = task < groups * qtiles;
  const int64_t g = active ? task / qtiles : 0;
  const int64_t query = (active ? task % qtiles : 0) * 32 + col;
  const bool query_valid = active && query < window;
  const float query_position =
      query_valid ? static_cast<float>(query_positions[query]) : -INFINITY;

  bf16x8 qop[KS];
  {
    const __bf16* qrow = seg.queries + (g * query_stride + query) * D + half * (D / 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<__bf16>(0.0f);
      if (query_valid) v = *reinterpret_cast<const bf16x8*>(qrow + 8 * ks);
      qop[ks] = v;
    }
  }
  float qmin = query_valid ? query_position : INFINITY;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) qmin = fminf(qmin, __shfl_xor(qmin, o, 64));

  const int64_t length = seg.length;
  const int64_t ktiles = (length + 31) / 32;
  const float* pv_seg = pv + seg.pv_offset;

  TileStager<D> stager;
  float pv_reg[2] = {0.0f, 0.0f};
  float kpos_reg = INFINITY;
  auto fetch = [&](int64_t kt) {
    const int64_t t0 = kt * 32;
    stager.load(seg.keys + t0 * D, length - t0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int gg = idx / 32, k = idx % 32;
      pv_reg[i] = (gg < groups && t0 + k < length) ? pv_seg[gg * length + t0 + k] : 0.0f;
    }
    kpos_reg = (threadIdx.x < 32 && t0 + threadIdx.x < length) ? seg.key_positions[t0 + threadIdx.x]
                                                                : INFINITY;
  };
  auto commit = [&](int buf) {
    stager.store(k_lds[buf]);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx < kMaxGroups * 32) pv_lds[buf][idx] = pv_reg[i];
    }
    if (threadIdx.x < 32) {
      kpos_lds[buf][threadIdx.x] = kpos_reg;
      float m = kpos_reg;
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      if (threadIdx.x == 0) kmax_lds[buf] = m;
    }
  };

  float m_run = -INFINITY, S = 0.0f, A = 0.0f;
  fetch(0);
  commit(0);
  __syncthreads();
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) fetch(kt + 1);
    if (active) {
      f32x16 acc = mfma_tile_zero();
      const __bf16* arow = k_lds[buf] + col * ROW + half * (D / 2);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + 8 * ks);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[ks], acc, 0, 0, 0);
      }
      const bool need_mask = kmax_lds[buf] > qmin;
      float z[16];
      float tile_max = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = logit_value(acc[r], scale);
        if (need_mask) v = kpos_lds[buf][acc_key(r, half)] <= query_position ? v : -INFINITY;
        z[r] = v;
        tile_max = fmaxf(tile_max, v);
      }
      const float m_new = fmaxf(m_run, tile_max);
      const float factor = (m_run == m_new) ? 1.0f : __builtin_amdgcn_exp2f((m_run - m_new) * kLog2e);
      S *= factor;
      A *= factor;
      const float nml = (m_new == -INFINITY) ? 0.0f : -m_new * kLog2e;
      const float* pv_row = pv_lds[buf] + g * 32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z[r], kLog2e, nml));
        S += e;
        A = __builtin_fmaf(e, pv_row[acc_key(r, half)], A);
      }
      m_run = m_new;
    }
    if (kt + 1 < ktiles) commit(buf ^ 1);
    __syncthreads();
  }
  // Merge the two half-waves (same query, disjoint keys).
  const float m_other = __shfl_xor(m_run, 32, 64);
  const float S_other = __shfl_xor(S, 32, 64);
  const float A_other = __shfl_xor(A, 32, 64);
  if (!query_valid || half != 0) return;
  const float m = fmaxf(m_run, m_other);
  float4 out;
  if (m == -INFINITY) {
    out = make_float4(NAN, NAN, NAN, NAN);
  } else {
    const float f1 = (m_run == m) ? 1.0f : __builtin_amdgcn_exp2f((m_run - m) * kLog2e);
    const float f2 = (m_other == m) ? 1.0f : __builtin_amdgcn_exp2f((m_other - m) * kLog2e);
    const float total = S * f1 + S_other * f2;
    const float weighted = A * f1 + A_other * f2;
    out = make_float4(-m * kLog2e, total, epsilon * total, weighted / total);
  }
  stats[seg.stats_offset + g * window + query] = out;
}

// ---------------------------------------------------------------------------------------
// 3. Column scores. Workgroup = 128 candidate keys (4 waves x 32, K operand resident in
// registers); streams the G * ceil(W/32) Q tiles through LDS in (query tile, group) order.
template <int D>
__global__ __launch_bounds__(256) void column_scores_kernel(
    const int64_t* __restrict__ table, int64_t groups, int64_t window, int64_t query_stride,
    const int64_t* __restrict__ query_positions, const float* __restrict__ margin, float scale,
    int64_t tiles_per_segment, const float* __restrict__ pv, const float4* __restrict__ stats,
    float* __restrict__ scores, int* __restrict__ nonfinite) {
  constexpr int KS = D / 16;
  constexpr int ROW = D + 8;
  __shared__ __bf16 q_lds[2][32 * ROW];
  __shared__ float pv_lds[kMaxGroups * kTileKeys];
  __shared__ float kpos_lds[kTileKeys];
  __shared__ int keybad_lds[kTileKeys];
  __shared__ float qmin_lds[kMaxQueryTiles];

  const int64_t s = blockIdx.x / tiles_per_segment;
  const int64_t tile = blockIdx.x % tiles_per_segment;
  const Segment seg = load_segment(table, s);
  const int64_t count = seg.last - seg.first;
  if (tile * kTileKeys >= count) return;  // uniform across the workgroup, before any barrier
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = lane >> 5, col = lane & 31;
  const int64_t length = seg.length;
  const int64_t key0 = seg.first + tile * kTileKeys;
  const int64_t wave_key0 = key0 + wave * 32;
  const int64_t qtiles = (window + 31) / 32;
  const float* pv_seg = pv + seg.pv_offset;

  // K operand of this wave's 32 keys.
  bf16x8 kop[KS];
  {
    const int64_t key = wave_key0 + col;
    const __bf16* krow = seg.keys + key * D + half * (D / 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<__bf16>(0.0f);
      if (key < length) v = *reinterpret_cast<const bf16x8*>(krow + 8 * ks);
      kop[ks] = v;
    }
  }
  for (int64_t i = threadIdx.x; i < groups * kTileKeys; i += 256) {
    const int64_t gg = i / kTileKeys, key = key0 + i % kTileKeys;
    pv_lds[i] = key < length ? pv_seg[gg * length + key] : 0.0f;
  }
  if (threadIdx.x < kTileKeys) {
    const int64_t key = key0 + threadIdx.x;
    kpos_lds[threadIdx.x] = key < length ? seg.key_positions[key] : INFINITY;
  }
  for (int64_t i = threadIdx.x; i < qtiles; i += 256) {
    float m = INFINITY;
    for (int64_t w = i * 32; w < i * 32 + 32 && w < window; ++w)
      m = fminf(m, static_cast<float>(query_positions[w]));
    qmin_lds[i] = m;
  }
  __syncthreads();
  if (threadIdx.x < kTileKeys) {
    int bad = 0;
    for (int64_t gg = 0; gg < groups; ++gg) bad |= !isfinite(pv_lds[gg * kTileKeys + threadIdx.x]);
    keybad_lds[threadIdx.x] = bad;
  }
  // Largest candidate key position of this wave (keys at or past `last` never matter).
  float kmax = (wave_key0 + col < seg.last) ? kpos_lds[wave * 32 + col] : -INFINITY;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) kmax = fmaxf(kmax, __shfl_xor(kmax, o, 64));

  const int64_t units = qtiles * groups;
  TileStager<D> stager;
  auto fetch = [&](int64_t u) {
    const int64_t qt = u / groups, gg = u % groups;
    stager.load(seg.queries + (gg * query_stride + qt * 32) * D, window - qt * 32);
  };

  float drop[16], lo[16], hi[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    drop[r] = 0.0f;
    lo[r] = INFINITY;
    hi[r] = -INFINITY;
  }
  int row_bad = 0;
  float query_position = 0.0f;
  fetch(0);
  stager.store(q_lds[0]);
  __syncthreads();
  for (int64_t u = 0; u < units; ++u) {
    const int buf = u & 1;
    if (u + 1 < units) fetch(u + 1);
    const int64_t qt = u / groups, g = u % groups;
    const int64_t query = qt * 32 + col;
    const bool query_valid = query < window;
    if (g == 0) query_position = query_valid ? static_cast<float>(query_positions[query]) : 0.0f;
    float4 st = make_float4(0.0f, 1.0f, 1.0f, 0.0f);
    if (query_valid) {
      st = stats[seg.stats_offset + g * window + query];
      row_bad |= !(isfinite(st.x) && isfinite(st.y) && isfinite(st.w));
    }
    f32x16 acc = mfma_tile_zero();
    const __bf16* brow = q_lds[buf] + col * ROW + half * (D / 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(brow + 8 * ks);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[ks], b, acc, 0, 0, 0);
    }
    const bool need_mask = kmax > qmin_lds[qt];
    const float* pv_row = pv_lds + g * kTileKeys + wave * 32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = acc_key(r, half);
      float z = logit_value(acc[r], scale);
      if (need_mask) z = kpos_lds[wave * 32 + key] <= query_position ? z : -INFINITY;
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z, kLog2e, st.x));
      const float den = fmaxf(st.y - e, st.z);
      const float ratio = e * __builtin_amdgcn_rcpf(den);
      drop[r] = __builtin_fmaf(ratio, pv_row[key] - st.w, drop[r]);
    }
    if (g == groups - 1) {
      if (query_valid) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          lo[r] = fminf(lo[r], drop[r]);
          hi[r] = fmaxf(hi[r], drop[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) drop[r] = 0.0f;
    }
    if (u + 1 < units) stager.store(q_lds[buf ^ 1]);
    __syncthreads();
  }
  // Reduce over the 32 query lanes of each half (same keys, different queries).
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      lo[r] = fminf(lo[r], __shfl_xor(lo[r], o, 64));
      hi[r] = fmaxf(hi[r], __shfl_xor(hi[r], o, 64));
    }
  }
  const bool any_row_bad = __any(row_bad);
  if (col >= 16) return;
  float mn = lo[0], mx = hi[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) {
    if (col == r) {
      mn = lo[r];
      mx = hi[r];
    }
  }
  const int key_local = wave * 32 + acc_key(col, half);
  const int64_t key = key0 + key_local;
  if (key >= seg.last) return;
  float score;
  if (any_row_bad || keybad_lds[key_local] || !isfinite(mn) || !isfinite(mx)) {
    score = NAN;
  } else {
    const double m = static_cast<double>(margin[0]);
    const double p = 1.0 / (1.0 + exp(-m));
    const double base = softplus64(m);
    score = static_cast<float>(fmax(risk64(m, p, base, mn), risk64(m, p, base, mx)));
  }
  scores[seg.out_offset + (key - seg.first)] = score;
  if (nonfinite != nullptr && !isfinite(score)) atomicAdd(nonfinite, 1);
}

// ---------------------------------------------------------------------------------------
// Test hook: raw bf16 logits of one segment with the same operand layout and MFMA order.
template <int D>
__global__ __launch_bounds__(64) void debug_logits_kernel(const int64_t* __restrict__ table,
                                                         int64_t segment, int64_t window,
                                                         int64_t query_stride, int64_t length,
                                                         uint16_t* __restrict__ out) {
  constexpr int KS = D / 16;
  const Segment seg = load_segment(table, segment);
  const int lane = threadIdx.x, half = lane >> 5, col = lane & 31;
  const int64_t kt = blockIdx.x, qt = blockIdx.y, g = blockIdx.z;
  const int64_t key = kt * 32 + col, query = qt * 32 + col;
  f32x16 acc = mfma_tile_zero();
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = static_cast<__bf16>(0.0f);
      b[e] = static_cast<__bf16>(0.0f);
    }
    if (key < length)
      a = *reinterpret_cast<const bf16x8*>(seg.keys + key * D + half * (D / 2) + 8 * ks);
    if (query < window)
      b = *reinterpret_cast<const bf16x8*>(seg.queries + (g * query_stride + query) * D +
                                           half * (D / 2) + 8 * ks);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
  if (query >= window) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = kt * 32 + acc_key(r, half);
    if (t < length) {
      const __bf16 v = static_cast<__bf16>(acc[r]);
      out[(g * window + query) * length + t] = *reinterpret_cast<const uint16_t*>(&v);
    }
  }
}

inline size_t align256(size_t v) { return (v + 255) & ~size_t{255}; }

template <int D>
int launch_score(const int64_t* table, int64_t segments, int64_t groups, int64_t window,
                 int64_t max_length, int64_t max_candidates, int64_t query_stride,
                 const int64_t* query_positions, const float* margin, float scale, float eps,
                 float4* stats, float* pv, float* scores, int* nonfinite, int stages,
                 hipStream_t stream) {
  if (stages & 1) {
    constexpr int rows_per_block = 256 / (D / 8);
    dim3 pv_grid(static_cast<unsigned>(ceil_div(max_length, 4 * rows_per_block)),
                 static_cast<unsigned>(segments));
    projected_values_kernel<D><<<pv_grid, 256, 0, stream>>>(table, groups, pv, nonfinite);
    if (int rc = check_launch("projected_values")) return rc;
  }
  if (stages & 2) {
    const int64_t qtiles = ceil_div(window, 32);
    const int64_t wg_per_segment = ceil_div(groups * qtiles, 4);
    row_stats_kernel<D><<<static_cast<unsigned>(segments * wg_per_segment), 256, 0, stream>>>(
        table, groups, window, query_stride, query_positions, scale, eps, wg_per_segment, pv,
        stats);
    if (int rc = check_launch("row_stats")) return rc;
  }
  if (stages & 4) {
    const int64_t tiles = ceil_div(max_candidates, kTileKeys);
    column_scores_kernel<D><<<static_cast<unsigned>(segments * tiles), 256, 0, stream>>>(
        table, groups, window, query_stride, query_positions, margin, scale, tiles, pv, stats,
        scores, nonfinite);
    if (int rc = check_launch("column_scores")) return rc;
  }
  return LR_OK;
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" size_t lr_score_workspace_bytes(int64_t segments, int64_t groups, int64_t window,
                                           int64_t projected_floats) {
  if (segments < 0 || groups < 0 || window < 0 || projected_floats < 0) return 0;
  return align256(static_cast<size_t>(segments * groups * window) * sizeof(float4)) +
         align256(static_cast<size_t>(projected_floats) * sizeof(float));
}

extern "C" int lr_score_segments(const int64_t* segment_table, int64_t segments, int64_t groups,
                                 int64_t window, int64_t dim, int64_t max_length,
                                 int64_t max_candidates, int64_t query_group_stride,
                                 const int64_t* query_positions, const float* margin,
                                 float scale, double epsilon, void* workspace,
                                 size_t workspace_bytes, float* scores, int32_t* nonfinite,
                                 int stages, void* stream) {
  clear_error();
  LR_REQUIRE(segments > 0 && groups > 0 && window > 0, "Empty attention dimensions");
  LR_REQUIRE(groups <= kMaxGroups, "At most 16 query heads per KV head are supported");
  LR_REQUIRE(window <= 32 * kMaxQueryTiles, "Query window exceeds 8192");
  LR_REQUIRE(dim == 64 || dim == 128 || dim == 256, "Fused scorer supports head_dim 64/128/256");
  LR_REQUIRE(max_length > 0 && max_candidates > 0 && max_candidates <= max_length,
             "Invalid candidate interval");
  LR_REQUIRE(query_group_stride >= window, "Invalid query layout");
  LR_REQUIRE(epsilon > 0.0, "Chunk size and denominator epsilon must be positive");
  LR_REQUIRE(stages >= 0 && stages <= 7, "stages is a bitmask of 1 | 2 | 4");
  LR_REQUIRE(segment_table && query_positions && margin && workspace && scores,
             "Expected contiguous CUDA tensor");
  LR_REQUIRE(segments * ceil_div(max_candidates, kTileKeys) < (int64_t{1} << 31),
             "Too many segments");
  // The projected-value floats needed are bounded by segments * groups * max_length; the
  // caller sized the workspace with the same bound through lr_score_workspace_bytes.
  const size_t stats_bytes = align256(static_cast<size_t>(segments * groups * window) * sizeof(float4));
  const size_t need = lr_score_workspace_bytes(segments, groups, window, segments * groups * max_length);
  LR_REQUIRE(workspace_bytes >= need, "Workspace too small");
  float4* stats = static_cast<float4*>(workspace);
  float* pv = reinterpret_cast<float*>(static_cast<char*>(workspace) + stats_bytes);
  const hipStream_t s = as_stream(stream);
  const float eps = static_cast<float>(epsilon);
  switch (dim) {
    case 64:
      return launch_score<64>(segment_table, segments, groups, window, max_length, max_candidates,
                              query_group_stride, query_positions, margin, scale, eps, stats, pv,
                              scores, nonfinite, stages == 0 ? 7 : stages, s);
    case 128:
      return launch_score<128>(segment_table, segments, groups, window, max_length, max_candidates,
                               query_group_stride, query_positions, margin, scale, eps, stats, pv,
                               scores, nonfinite, stages == 0 ? 7 : stages, s);
    default:
      return launch_score<256>(segment_table, segments, groups, window, max_length, max_candidates,
                               query_group_stride, query_positions, margin, scale, eps, stats, pv,
                               scores, nonfinite, stages == 0 ? 7 : stages, s);
  }
}

extern "C" int lr_debug_segment_logits(const int64_t* segment_table, int64_t segment,
                                       int64_t groups, int64_t window, int64_t dim,
                                       int64_t length, int64_t query_group_stride, uint16_t* out,
                                       void* stream) {
  clear_error();
  LR_REQUIRE(groups > 0 && window > 0 && length > 0 && segment >= 0, "Empty attention dimensions");
  LR_REQUIRE(dim == 64 || dim == 128 || dim == 256, "Fused scorer supports head_dim 64/128/256");
  LR_REQUIRE(groups <= 65535 && ceil_div(window, 32) <= 65535, "Too many query tiles");
  LR_REQUIRE(segment_table && out, "Expected contiguous CUDA tensor");
  dim3 grid(static_cast<unsigned>(ceil_div(length, 32)), static_cast<unsigned>(ceil_div(window, 32)),
            static_cast<unsigned>(groups));
  const hipStream_t s = as_stream(stream);
  switch (dim) {
    case 64:
      debug_logits_kernel<64><<<grid, 64, 0, s>>>(segment_table, segment, window,
                                                  query_group_stride, length, out);
      break;
    case 128:
      debug_logits_kernel<128><<<grid, 64, 0, s>>>(segment_table, segment, window,
                                                   query_group_stride, length, out);
      break;
    default:
      debug_logits_kernel<256><<<grid, 64, 0, s>>>(segment_table, segment, window,
                                                   query_group_stride, length, out);
      break;
  }
  return check_launch("debug_segment_logits");
}
