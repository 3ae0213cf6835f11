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
//   1. projected_values_kernel: pv for every key of every segment (VALU, reads V once), and
//      once the margin's terms of the risk (sigmoid and softplus of the margin, f64).
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
#include <type_traits>

#include "lr_common.hpp"

namespace lr {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Loads through the global address space (the segment table holds generic pointers; casting
// lets the compiler emit global_load instead of flat_load).
template <typename T>
__device__ __forceinline__ T gload(const void* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
// The same with a nontemporal load, for data read exactly once (V in the projected-values
// pass: measured faster than the default load on gfx950).
template <typename T>
__device__ __forceinline__ T gload_stream(const void* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) T*)p);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxGroups = 16;
constexpr int kMaxQueryTiles = 256;  // window <= 8192
constexpr int kTileKeys = 128;       // fewest candidate keys per column-pass workgroup
constexpr int kProjectedRowsPerLane = 8;  // V rows each projected-values lane loads at once

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

// x rounded to bf16 (round to nearest even) and returned as f32 in one instruction: the pair
// {0, x} packs bf16(0) = 0x0000 into the low half and bf16(x) into the high half, which is
// exactly the f32 bit pattern of bf16(x).
__device__ __forceinline__ float bf16_round_fast(float x) {
  const f32x2 v = {0.0f, x};
  return __builtin_bit_cast(float, __builtin_convertvector(v, bf16x2));
}

// logit_value with one conversion per rounding step (three VALU ops per logit).
__device__ __forceinline__ float logit_fast(float acc, float scale) {
  return bf16_round_fast(bf16_round_fast(acc) * scale);
}

// What the scorer passes work on. With a power-of-two scale (1/sqrt(d) for d = 64 and 256) the
// second rounding is exact (bf16(x) * 2^k is a bf16 value), so the passes work on u = bf16(acc)
// and fold the scale into the constant that converts logits to exp2 arguments: every use is
// z * log2(e) = u * (scale * log2(e)) with scale * log2(e) exact, in an FMA that rounds once,
// and max(z) = scale * max(u). One conversion per logit instead of two and a multiply.
template <bool P2>
__device__ __forceinline__ float logit_input(float acc, float scale) {
  if constexpr (P2) return bf16_round_fast(acc);
  else return logit_fast(acc, scale);
}
template <bool P2>
__device__ __forceinline__ float log2e_per_input(float scale) {
  if constexpr (P2) return scale * kLog2e;
  else return kLog2e;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// IEEE 754-2019 minimum / maximum (NaN-propagating, -0 < +0) of three values in one
// instruction; the compiler forms these only with a repeated operand.
__device__ __forceinline__ float minimum3(float a, float b, float c) {
  float r;
  asm("v_minimum3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float maximum3(float a, float b, float c) {
  float r;
  asm("v_maximum3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ f32x16 mfma_tile_zero() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ double softplus64(double v) { return v > 20.0 ? v : log1p(exp(v)); }

// The margin's terms of the risk, the same for every candidate: p = sigmoid(m) and
// softplus(m). The first scorer kernel computes them once into the workspace.
struct RiskTerms {
  double probability, base_softplus;
};
__device__ __forceinline__ RiskTerms risk_terms(float margin) {
  const double m = static_cast<double>(margin);
  return RiskTerms{1.0 / (1.0 + exp(-m)), softplus64(m)};
}

__device__ __forceinline__ double risk64(double margin, double probability, double base_softplus,
                                         float drop) {
  const double compared = margin - static_cast<double>(drop);
  return fmax(0.0, probability * (margin - compared) - base_softplus + softplus64(compared));
}

// ---------------------------------------------------------------------------------------
// 1. Projected values pv[g, t] = grad[g] . V[t] for every key of every segment. A lane group
// of D/8 lanes reads one V row with 16-byte loads (fully coalesced); each lane issues all its
// kRows row loads before any arithmetic, so several loads per lane are in flight. Per chunk of
// four groups, a lane holds 16 partial sums (4 rows x 4 groups, each over its 8 columns); a
// reduce-scatter across the lane group (DPP exchanges within a 16-lane row, a shuffle across
// rows) leaves every lane with whole sums, which it stores.
constexpr int kQuadXor1 = 0xB1;       // DPP quad_perm [1,0,3,2]: partner lane ^ 1
constexpr int kQuadXor2 = 0x4E;       // DPP quad_perm [2,3,0,1]: partner lane ^ 2
constexpr int kRowHalfMirror = 0x141;  // DPP: lane i <-> 7 - i within each 8 lanes (differs in bit 2)
constexpr int kRowMirror = 0x140;      // DPP: lane i <-> 15 - i within each 16 lanes (differs in bit 3)

// The value of the partner lane across lane bit `bit` (partners agree on every higher bit).
template <int BIT>
__device__ __forceinline__ float partner(float x) {
  if constexpr (BIT == 0) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kQuadXor1, 0xF, 0xF, false));
  else if constexpr (BIT == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kQuadXor2, 0xF, 0xF, false));
  else if constexpr (BIT == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kRowHalfMirror, 0xF, 0xF, false));
  else if constexpr (BIT == 3) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kRowMirror, 0xF, 0xF, false));
  else return __shfl_xor(x, 1 << BIT, 64);
}

// Reduce-scatter of v[0..N) over the lane bits BIT..0 of `lane`: each stage keeps the half
// selected by the lane's bit and adds the partner's copy of it; once one value is left the
// remaining stages add it across partners. Afterwards lane L holds the sums of indices
// (L >> (bits left over)) * n + [0, n), n = N >> (BIT + 1) (at least 1).
template <int BIT, int N>
__device__ __forceinline__ void reduce_scatter(float (&v)[16], int lane) {
  const bool upper = (lane >> BIT) & 1;
  if constexpr (N > 1) {
    constexpr int H = N / 2;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float keep = upper ? v[H + i] : v[i];
      const float send = upper ? v[i] : v[H + i];
      v[i] = keep + partner<BIT>(send);
    }
  } else {
    v[0] += partner<BIT>(v[0]);
  }
  if constexpr (BIT > 0) reduce_scatter<BIT - 1, (N > 1 ? N / 2 : 1)>(v, lane);
}

template <int D>
__global__ __launch_bounds__(256) void projected_values_kernel(const int64_t* __restrict__ table,
                                                               int64_t groups64,
                                                               float* __restrict__ pv,
                                                               int* __restrict__ nonfinite,
                                                               const float* __restrict__ margin,
                                                               RiskTerms* __restrict__ terms) {
  constexpr int LPR = D / 8;          // lanes per row (a power of two, 8..32)
  constexpr int LOG_LPR = LPR == 8 ? 3 : LPR == 16 ? 4 : 5;
  static_assert(LPR == (1 << LOG_LPR), "D must be 64, 128 or 256");
  constexpr int RPB = 256 / LPR;      // lane groups per block
  constexpr int kRows = kProjectedRowsPerLane;
  static_assert(kRows % 4 == 0, "rows are reduced four at a time");
  // after the reduce-scatter of 16 values: values per lane, and lanes holding the same sums
  constexpr int kKept = LOG_LPR >= 4 ? 1 : 16 >> LOG_LPR;
  constexpr int kCopies = LOG_LPR > 4 ? 1 << (LOG_LPR - 4) : 1;
  __shared__ float grad[kMaxGroups * D];
  const Segment seg = load_segment(table, blockIdx.y);
  const int groups = static_cast<int>(groups64);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    if (nonfinite != nullptr) *nonfinite = 0;
    *terms = risk_terms(margin[0]);
  }
  for (int i = threadIdx.x; i < groups * D; i += 256) grad[i] = seg.gradient[i];
  const int lane = threadIdx.x % LPR;
  const int length = static_cast<int>(seg.length);
  constexpr int kChunk = kRows * RPB;  // rows per block step
  const int stride = static_cast<int>(gridDim.x) * kChunk;
  float* out = pv + seg.pv_offset;
  // Block steps of kChunk rows, strided over the grid; the next step's rows are loaded while
  // the current step's are reduced.
  auto load = [&](int first, bf16x8 (&raw)[kRows]) {
    const int base = first + static_cast<int>(threadIdx.x / LPR);
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      const int t = base + k * RPB;
#pragma unroll
      for (int e = 0; e < 8; ++e) raw[k][e] = static_cast<__bf16>(0.0f);
      if (t < length) raw[k] = gload_stream<bf16x8>(seg.values + static_cast<int64_t>(t) * D + 8 * lane);
    }
  };
  auto reduce = [&](int first, const bf16x8 (&raw)[kRows]) {
    const int base = first + static_cast<int>(threadIdx.x / LPR);
    for (int g0 = 0; g0 < groups; g0 += 4) {
      f32x4 w[4][2];
#pragma unroll
      for (int gl = 0; gl < 4; ++gl) {
        const bool live = g0 + gl < groups;
        w[gl][0] = live ? *reinterpret_cast<const f32x4*>(grad + (g0 + gl) * D + 8 * lane) : f32x4{0, 0, 0, 0};
        w[gl][1] = live ? *reinterpret_cast<const f32x4*>(grad + (g0 + gl) * D + 8 * lane + 4) : f32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int k0 = 0; k0 < kRows; k0 += 4) {
        float v[16];  // index 4 * (row k - k0) + group gl
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          float x[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = static_cast<float>(raw[k0 + kk][e]);
#pragma unroll
          for (int gl = 0; gl < 4; ++gl) {
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) a = __builtin_fmaf(w[gl][0][e], x[e], a);
#pragma unroll
            for (int e = 0; e < 4; ++e) a = __builtin_fmaf(w[gl][1][e], x[4 + e], a);
            v[4 * kk + gl] = a;
          }
        }
        reduce_scatter<LOG_LPR - 1, 16>(v, lane);
        if (lane % kCopies == 0) {
#pragma unroll
          for (int j = 0; j < kKept; ++j) {
            const int index = (lane / kCopies) * kKept + j;
            const int t = base + (k0 + index / 4) * RPB;
            const int g = g0 + index % 4;
            if (t < length && g < groups) out[static_cast<int64_t>(g) * length + t] = v[j];
          }
        }
      }
    }
  };
  int first = static_cast<int>(blockIdx.x) * kChunk;
  bf16x8 cur[kRows], next[kRows];
  load(first, cur);
  __syncthreads();  // gradient in LDS
  for (; first < length; first += stride) {
    if (first + stride < length) load(first + stride, next);
    reduce(first, cur);
#pragma unroll
    for (int k = 0; k < kRows; ++k) cur[k] = next[k];
  }
}

// Direct global -> LDS copies (global_load_lds_dword / _dwordx4): lane L of a wave writes its
// granule at LDS `wave_base` + L * granule; `wave_base` must be the same for the whole wave.
// Nothing passes through VGPRs. Completion is awaited with dma_wait() before the barrier that
// publishes the data.
// The copies are issued by inline assembly, not by the compiler's builtin: for the builtin the
// compiler makes every later LDS read that it cannot prove disjoint from the copy wait for it
// (s_waitcnt vmcnt(0)), and a buffer picked at run time is never provably disjoint, so the
// copy of the next stage would be waited for at the first read of the current one. Copies the
// compiler does not see only lengthen its own vmcnt waits (counts drain in order), never
// shorten them. M0 (the wave's LDS base for the copy) is set inside the same statement; no
// compiler-generated code in these kernels keeps a value in M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is a reserved register; clobbered on purpose
// Copy from a per-lane address to the (wave-uniform) LDS byte address `lds`.
__device__ __forceinline__ void dma16_to(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4_to(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(src), "s"(lds) : "memory", "m0");
}
// The same copies addressed as a wave-uniform base (an SGPR pair) plus a per-lane 32-bit byte
// offset: the per-copy address arithmetic is then scalar, and a lane's offset can be computed
// once.
__device__ __forceinline__ void dma16_at(const void* base, uint32_t offset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(offset), "s"(base), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4_at(const void* base, uint32_t offset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(offset), "s"(base), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a __shared__ object.
template <typename T>
__device__ __forceinline__ uint32_t lds_address(T* object) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) T*)object));
}

__device__ __forceinline__ uint32_t wave_index() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// vmcnt(0) through the builtin, so that the compiler knows every vector-memory load has landed
// here (loads issued before a loop, such as the resident MFMA operands, are then not waited for
// again inside it); the empty statement keeps LDS accesses from moving across the wait.
__device__ __forceinline__ void dma_wait() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
  asm volatile("" ::: "memory");
}

// Swizzled LDS rows: D bf16 per row, no padding; 16-byte chunk c of row r is stored in chunk
// slot c ^ (r % P), so the lanes that read chunk c of consecutive rows (an MFMA operand) touch
// P different 16-byte bank groups per P rows. P = 16 for d = 128 (its 16 chunks per row allow
// it; measured 2% faster in the row pass than P = 8), else 8.
template <int D>
constexpr int swizzle_period() { return D == 128 ? 16 : 8; }

template <int D>
__device__ __forceinline__ int swizzled_chunk(int row, int chunk) {
  return chunk ^ (row & (swizzle_period<D>() - 1));
}

// DMA of `ROWS` consecutive rows (row0..) of a [*, D] bf16 matrix into swizzled LDS rows at LDS
// byte address `lds`; rows at or past `last_row` re-read row `last_row` (callers mask them). All
// 256 threads call it. Copy i moves rows [i * RPI, (i + 1) * RPI), RPI = 256 / (D / 8), a
// multiple of the swizzle period, so a thread's (row % RPI, chunk) and hence its swizzled byte
// offset within the copy (`dma_row_offset`) are the same for every i: while every row lies
// before `last_row` the addresses are a scalar base plus that fixed offset.
template <int D>
__device__ __forceinline__ uint32_t dma_row_offset() {
  constexpr int CH = D / 8;
  const int row = threadIdx.x / CH, chunk = threadIdx.x % CH;
  return static_cast<uint32_t>((row * D + 8 * swizzled_chunk<D>(row, chunk)) * 2);
}

template <int D, int ROWS>
__device__ __forceinline__ void dma_rows(const __bf16* matrix, int row0, int last_row,
                                         uint32_t lds, uint32_t row_offset) {
  constexpr int CH = D / 8, CHUNKS = ROWS * CH, RPI = 256 / CH;
  static_assert(CHUNKS % 256 == 0 && RPI % swizzle_period<D>() == 0,
                "whole waves per copy, whole swizzle periods");
  const uint32_t wave_lds = lds + wave_index() * 64 * 16;
  if (row0 + ROWS - 1 <= last_row) {
    const char* base = reinterpret_cast<const char*>(matrix + static_cast<int64_t>(row0) * D);
#pragma unroll
    for (int i = 0; i < CHUNKS / 256; ++i)
      dma16_at(base + static_cast<int64_t>(i) * RPI * D * 2, row_offset, wave_lds + 256 * 16 * i);
  } else {
#pragma unroll
    for (int i = 0; i < CHUNKS / 256; ++i) {
      const int slot = 256 * i + threadIdx.x;
      const int row = slot / CH, chunk = slot % CH;
      const int source = min(row0 + row, last_row);
      dma16_to(matrix + static_cast<int64_t>(source) * D + 8 * swizzled_chunk<D>(row, chunk),
               wave_lds + 256 * 16 * i);
    }
  }
}

// ---------------------------------------------------------------------------------------
// 2. Row statistics. One wave per (group, 32-query tile) task, four tasks per workgroup; the
// workgroup streams all key tiles of its segment through LDS (double buffered).
// Output per row (g, w): {-m*log2(e), S, eps*S, op} with m the masked row max, S the sum of
// exp(z - m) and op = sum exp(z - m) * pv / S; {NaN x4} for a fully masked row.
// Three waves per SIMD (at most 168 VGPRs) measure faster here than two without spills for
// d <= 128; d = 256 runs two (at most 256 VGPRs; its 74 KB of LDS also fit two workgroups per CU).
template <int D, bool P2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 3 : 2))) void row_stats_kernel(
    const int64_t* __restrict__ table, int64_t groups64, int64_t window64, int64_t query_stride,
    const int64_t* __restrict__ query_positions, float scale, float epsilon,
    int64_t wg_per_segment, const float* __restrict__ pv, float4* __restrict__ stats) {
  constexpr int KS = D / 16;
  __shared__ __bf16 k_lds[2][64 * D];  // swizzled rows
  __shared__ float pv_lds[2][kMaxGroups * 64];
  __shared__ float kpos_lds[2][64];

  const int groups = static_cast<int>(groups64), window = static_cast<int>(window64);
  const int per = static_cast<int>(wg_per_segment);
  const int block = static_cast<int>(xcd_local_block(blockIdx.x, gridDim.x));
  const int s = block / per;
  const int wg = block - s * per;
  const Segment seg = load_segment(table, s);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = lane >> 5, col = lane & 31;
  const int qtiles = (window + 31) / 32;
  const int task = wg * 4 + wave;
  const bool active = task < groups * qtiles;
  const int g = active ? task / qtiles : 0;
  const int query = (active ? task - (task / qtiles) * qtiles : 0) * 32 + col;
  const bool query_valid = active && query < window;
  const float query_position =
      query_valid ? static_cast<float>(query_positions[query]) : -INFINITY;

  bf16x8 qop[KS];
  {
    const __bf16* qrow = seg.queries + (static_cast<int64_t>(g) * query_stride + query) * D + half * (D / 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<__bf16>(0.0f);
      if (query_valid) v = gload<bf16x8>(qrow + 8 * ks);
      qop[ks] = v;
    }
  }
  float qmin = query_valid ? query_position : INFINITY;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) qmin = fminf(qmin, __shfl_xor(qmin, o, 64));

  const int length = static_cast<int>(seg.length);
  const int ktiles = (length + 63) / 64;  // 64-key stages: two 32-key MFMA tiles each
  const float* pv_seg = pv + seg.pv_offset;

  // Key stage kt -> LDS buffer `buf`, all by direct copy: K rows, projected values and key
  // positions (rows past the end re-read the last row; commit() then gives their positions
  // +inf, which masks them). No compiler-visible load is left in the loop, so no wait the
  // compiler adds can fall between issuing the copies and the stage's LDS reads.
  const uint32_t k_lds0 = lds_address(&k_lds[0][0]), pv_lds0 = lds_address(&pv_lds[0][0]);
  const uint32_t kpos_lds0 = lds_address(&kpos_lds[0][0]);
  const uint32_t row_offset = dma_row_offset<D>();
  const int wave_id = static_cast<int>(wave_index());
  auto fetch = [&](int kt, int buf) {
    const int t0 = kt * 64;
    dma_rows<D, 64>(seg.keys, t0, length - 1, k_lds0 + buf * static_cast<uint32_t>(sizeof(k_lds[0])),
                    row_offset);
    const bool whole = t0 + 63 <= length - 1;  // no row of the stage past the end
    const uint32_t lane_bytes = 4 * (threadIdx.x & 63);
#pragma unroll
    for (int i = 0; i < kMaxGroups / 4; ++i) {
      const int gg = 4 * i + wave_id;  // uniform per wave
      if (gg < groups) {
        const uint32_t dst = pv_lds0 + buf * static_cast<uint32_t>(sizeof(pv_lds[0])) + 4 * (256 * i + 64 * wave_id);
        const float* row = pv_seg + static_cast<int64_t>(gg) * length;
        if (whole) dma4_at(row + t0, lane_bytes, dst);
        else dma4_to(row + min(t0 + static_cast<int>(threadIdx.x & 63), length - 1), dst);
      }
    }
    if (wave_id == 0) {
      const uint32_t dst = kpos_lds0 + buf * static_cast<uint32_t>(sizeof(kpos_lds[0]));
      if (whole) dma4_at(seg.key_positions + t0, lane_bytes, dst);
      else dma4_to(seg.key_positions + min(t0 + static_cast<int>(threadIdx.x), length - 1), dst);
    }
  };
  // After dma_wait(): the wave that copied the key positions overwrites those of rows past the
  // end (its own copy has landed, and LDS accesses of one wave complete in order).
  auto commit = [&](int kt, int buf) {
    if (threadIdx.x < 64 && kt * 64 + static_cast<int>(threadIdx.x) >= length)
      kpos_lds[buf][threadIdx.x] = INFINITY;
  };

  // (log2e_per_input is called at each use: a copy held across the loop cost a register at
  // d = 128 and three waves per SIMD, where the kernel sits at the 168-register limit.)
  float m_run = -INFINITY, S = 0.0f, A = 0.0f;
  // One 64-key stage: 32 logits of this lane (two 32-key tiles, keys acc_key(r, half)).
  auto stage = [&](int buf, auto masked) {
    constexpr bool kMask = decltype(masked)::value;
    float z[32];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      bf16x8 a[KS];
      const __bf16* arow = k_lds[buf] + (32 * t + col) * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        a[ks] = *reinterpret_cast<const bf16x8*>(arow + 8 * swizzled_chunk<D>(col, half * KS + ks));
      f32x16 acc = mfma_tile_zero();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks], qop[ks], acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) z[16 * t + r] = logit_input<P2>(acc[r], scale);
    }
    if constexpr (kMask) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const f32x4 kp = *reinterpret_cast<const f32x4*>(&kpos_lds[buf][8 * c + 4 * half]);
#pragma unroll
        for (int j = 0; j < 4; ++j) z[4 * c + j] = kp[j] <= query_position ? z[4 * c + j] : -INFINITY;
      }
    }
    float tile_max = z[0];
#pragma unroll
    for (int r = 1; r < 32; ++r) tile_max = fmaxf(tile_max, z[r]);
    const float m_new = fmaxf(m_run, tile_max);
    const float factor = (m_run == m_new)
                             ? 1.0f
                             : __builtin_amdgcn_exp2f((m_run - m_new) * log2e_per_input<P2>(scale));
    S *= factor;
    A *= factor;
    const float nml = (m_new == -INFINITY) ? 0.0f : -m_new * log2e_per_input<P2>(scale);
    const float* pv_row = pv_lds[buf] + g * 64;
    // The stage's 32 terms go into partial sums that join the running sums once per stage:
    // a lane's running sums then take one addition per stage instead of one per key, which
    // keeps their rounding error at the reference's level over long heads (33,792 keys:
    // 2e-6 against 3e-5 relative on the scores, per key summed straight into S and A).
    float s_part = 0.0f, a_part = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(pv_row + 8 * c + 4 * half);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e =
            __builtin_amdgcn_exp2f(__builtin_fmaf(z[4 * c + j], log2e_per_input<P2>(scale), nml));
        s_part += e;
        a_part = __builtin_fmaf(e, w[j], a_part);
      }
    }
    S += s_part;
    A += a_part;
    m_run = m_new;
  };

  fetch(0, 0);
  dma_wait();
  commit(0, 0);
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) fetch(kt + 1, buf ^ 1);  // buf ^ 1 was last read before the previous barrier
    if (active) {
      // masked form only if some key of the stage lies after some query of this wave
      if (__any(kpos_lds[buf][lane] > qmin)) stage(buf, std::true_type{});
      else stage(buf, std::false_type{});
    }
    if (more) {
      dma_wait();
      commit(kt + 1, buf ^ 1);
    }
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
    const float lg = log2e_per_input<P2>(scale);
    const float f1 = (m_run == m) ? 1.0f : __builtin_amdgcn_exp2f((m_run - m) * lg);
    const float f2 = (m_other == m) ? 1.0f : __builtin_amdgcn_exp2f((m_other - m) * lg);
    const float total = S * f1 + S_other * f2;
    const float weighted = A * f1 + A_other * f2;
    out = make_float4(-m * lg, total, epsilon * total, weighted / total);
  }
  stats[seg.stats_offset + static_cast<int64_t>(g) * window + query] = out;
}

// ---------------------------------------------------------------------------------------
// 3. Column scores. Workgroup = 4 waves x KT tiles of 32 candidate keys; each wave keeps the
// K operand of its KT tiles in registers. It streams the G * ceil(W/32) (query tile, group)
// units in query-tile-major order through LDS, one unit per double-buffered stage: the 32
// query rows by direct copy into swizzled rows, with each row's statistics and query
// position. A unit's B operand (its 32 query rows) is read from LDS once and multiplied into
// all KT key tiles. After a query tile's last group every lane holds 16 drops per key tile
// (its query x 16 keys); a transpose through LDS reduces them over the tile's queries, so a
// lane keeps one running (min, max) pair per key tile.
// On gfx950 the MFMAs of one wave hide only part of their time behind another wave's VALU
// work (about 60% in a probe of two waves per SIMD), so the kernel is bound by VALU issue plus
// the exposed MFMA time; KT = 2 halves the per-unit overhead (copies, statistics, branches,
// barrier, B reads) per key, at two waves per SIMD.
// Key tiles per wave: two for d = 128 (measured faster there), one for d = 64 (three waves per
// SIMD fit) and d = 256 (the K operand alone takes 64 registers per tile).
template <int D>
constexpr int column_key_tiles() { return D == 128 ? 2 : 1; }

// Transpose scratch of the column reduction: source lane L's 16 drops start at red_slot(L).
// Rows are 20 floats apart (16-byte aligned; 8 or 16 consecutive lanes' 16-byte writes fall in
// distinct banks) and lanes 16..31, 32..47, 48..63 are skewed by 16, 32, 48 floats, so a read
// of one element of 16 consecutive source lanes by the 4 x 16 reducer lanes (same element
// index r, source lanes L = 16 k + q) touches 64 distinct banks (32 per half-wave).
constexpr int kRedStride = 20;
constexpr int kRedFloats = 63 * kRedStride + 48 + 16;
__device__ __forceinline__ int red_slot(int source_lane) {
  return source_lane * kRedStride + 16 * ((source_lane >> 4) & 3);
}

// Waves per SIMD the register budget is held to: two with two key tiles (d = 128) and for
// d = 256 (its 64 KB of LDS also fit two workgroups per CU), three for d = 64.
template <int D>
constexpr int column_waves_per_simd() { return column_key_tiles<D>() == 2 ? 2 : D <= 128 ? 3 : 2; }

// Units per barrier-separated stage: two for d = 128, where the LDS of a second query tile
// fits the two workgroups per CU that the registers allow (halving the barriers per unit;
// measured slightly faster there, slightly slower for d = 64).
template <int D>
constexpr int column_units_per_stage() { return D == 128 ? 2 : 1; }

template <int D, bool P2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(column_waves_per_simd<D>()))) void column_scores_kernel(
    const int64_t* __restrict__ table, int64_t groups64, int64_t window64, int64_t query_stride,
    const int64_t* __restrict__ query_positions, const float* __restrict__ margin, float scale,
    int64_t tiles_per_segment, const float* __restrict__ pv, const float4* __restrict__ stats,
    const RiskTerms* __restrict__ terms, float* __restrict__ scores, int* __restrict__ nonfinite) {
  constexpr int KS = D / 16;
  constexpr int KT = column_key_tiles<D>();
  const float lg = log2e_per_input<P2>(scale);  // logit input -> exp2 argument
  constexpr int kKeys = 4 * 32 * KT;  // candidate keys per workgroup
  constexpr int UP = column_units_per_stage<D>();
  __shared__ __bf16 q_lds[2][UP][32 * D];  // swizzled rows, double-buffered stages of UP units
  __shared__ float4 st_lds[2][UP][32];
  __shared__ float qp_lds[2][UP][32];
  __shared__ float pv_lds[kMaxGroups * kKeys];
  __shared__ float kpos_lds[kKeys];
  __shared__ int keybad_lds[kKeys];
  __shared__ float red_lds[4][kRedFloats];  // per-wave transpose scratch (one key tile at a time)
  __shared__ int rowbad_lds;

  const int groups = static_cast<int>(groups64), window = static_cast<int>(window64);
  const int per = static_cast<int>(tiles_per_segment);
  const int block = static_cast<int>(xcd_local_block(blockIdx.x, gridDim.x));
  const int s = block / per;
  const int tile = block - s * per;
  const Segment seg = load_segment(table, s);
  const int count = static_cast<int>(seg.last - seg.first);
  if (tile * kKeys >= count) return;  // uniform across the workgroup, before any barrier
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = lane >> 5, col = lane & 31;
  const int length = static_cast<int>(seg.length);
  const int key0 = static_cast<int>(seg.first) + tile * kKeys;
  const int wave_key0 = key0 + wave * 32 * KT;  // key tile t: wave_key0 + 32 t + [0, 32)
  const int qtiles = (window + 31) / 32;
  const int units = qtiles * groups;
  const float* pv_seg = pv + seg.pv_offset;
  const float4* stats_seg = stats + seg.stats_offset;

  // K operand of this wave's KT x 32 keys.
  bf16x8 kop[KT][KS];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const int key = wave_key0 + 32 * t + col;
    const __bf16* krow = seg.keys + static_cast<int64_t>(key) * D + half * (D / 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<__bf16>(0.0f);
      if (key < length) v = gload<bf16x8>(krow + 8 * ks);
      kop[t][ks] = v;
    }
  }
  for (int i = threadIdx.x; i < groups * kKeys; i += 256) {
    const int gg = i / kKeys, key = key0 + (i - gg * kKeys);
    pv_lds[i] = key < length ? gload<float>(pv_seg + static_cast<int64_t>(gg) * length + key) : 0.0f;
  }
  for (int i = threadIdx.x; i < kKeys; i += 256) {
    const int key = key0 + i;
    kpos_lds[i] = key < length ? gload<float>(seg.key_positions + key) : INFINITY;
  }
  if (threadIdx.x == 0) rowbad_lds = 0;

  // Stage loader for the (up to) UP units of a stage into buffer buf: the query rows by direct
  // copy (rows past the window re-read the last query; their results are never used), and on
  // lanes 32k..32k+31 of wave 0 the statistics and query positions of the stage's unit k
  // (padded rows and units past the end: harmless values that take the fast epilogue). The
  // statistics loads go first: a wait the compiler adds before them (they reuse the registers
  // of the previous stage's loads) then falls before the copies are issued. Their values are
  // first used in commit(), after the wait that also covers the row copies.
  float4 st_reg = make_float4(0.0f, 2.0f, 0.0f, 0.0f);
  int64_t qp_raw = 0;
  bool row_loaded = false;
  int bad_reg = 0;
  int fetch_u = 0, fetch_qt = 0, fetch_g = 0;  // first unit of the next fetch, (query tile, group)
  const uint32_t q_lds0 = lds_address(&q_lds[0][0][0]);
  const uint32_t row_offset = dma_row_offset<D>();
  auto fetch = [&](int buf) {
    if (threadIdx.x < 32 * UP) {
      const int k = threadIdx.x / 32;
      int g_k = fetch_g + k, qt_k = fetch_qt;
      if (g_k >= groups) g_k -= groups, ++qt_k;
      const int query = qt_k * 32 + threadIdx.x % 32;
      row_loaded = fetch_u + k < units && query < window;
      if (row_loaded) {
        st_reg = stats_seg[static_cast<int64_t>(g_k) * window + query];
        qp_raw = query_positions[query];
      }
    }
#pragma unroll
    for (int k = 0; k < UP; ++k) {
      if (fetch_u < units)
        dma_rows<D, 32>(seg.queries + static_cast<int64_t>(fetch_g) * query_stride * D,
                        fetch_qt * 32, window - 1,
                        q_lds0 + static_cast<uint32_t>((buf * UP + k) * sizeof(q_lds[0][0])),
                        row_offset);
      ++fetch_u;
      if (++fetch_g == groups) {
        fetch_g = 0;
        ++fetch_qt;
      }
    }
  };
  auto commit = [&](int buf) {
    if (threadIdx.x < 32 * UP) {
      float4 st = make_float4(0.0f, 2.0f, 0.0f, 0.0f);  // padded rows take the fast epilogue
      float qp = INFINITY;
      if (row_loaded) {
        st = st_reg;
        qp = static_cast<float>(qp_raw);
        bad_reg |= !(isfinite(st.x) && isfinite(st.y) && isfinite(st.w));
      }
      st_lds[buf][threadIdx.x / 32][threadIdx.x % 32] = st;
      qp_lds[buf][threadIdx.x / 32][threadIdx.x % 32] = qp;
    }
  };
  fetch(0);
  __syncthreads();  // rowbad_lds cleared before any loader may set it
  dma_wait();
  commit(0);
  __syncthreads();
  for (int i = threadIdx.x; i < kKeys; i += 256) {
    int bad = 0;
    for (int gg = 0; gg < groups; ++gg) bad |= !isfinite(pv_lds[gg * kKeys + i]);
    keybad_lds[i] = bad;
  }
  // Largest candidate key position of this wave (keys at or past `last` never matter).
  float kmax = -INFINITY;
#pragma unroll
  for (int t = 0; t < KT; ++t)
    if (wave_key0 + 32 * t + col < seg.last) kmax = fmaxf(kmax, kpos_lds[wave * 32 * KT + 32 * t + col]);
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) kmax = fmaxf(kmax, __shfl_xor(kmax, o, 64));

  float drop[KT][16];
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) drop[t][r] = 0.0f;
  // Reducer role in the tile transpose: lane = (half, r, part); it owns key acc_key(r, half)
  // of each key tile and queries part*16 .. part*16+15 of each query tile; lane ^ 1 owns the
  // other 16.
  const int part = lane & 1, r_red = (lane >> 1) & 15, half_red = lane >> 5;
  float lo[KT], hi[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) lo[t] = INFINITY, hi[t] = -INFINITY;
  float* red = red_lds[wave];
  const float* kpos_wave = kpos_lds + wave * 32 * KT;

  int qt = 0, g = 0;  // unit u = (query tile, group)
  const int stages = (units + UP - 1) / UP;
  for (int stage = 0; stage < stages; ++stage) {
    const int buf = stage & 1;
    // the next stage goes to the other buffer; its last readers passed the previous barrier
    const bool more = stage + 1 < stages;
    if (more) fetch(buf ^ 1);
#pragma unroll
    for (int k = 0; k < UP; ++k) {
    if (stage * UP + k >= units) break;  // uniform
    // A wave whose keys all lie at or past the candidate range's end (the tail of a segment's
    // last workgroup) only takes part in the copies and barriers.
    if (wave_key0 >= seg.last) {
      if (++g == groups) {
        g = 0;
        ++qt;
      }
      continue;
    }
    const float4 st = st_lds[buf][k][col];
    const float query_position = qp_lds[buf][k][col];
    // ratio = p / max(1 - p, eps) = e / max(S - e, eps*S) for the lane's (key, query) pairs.
    // The general form applies the causal mask and the clamp. The fast form drops the clamp,
    // which is exact for every visible key when every row has S >= 2 and eps*S <= 1/2: then
    // e <= 1 gives S - e >= 1 > eps*S. It also takes the ratio as 1 / (S*u - 1) with
    // u = 1/e = exp(m - z), one operation fewer than e / (S - e). Where some key of this wave
    // lies after some query of the unit, the masked fast form sets those pairs' ratios to 0
    // afterwards (whatever the fast form gave for them).
    const bool general = __any(!(st.y >= 2.0f && st.z <= 0.5f));
    const bool masked = __any(kmax > query_position);
    float ratio[KT][16];
    // ratio of key tile t from its logit inputs z (logit_input of the accumulators)
    auto ratio_general = [&](int t, const float (&z_in)[16]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 kp = *reinterpret_cast<const f32x4*>(kpos_wave + 32 * t + 8 * c + 4 * half);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * c + j;
          const float z = kp[j] <= query_position ? z_in[r] : -INFINITY;
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z, lg, st.x));
          ratio[t][r] = e * __builtin_amdgcn_rcpf(fmaxf(st.y - e, st.z));
        }
      }
    };
    auto ratio_fast = [&](int t, const float (&z_in)[16]) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = __builtin_amdgcn_exp2f(__builtin_fmaf(z_in[r], -lg, -st.x));
        ratio[t][r] = __builtin_amdgcn_rcpf(__builtin_fmaf(st.y, v, -1.0f));
      }
    };
    auto ratio_masked = [&](int t, const float (&z_in)[16]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 kp = *reinterpret_cast<const f32x4*>(kpos_wave + 32 * t + 8 * c + 4 * half);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * c + j;
          const float v = __builtin_amdgcn_exp2f(__builtin_fmaf(z_in[r], -lg, -st.x));
          const float q = __builtin_amdgcn_rcpf(__builtin_fmaf(st.y, v, -1.0f));
          ratio[t][r] = kp[j] <= query_position ? q : 0.0f;
        }
      }
    };
    {
      bf16x8 b[KS];
      const __bf16* brow = q_lds[buf][k] + col * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        b[ks] = *reinterpret_cast<const bf16x8*>(brow + 8 * swizzled_chunk<D>(col, half * KS + ks));
      f32x16 acc0 = mfma_tile_zero();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[0][ks], b[ks], acc0, 0, 0, 0);
      float z0[16];
      if constexpr (KT == 2) {
        // Key tile 1's MFMAs run while the wave rounds key tile 0's logits: one MFMA, then its
        // share of that VALU work (a wave issues in order, so the placement is what lets the
        // two overlap). The rounding is common to both forms of the ratio, so it comes before
        // the branch between them.
        constexpr int kPer = 16 / KS;  // tile-0 elements per tile-1 MFMA
        __builtin_amdgcn_sched_barrier(0);  // tile 0's MFMAs stay ahead of this region
        f32x16 acc1 = mfma_tile_zero();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[1][ks], b[ks], acc1, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < kPer; ++e) z0[ks * kPer + e] = logit_input<P2>(acc0[ks * kPer + e], scale);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, (P2 ? 1 : 3) * kPer, 0);
        }
        float z1[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) z1[r] = logit_input<P2>(acc1[r], scale);
        if (general) {
          ratio_general(0, z0);
          ratio_general(1, z1);
        } else if (masked) {
          ratio_masked(0, z0);
          ratio_masked(1, z1);
        } else {
          ratio_fast(0, z0);
          ratio_fast(1, z1);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) z0[r] = logit_input<P2>(acc0[r], scale);
        if (general) ratio_general(0, z0);
        else if (masked) ratio_masked(0, z0);
        else ratio_fast(0, z0);
      }
    }
    // The drops restart with each query tile: its first group writes them, the others add.
    const float* pv_row = pv_lds + g * kKeys + wave * 32 * KT;
    if (g == 0) {
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 w = *reinterpret_cast<const f32x4*>(pv_row + 32 * t + 8 * c + 4 * half);
#pragma unroll
          for (int j = 0; j < 4; ++j) drop[t][4 * c + j] = ratio[t][4 * c + j] * (w[j] - st.w);
        }
    } else {
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 w = *reinterpret_cast<const f32x4*>(pv_row + 32 * t + 8 * c + 4 * half);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            drop[t][4 * c + j] = __builtin_fmaf(ratio[t][4 * c + j], w[j] - st.w, drop[t][4 * c + j]);
        }
    }
    if (g == groups - 1) {
      // Min / max of each key tile's drops over the query tile's queries, through this wave's
      // LDS scratch. LDS accesses of one wave complete in order, so the reads see this wave's
      // writes (and the next tile's writes follow this tile's reads).
      const int valid = min(max(window - qt * 32 - part * 16, 0), 16);  // padded queries skipped
#pragma unroll
      for (int t = 0; t < KT; ++t) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<f32x4*>(red + red_slot(lane) + 4 * c) =
              f32x4{drop[t][4 * c], drop[t][4 * c + 1], drop[t][4 * c + 2], drop[t][4 * c + 3]};
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        const float* column = red + red_slot(half_red * 32 + part * 16) + r_red;
        float tile_lo = INFINITY, tile_hi = -INFINITY;
        // NaN-propagating, as torch's amin / amax
        if (valid == 16) {
#pragma unroll
          for (int q = 0; q < 16; q += 2) {  // three-input minimum / maximum
            const float x0 = column[q * kRedStride], x1 = column[(q + 1) * kRedStride];
            tile_lo = minimum3(tile_lo, x0, x1);
            tile_hi = maximum3(tile_hi, x0, x1);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const float x = column[q * kRedStride];
            tile_lo = __builtin_elementwise_minimum(tile_lo, q < valid ? x : INFINITY);
            tile_hi = __builtin_elementwise_maximum(tile_hi, q < valid ? x : -INFINITY);
          }
        }
        lo[t] = __builtin_elementwise_minimum(lo[t], tile_lo);
        hi[t] = __builtin_elementwise_maximum(hi[t], tile_hi);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      }
    }
    if (++g == groups) {
      g = 0;
      ++qt;
    }
    }  // unit k of the stage
    if (more) {
      dma_wait();
      commit(buf ^ 1);
    }
    __syncthreads();
  }
  if (bad_reg) rowbad_lds = 1;
  __syncthreads();
  const bool any_row_bad = rowbad_lds != 0;
  const double m = static_cast<double>(margin[0]);
  const double p = terms->probability, base = terms->base_softplus;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    // Combine the two reducer lanes of each key, then part 0 takes the risk of the minimum and
    // part 1 of the maximum (f64, every lane busy).
    const float mn = __builtin_elementwise_minimum(lo[t], __shfl_xor(lo[t], 1, 64));
    const float mx = __builtin_elementwise_maximum(hi[t], __shfl_xor(hi[t], 1, 64));
    const int key_local = wave * 32 * KT + 32 * t + acc_key(r_red, half_red);
    const int key = key0 + key_local;
    const bool bad = any_row_bad || keybad_lds[key_local] || !isfinite(mn) || !isfinite(mx);
    const double risk = bad ? 0.0 : risk64(m, p, base, part ? mx : mn);
    const double other_risk = __shfl_xor(risk, 1, 64);
    if (part == 0 && key < seg.last) {
      const float score = bad ? NAN : static_cast<float>(fmax(risk, other_risk));
      scores[seg.out_offset + (key - seg.first)] = score;
      if (nonfinite != nullptr && !isfinite(score)) atomicAdd(nonfinite, 1);
    }
  }
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
                 float4* stats, float* pv, RiskTerms* terms, float* scores, int* nonfinite,
                 int stages, bool general_scale, hipStream_t stream) {
  int scale_exponent = 0;
  const bool p2 = !general_scale && scale > 0.0f && std::isfinite(scale) &&
                  std::frexp(scale, &scale_exponent) == 0.5f && scale_exponent > -60;
  if (stages & 1) {
    // about six block steps per block: each block overlaps its next step's loads with the
    // current step's arithmetic (cfg1 shape: 3 blocks per segment, one wave of resident blocks)
    constexpr int rows_per_block = 256 / (D / 8);
    const int64_t steps = ceil_div(max_length, kProjectedRowsPerLane * rows_per_block);
    dim3 pv_grid(static_cast<unsigned>(ceil_div(steps, int64_t{6})), static_cast<unsigned>(segments));
    projected_values_kernel<D><<<pv_grid, 256, 0, stream>>>(table, groups, pv, nonfinite, margin,
                                                            terms);
    if (int rc = check_launch("projected_values")) return rc;
  }
  if (stages & 2) {
    const int64_t qtiles = ceil_div(window, 32);
    const int64_t wg_per_segment = ceil_div(groups * qtiles, 4);
    if (p2)
      row_stats_kernel<D, true><<<static_cast<unsigned>(segments * wg_per_segment), 256, 0, stream>>>(
          table, groups, window, query_stride, query_positions, scale, eps, wg_per_segment, pv,
          stats);
    else
      row_stats_kernel<D, false><<<static_cast<unsigned>(segments * wg_per_segment), 256, 0, stream>>>(
          table, groups, window, query_stride, query_positions, scale, eps, wg_per_segment, pv,
          stats);
    if (int rc = check_launch("row_stats")) return rc;
  }
  if (stages & 4) {
    const int64_t tiles = ceil_div(max_candidates, 4 * 32 * column_key_tiles<D>());
    if (p2)
      column_scores_kernel<D, true><<<static_cast<unsigned>(segments * tiles), 256, 0, stream>>>(
          table, groups, window, query_stride, query_positions, margin, scale, tiles, pv, stats,
          terms, scores, nonfinite);
    else
      column_scores_kernel<D, false><<<static_cast<unsigned>(segments * tiles), 256, 0, stream>>>(
          table, groups, window, query_stride, query_positions, margin, scale, tiles, pv, stats,
          terms, scores, nonfinite);
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
         align256(static_cast<size_t>(projected_floats) * sizeof(float)) +
         align256(sizeof(RiskTerms));
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
  LR_REQUIRE(stages >= 0 && stages <= 15, "stages is a bitmask of 1 | 2 | 4 (| 8)");
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
  RiskTerms* terms = reinterpret_cast<RiskTerms*>(
      static_cast<char*>(workspace) + need - align256(sizeof(RiskTerms)));
  const hipStream_t s = as_stream(stream);
  const float eps = static_cast<float>(epsilon);
  const bool general_scale = (stages & 8) != 0;
  const int run = (stages & 7) == 0 ? 7 : (stages & 7);
  switch (dim) {
    case 64:
      return launch_score<64>(segment_table, segments, groups, window, max_length, max_candidates,
                              query_group_stride, query_positions, margin, scale, eps, stats, pv,
                              terms, scores, nonfinite, run, general_scale, s);
    case 128:
      return launch_score<128>(segment_table, segments, groups, window, max_length, max_candidates,
                               query_group_stride, query_positions, margin, scale, eps, stats, pv,
                               terms, scores, nonfinite, run, general_scale, s);
    default:
      return launch_score<256>(segment_table, segments, groups, window, max_length, max_candidates,
                               query_group_stride, query_positions, margin, scale, eps, stats, pv,
                               terms, scores, nonfinite, run, general_scale, s);
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
