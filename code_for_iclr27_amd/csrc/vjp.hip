// The audit's vector-Jacobian helpers around the scorer: fp32 output-head logits of the last
// hidden state, the one-vs-rest margin statistics, the hidden-state gradient of that margin and
// the per-layer pre-projection gradient (src/lazy_recall/_core/scoring.py:26-76,
// batch_audit.py:11-24, scoring.py:228-237).
//
// Every kernel streams one weight matrix (the vocabulary head [V, D] or o_proj [hidden, Hq*d])
// from HBM once, in its own dtype (bf16/f16/f32), and does the arithmetic in f32 as the
// reference's `.float()` GEMMs do; the reference instead materialises f32 copies of 4096-row
// weight chunks (written and re-read) and the [rows, V] probability matrix.
//   head_logits_kernel   Y[r, v] = sum_d X[r, d] * W[v, d] (+ b[v]); a wave owns 4 rows of W,
//                        lanes split D (16 B loads), X staged in LDS, one wave reduction per row.
//   margin stats         per logits row: target (given, or the first argmax), competitor max M,
//                        competitor sum S = sum_{v != t} exp(l_v - M), margin l_t - (M + log S)
//                        (three launches over 4096-logit chunks).
//   row_sum_kernel       Z_blk[r, :] = sum_{v in blk} c[r, v] * W[v, :] over a block of rows of
//                        W, with c = softmax over the competitors (exp(l - M) / S, 0 at the
//                        target) or a given coefficient vector; one thread per 8 columns of
//                        a 2048-column block, 8 rows of W in flight per thread.
//   row_sum_reduce_kernel  the blocks' partials summed in a fixed order, then
//                        out = (base - Z) * due (hidden gradient, base = W[target]) or
//                        out = Z * gate (pre-projection gradient).

#include <algorithm>

#include "lr_common.hpp"

namespace lr {
namespace {

typedef float vjp_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned vjp_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kLogitThreads = 256;
constexpr int kLogitRowsPerWave = 4;
constexpr int kLogitRowsPerBlock = kLogitRowsPerWave * (kLogitThreads / 64);
constexpr int kLogitLdsFloats = 16384;  // X rows staged per launch: rows * D <= this (64 KB)
constexpr int kReduceThreads = 1024;
constexpr int kReduceColumns = 64;

// Eight consecutive elements of a weight row as f32.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (std::is_same<T, float>::value) {
    const vjp_f32x4 a = *reinterpret_cast<const vjp_f32x4*>(p);
    const vjp_f32x4 b = *reinterpret_cast<const vjp_f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  } else if constexpr (std::is_same<T, __bf16>::value) {
    const vjp_u32x4 raw = *reinterpret_cast<const vjp_u32x4*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __builtin_bit_cast(float, raw[e] << 16);
      v[2 * e + 1] = __builtin_bit_cast(float, raw[e] & 0xffff0000u);
    }
  } else {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const h8 h = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(h[e]);
  }
}

template <typename T>
__device__ __forceinline__ float load1(const T* p) {
  return static_cast<float>(*p);
}

// grid: ceil(V / 16) blocks of 256 threads. X rows [row0, row0 + RP) of [rows, D] in LDS.
template <typename T, int RP>
__global__ __launch_bounds__(kLogitThreads) void head_logits_kernel(
    const float* __restrict__ hidden, int64_t rows_here, int64_t dim, const T* __restrict__ weight,
    const T* __restrict__ bias, int64_t vocab, float* __restrict__ out, int64_t out_stride) {
  extern __shared__ __align__(16) float x[];  // [RP, dim]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int64_t i = tid; i < RP * dim; i += kLogitThreads) {
    const int64_t r = i / dim;
    x[i] = r < rows_here ? hidden[i] : 0.f;
  }
  __syncthreads();
  const int64_t chunks = dim / 8;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * kLogitRowsPerBlock + wave * kLogitRowsPerWave;
  const T* wrow[kLogitRowsPerWave];
#pragma unroll
  for (int i = 0; i < kLogitRowsPerWave; ++i) {
    const int64_t v = v0 + i < vocab ? v0 + i : vocab - 1;  // clamped; not written
    wrow[i] = weight + v * dim;
  }
  float acc[kLogitRowsPerWave][RP];
#pragma unroll
  for (int i = 0; i < kLogitRowsPerWave; ++i)
#pragma unroll
    for (int r = 0; r < RP; ++r) acc[i][r] = 0.f;
#pragma unroll 2
  for (int64_t c = lane; c < chunks; c += 64) {
    float w[kLogitRowsPerWave][8];
#pragma unroll
    for (int i = 0; i < kLogitRowsPerWave; ++i) load8<T>(wrow[i] + 8 * c, w[i]);
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      const vjp_f32x4 lo = *reinterpret_cast<const vjp_f32x4*>(&x[r * dim + 8 * c]);
      const vjp_f32x4 hi = *reinterpret_cast<const vjp_f32x4*>(&x[r * dim + 8 * c + 4]);
      const float xv[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int i = 0; i < kLogitRowsPerWave; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i][r] = __builtin_fmaf(xv[e], w[i][e], acc[i][r]);
    }
  }
#pragma unroll
  for (int i = 0; i < kLogitRowsPerWave; ++i)
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
      for (int offset = 32; offset > 0; offset >>= 1) acc[i][r] += __shfl_xor(acc[i][r], offset);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < kLogitRowsPerWave; ++i) {
      const int64_t v = v0 + i;
      if (v >= vocab) break;
      const float b = bias ? load1(bias + v) : 0.f;
#pragma unroll
      for (int r = 0; r < RP; ++r)
        if (r < rows_here) out[r * out_stride + v] = bias ? acc[i][r] + b : acc[i][r];
    }
  }
}

// Per-thread top-two state: the best (value, index), larger value first and ties to the lower
// index, and the largest value at any other index.
struct TopTwo {
  float v1;
  int64_t i1;
  float v2;
};

__device__ __forceinline__ void top_two_add(TopTwo& s, float v, int64_t i) {
  if (v > s.v1 || (v == s.v1 && i < s.i1)) {
    s.v2 = fmaxf(s.v2, s.v1);
    s.v1 = v;
    s.i1 = i;
  } else {
    s.v2 = fmaxf(s.v2, v);
  }
}

__device__ __forceinline__ void top_two_merge(TopTwo& s, const TopTwo& o) {
  if (o.v1 > s.v1 || (o.v1 == s.v1 && o.i1 < s.i1)) {
    s.v2 = fmaxf(fmaxf(s.v2, s.v1), o.v2);
    s.v1 = o.v1;
    s.i1 = o.i1;
  } else {
    s.v2 = fmaxf(fmaxf(s.v2, o.v1), o.v2);
  }
}

// Margin statistics in three short launches over chunks of kStatChunk logits (a single block
// per row is latency-bound at vocab 128K):
//   chunk_top_kernel    per (row, chunk): the top-two state (argmax mode) or, with a given
//                       target, that target's logit and the max of the chunk's other logits;
//   chunk_sum_kernel    per (row, chunk): every block merges the row's chunk states in chunk
//                       order (target t, competitor max M), then sums exp(l - M) over the
//                       chunk's logits other than t;
//   margin_finish_kernel  per row: the same merge, the chunk sums in chunk order, the margin.
constexpr int kStatChunk = 4096;
constexpr int kStatBlock = 256;

__device__ __forceinline__ void visit_logit(TopTwo& st, float value, int64_t i, int64_t given) {
  if (given >= 0) {
    if (i == given) {
      st.v1 = value;
      st.i1 = i;
    } else {
      st.v2 = fmaxf(st.v2, value);
    }
  } else {
    top_two_add(st, value, i);
  }
}

__device__ __forceinline__ void merge_state(TopTwo& st, const TopTwo& o, int64_t given) {
  if (given >= 0) {
    if (o.i1 == given) {
      st.v1 = o.v1;
      st.i1 = o.i1;
    }
    st.v2 = fmaxf(st.v2, o.v2);
  } else {
    top_two_merge(st, o);
  }
}

// Block-wide merge of per-thread states; the result is returned to every thread.
__device__ TopTwo block_merge(TopTwo st, int64_t given, TopTwo* scratch) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int offset = 32; offset > 0; offset >>= 1) {
    const TopTwo o{__shfl_xor(st.v1, offset), __shfl_xor(st.i1, offset), __shfl_xor(st.v2, offset)};
    merge_state(st, o, given);
  }
  __syncthreads();
  if (lane == 0) scratch[wave] = st;
  __syncthreads();
  TopTwo total = scratch[0];
  for (int w = 1; w < kStatBlock / 64; ++w) merge_state(total, scratch[w], given);
  return total;
}

__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = scratch[0];
  for (int w = 1; w < kStatBlock / 64; ++w) total += scratch[w];
  return total;
}

// The row's chunk states merged in chunk order (threads take chunks tid, tid + 256, ...).
__device__ TopTwo merge_chunks(const TopTwo* states, int64_t chunks, int64_t vocab, int64_t given,
                               TopTwo* scratch) {
  constexpr float kNegInf = -__builtin_huge_valf();
  TopTwo st{kNegInf, vocab, kNegInf};
  for (int64_t c = threadIdx.x; c < chunks; c += kStatBlock) merge_state(st, states[c], given);
  TopTwo total = block_merge(st, given, scratch);
  if (given >= 0) total.i1 = given;
  return total;
}

__global__ __launch_bounds__(kStatBlock) void chunk_top_kernel(
    const float* __restrict__ logits, int64_t vocab, const int64_t* __restrict__ targets,
    TopTwo* __restrict__ states, int64_t chunks) {
  __shared__ TopTwo scratch[kStatBlock / 64];
  constexpr float kNegInf = -__builtin_huge_valf();
  const int64_t r = blockIdx.y, c = blockIdx.x;
  const int64_t given = targets ? targets[r] : -1;
  const float* row = logits + r * vocab;
  const int64_t begin = c * kStatChunk, end = begin + kStatChunk < vocab ? begin + kStatChunk : vocab;
  TopTwo st{kNegInf, vocab, kNegInf};
  constexpr int kPer = kStatChunk / kStatBlock;
  if (end - begin == kStatChunk) {  // whole chunk: every load issued before use
    float v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) v[u] = row[begin + threadIdx.x + u * kStatBlock];
#pragma unroll
    for (int u = 0; u < kPer; ++u) visit_logit(st, v[u], begin + threadIdx.x + u * kStatBlock, given);
  } else {
    for (int64_t i = begin + threadIdx.x; i < end; i += kStatBlock) visit_logit(st, row[i], i, given);
  }
  const TopTwo total = block_merge(st, given, scratch);
  if (threadIdx.x == 0) states[r * chunks + c] = total;
}

__global__ __launch_bounds__(kStatBlock) void chunk_sum_kernel(
    const float* __restrict__ logits, int64_t vocab, const int64_t* __restrict__ targets,
    const TopTwo* __restrict__ states, int64_t chunks, float* __restrict__ sums) {
  __shared__ TopTwo scratch[kStatBlock / 64];
  __shared__ float sum_scratch[kStatBlock / 64];
  const int64_t r = blockIdx.y, c = blockIdx.x;
  const int64_t given = targets ? targets[r] : -1;
  const TopTwo total = merge_chunks(states + r * chunks, chunks, vocab, given, scratch);
  const int64_t target = total.i1;
  const float mx = total.v2;
  const float* row = logits + r * vocab;
  const int64_t begin = c * kStatChunk, end = begin + kStatChunk < vocab ? begin + kStatChunk : vocab;
  float sum = 0.f;
  constexpr int kPer = kStatChunk / kStatBlock;
  if (end - begin == kStatChunk) {
    float v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) v[u] = row[begin + threadIdx.x + u * kStatBlock];
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      sum += begin + threadIdx.x + u * kStatBlock == target ? 0.f : expf(v[u] - mx);
  } else {
    for (int64_t i = begin + threadIdx.x; i < end; i += kStatBlock)
      if (i != target) sum += expf(row[i] - mx);
  }
  sum = block_sum(sum, sum_scratch);
  if (threadIdx.x == 0) sums[r * chunks + c] = sum;
}

__global__ __launch_bounds__(kStatBlock) void margin_finish_kernel(
    int64_t vocab, const int64_t* __restrict__ targets, const TopTwo* __restrict__ states,
    const float* __restrict__ sums, int64_t chunks, int64_t* __restrict__ targets_out,
    float* __restrict__ margins, float* __restrict__ stats) {
  __shared__ TopTwo scratch[kStatBlock / 64];
  const int64_t r = blockIdx.x;
  const int64_t given = targets ? targets[r] : -1;
  const TopTwo total = merge_chunks(states + r * chunks, chunks, vocab, given, scratch);
  if (threadIdx.x != 0) return;
  float sum = 0.f;
  for (int64_t c = 0; c < chunks; ++c) sum += sums[r * chunks + c];
  const int64_t target = total.i1;
  const bool valid = target >= 0 && target < vocab;
  margins[r] = valid ? total.v1 - (total.v2 + logf(sum)) : __builtin_nanf("");
  stats[2 * r] = total.v2;
  stats[2 * r + 1] = sum;
  if (targets_out) targets_out[r] = target;
}

struct RowSumArgs {
  const void* weight;         // [vocab, dim]
  int64_t vocab, dim;
  int64_t rows;               // coefficient rows (<= RP in one launch)
  int64_t rows_per_block;     // rows of W per block (multiple of 4)
  // Coefficients: softmax form (logits [rows, vocab], stats [rows, 2], targets [rows]) when
  // logits is set, else the given coefficients [rows, vocab].
  const float* logits;
  const float* stats;
  const int64_t* targets;
  const float* coefficients;
  float* partial;             // [blocks, rows, dim] (per layer with a layer table)
  // Several weights in one launch (blockIdx.z = layer): device [layers, 4] words (weight,
  // coefficients, gate or 0, out); weight and coefficients above are then unused.
  const int64_t* layer_table;
};

// grid: (ceil(dim / 2048) column blocks, ceil(vocab / rows_per_block) row blocks) of 256
// threads; thread t owns columns 8t .. 8t + 7 of its column block. kRowUnroll rows of W are
// loaded before they are used.
constexpr int kRowSumThreads = 256;
constexpr int kRowSumColumns = 8 * kRowSumThreads;
constexpr int kRowUnroll = 8;

template <typename T, int RP>
__global__ __launch_bounds__(kRowSumThreads) void row_sum_kernel(RowSumArgs a) {
  extern __shared__ float coef[];  // [rows_per_block][RP]
  const int tid = threadIdx.x;
  const void* weight_ptr = a.weight;
  const float* coefficients = a.coefficients;
  float* partial = a.partial;
  if (a.layer_table) {
    const int64_t* entry = a.layer_table + 4 * static_cast<int64_t>(blockIdx.z);
    weight_ptr = reinterpret_cast<const void*>(entry[0]);
    coefficients = reinterpret_cast<const float*>(entry[1]);
    partial += static_cast<int64_t>(blockIdx.z) * gridDim.y * a.rows * a.dim;
  }
  const int64_t v0 = static_cast<int64_t>(blockIdx.y) * a.rows_per_block;
  const int64_t count = a.vocab - v0 < a.rows_per_block ? a.vocab - v0 : a.rows_per_block;
  for (int64_t i = tid; i < a.rows_per_block * RP; i += kRowSumThreads) {
    const int64_t k = i / RP, r = i - k * RP;
    float c = 0.f;
    if (k < count && r < a.rows) {
      const int64_t v = v0 + k;
      if (a.logits) {
        c = v == a.targets[r] ? 0.f
                              : expf(a.logits[r * a.vocab + v] - a.stats[2 * r]) / a.stats[2 * r + 1];
      } else {
        c = coefficients[r * a.vocab + v];
      }
    }
    coef[i] = c;
  }
  __syncthreads();
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kRowSumColumns + 8 * tid;
  if (col >= a.dim) return;  // no barrier follows
  const T* weight = static_cast<const T*>(weight_ptr);
  float acc[RP][8];
#pragma unroll
  for (int r = 0; r < RP; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  // Whole groups of kRowUnroll rows with no per-row branch (a load under a branch is waited
  // for inside it), then the remaining rows one by one.
  int64_t k = 0;
  for (; k + kRowUnroll <= count; k += kRowUnroll) {
    float w[kRowUnroll][8];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) load8<T>(weight + (v0 + k + u) * a.dim + col, w[u]);
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u)
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const float c = coef[(k + u) * RP + r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(c, w[u][e], acc[r][e]);
      }
  }
  for (; k < count; ++k) {
    float w[8];
    load8<T>(weight + (v0 + k) * a.dim + col, w);
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      const float c = coef[k * RP + r];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(c, w[e], acc[r][e]);
    }
  }
  for (int r = 0; r < RP && r < a.rows; ++r) {
    float* p = partial + (static_cast<int64_t>(blockIdx.y) * a.rows + r) * a.dim + col;
    *reinterpret_cast<vjp_f32x4*>(p) = vjp_f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
    *reinterpret_cast<vjp_f32x4*>(p + 4) = vjp_f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
  }
}

// grid: (ceil(dim / 64), rows). Thread (group g, column c) sums blocks g, g + 16, ... of column
// c, then the 16 group sums are added in group order.
template <typename T>
__global__ __launch_bounds__(kReduceThreads) void row_sum_reduce_kernel(
    const float* __restrict__ partial, int64_t blocks, int64_t rows, int64_t dim,
    const T* __restrict__ weight, int64_t vocab, const int64_t* __restrict__ targets,
    const float* __restrict__ due, const float* __restrict__ gate, float* __restrict__ out,
    const int64_t* __restrict__ layer_table) {
  constexpr int kGroups = kReduceThreads / kReduceColumns;
  __shared__ float sums[kGroups][kReduceColumns];
  const int tid = threadIdx.x, g = tid / kReduceColumns, c = tid - g * kReduceColumns;
  if (layer_table) {  // blockIdx.z = layer: its partials, gate and output
    const int64_t* entry = layer_table + 4 * static_cast<int64_t>(blockIdx.z);
    partial += static_cast<int64_t>(blockIdx.z) * blocks * rows * dim;
    gate = reinterpret_cast<const float*>(entry[2]);
    out = reinterpret_cast<float*>(entry[3]);
  }
  const int64_t r = blockIdx.y;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kReduceColumns + c;
  float s = 0.f;
  if (d < dim) {
    constexpr int kUnroll = 4;
    for (int64_t b = g; b < blocks; b += kGroups * kUnroll) {
      float v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t bb = b + u * kGroups;
        v[u] = bb < blocks ? partial[(bb * rows + r) * dim + d] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) s += v[u];
    }
  }
  sums[g][c] = s;
  __syncthreads();
  if (g != 0 || d >= dim) return;
  for (int k = 1; k < kGroups; ++k) s += sums[k][c];
  float result;
  if (targets) {  // hidden gradient: W[target] - sum, times the row's due flag
    const int64_t t = targets[r];
    result = (t >= 0 && t < vocab) ? load1(weight + t * dim + d) - s : __builtin_nanf("");
    if (due) result *= due[r];
  } else {        // pre-projection gradient: sum, times the output gate
    result = gate ? s * gate[d] : s;
  }
  out[r * dim + d] = result;
}

template <typename F>
int dispatch_weight(int dtype, F&& f) {
  switch (dtype) {
    case LR_DTYPE_BF16: return f.template operator()<__bf16>();
    case LR_DTYPE_F16: return f.template operator()<_Float16>();
    default: return f.template operator()<float>();
  }
}

int row_pass(int64_t rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }

// Rows of W per block: enough blocks to fill the chip (about 1024), but at least 32 rows per
// coefficient row so that the f32 partials stay a few percent of the weight bytes.
int64_t rows_per_block(int64_t vocab, int64_t dim, int64_t rows_pass) {
  const int64_t column_blocks = ceil_div(dim, kRowSumColumns);
  const int64_t row_blocks = std::max<int64_t>(1, 1024 / column_blocks);
  const int64_t per = std::max<int64_t>(32 * rows_pass, ceil_div(vocab, row_blocks));
  return ceil_div(std::min<int64_t>(per, std::max<int64_t>(vocab, 1)), 4) * 4;
}

int check_weight(int dtype, int64_t vocab, int64_t dim, const void* weight) {
  LR_REQUIRE(dtype == LR_DTYPE_BF16 || dtype == LR_DTYPE_F16 || dtype == LR_DTYPE_F32,
             "Weights must be float32, float16 or bfloat16");
  LR_REQUIRE(vocab > 0 && dim > 0 && dim % 8 == 0 && dim <= 8192,
             "Weight rows must be a multiple of 8 elements, at most 8192");
  LR_REQUIRE(weight != nullptr && reinterpret_cast<uintptr_t>(weight) % 16 == 0,
             "Weights must be 16-byte aligned");
  return LR_OK;
}

// Weighted row sums of W in passes of at most 8 coefficient rows, then the reduction.
int weighted_rows(const void* weight, int dtype, int64_t vocab, int64_t dim, int64_t rows,
                  const float* logits, const float* stats, const int64_t* targets,
                  const float* coefficients, const float* due, const float* gate, float* out,
                  void* workspace, size_t workspace_size, hipStream_t stream);

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_head_logits(const float* hidden, int64_t rows, const void* weight,
                              const void* bias, int64_t vocab, int64_t dim, int dtype, float* out,
                              void* stream) {
  clear_error();
  if (int status = check_weight(dtype, vocab, dim, weight)) return status;
  LR_REQUIRE(rows > 0 && hidden && out, "Invalid hidden states");
  const hipStream_t s = as_stream(stream);
  const int64_t per_pass = std::min<int64_t>(8, kLogitLdsFloats / dim);
  const int64_t blocks = ceil_div(vocab, kLogitRowsPerBlock);
  for (int64_t r0 = 0; r0 < rows; r0 += per_pass) {
    const int64_t here = std::min<int64_t>(per_pass, rows - r0);
    const int rp = row_pass(here);
    const int status = dispatch_weight(dtype, [&]<typename T>() {
      const T* w = static_cast<const T*>(weight);
      const T* b = static_cast<const T*>(bias);
      auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kLogitThreads),
                           static_cast<size_t>(rp) * dim * sizeof(float), s, hidden + r0 * dim,
                           here, dim, w, b, vocab, out + r0 * vocab, vocab);
        return check_launch("head_logits");
      };
      switch (rp) {
        case 1: return launch(head_logits_kernel<T, 1>);
        case 2: return launch(head_logits_kernel<T, 2>);
        case 4: return launch(head_logits_kernel<T, 4>);
        default: return launch(head_logits_kernel<T, 8>);
      }
    });
    if (status) return status;
  }
  return LR_OK;
}

extern "C" size_t lr_margin_stats_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  const int64_t chunks = ceil_div(vocab, kStatChunk);
  return static_cast<size_t>(rows * chunks) * (sizeof(TopTwo) + sizeof(float));
}

extern "C" int lr_margin_stats(const float* logits, int64_t rows, int64_t vocab,
                               const int64_t* targets, int64_t* targets_out, float* margins,
                               float* stats, void* workspace, size_t workspace_size,
                               void* stream) {
  clear_error();
  LR_REQUIRE(rows > 0 && vocab > 1 && logits && margins && stats, "Invalid logits");
  LR_REQUIRE(rows < 65536, "Too many logits rows");
  LR_REQUIRE(workspace && workspace_size >= lr_margin_stats_workspace_bytes(rows, vocab) &&
                 reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
             "Margin workspace too small");
  const int64_t chunks = ceil_div(vocab, kStatChunk);
  TopTwo* states = static_cast<TopTwo*>(workspace);
  float* sums = reinterpret_cast<float*>(states + rows * chunks);
  const hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
  hipLaunchKernelGGL(chunk_top_kernel, grid, dim3(kStatBlock), 0, s, logits, vocab, targets,
                     states, chunks);
  if (int status = check_launch("margin_stats")) return status;
  hipLaunchKernelGGL(chunk_sum_kernel, grid, dim3(kStatBlock), 0, s, logits, vocab, targets,
                     states, chunks, sums);
  if (int status = check_launch("margin_stats")) return status;
  hipLaunchKernelGGL(margin_finish_kernel, dim3(static_cast<unsigned>(rows)), dim3(kStatBlock), 0,
                     s, vocab, targets, states, sums, chunks, targets_out, margins, stats);
  return check_launch("margin_stats");
}

extern "C" size_t lr_row_sum_workspace_bytes(int64_t rows, int64_t vocab, int64_t dim) {
  if (rows <= 0 || vocab <= 0 || dim <= 0) return 0;
  const int64_t pass = std::min<int64_t>(rows, 8);
  const int64_t blocks = ceil_div(vocab, rows_per_block(vocab, dim, row_pass(pass)));
  return static_cast<size_t>(blocks) * static_cast<size_t>(pass) * static_cast<size_t>(dim) *
         sizeof(float);
}

namespace lr {
namespace {

int weighted_rows(const void* weight, int dtype, int64_t vocab, int64_t dim, int64_t rows,
                  const float* logits, const float* stats, const int64_t* targets,
                  const float* coefficients, const float* due, const float* gate, float* out,
                  void* workspace, size_t workspace_size, hipStream_t stream) {
  LR_REQUIRE(workspace && workspace_size >= lr_row_sum_workspace_bytes(rows, vocab, dim),
             "Row-sum workspace too small");
  LR_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "Workspace must be 16-byte aligned");
  for (int64_t r0 = 0; r0 < rows; r0 += 8) {
    const int64_t here = std::min<int64_t>(8, rows - r0);
    const int rp = row_pass(here);
    const int64_t per_block = rows_per_block(vocab, dim, rp);
    const int64_t blocks = ceil_div(vocab, per_block);
    RowSumArgs args{};
    args.weight = weight;
    args.vocab = vocab;
    args.dim = dim;
    args.rows = here;
    args.rows_per_block = per_block;
    args.logits = logits ? logits + r0 * vocab : nullptr;
    args.stats = stats ? stats + 2 * r0 : nullptr;
    args.targets = targets ? targets + r0 : nullptr;
    args.coefficients = coefficients ? coefficients + r0 * vocab : nullptr;
    args.partial = static_cast<float*>(workspace);
    const size_t lds = static_cast<size_t>(per_block) * rp * sizeof(float);
    const dim3 grid(static_cast<unsigned>(ceil_div(dim, kRowSumColumns)),
                    static_cast<unsigned>(blocks));
    int status = dispatch_weight(dtype, [&]<typename T>() {
      auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kRowSumThreads), lds, stream, args);
        return check_launch("row_sum");
      };
      switch (rp) {
        case 1: return launch(row_sum_kernel<T, 1>);
        case 2: return launch(row_sum_kernel<T, 2>);
        case 4: return launch(row_sum_kernel<T, 4>);
        default: return launch(row_sum_kernel<T, 8>);
      }
    });
    if (status) return status;
    status = dispatch_weight(dtype, [&]<typename T>() {
      hipLaunchKernelGGL(row_sum_reduce_kernel<T>,
                         dim3(static_cast<unsigned>(ceil_div(dim, kReduceColumns)),
                              static_cast<unsigned>(here)),
                         dim3(kReduceThreads), 0, stream, static_cast<const float*>(workspace),
                         blocks, here, dim, static_cast<const T*>(weight), vocab,
                         targets ? targets + r0 : nullptr, due ? due + r0 : nullptr, gate,
                         out + r0 * dim, nullptr);
      return check_launch("row_sum_reduce");
    });
    if (status) return status;
  }
  return LR_OK;
}

}  // namespace
}  // namespace lr

extern "C" int lr_hidden_gradient(const float* logits, const float* stats, const int64_t* targets,
                                  int64_t rows, const void* weight, int64_t vocab, int64_t dim,
                                  int dtype, const float* due, float* out, void* workspace,
                                  size_t workspace_size, void* stream) {
  clear_error();
  if (int status = check_weight(dtype, vocab, dim, weight)) return status;
  LR_REQUIRE(rows > 0 && logits && stats && targets && out, "Invalid gradient inputs");
  return weighted_rows(weight, dtype, vocab, dim, rows, logits, stats, targets, nullptr, due,
                       nullptr, out, workspace, workspace_size, as_stream(stream));
}

extern "C" int lr_pre_gradient(const float* post_gradient, const void* o_weight, int64_t hidden,
                               int64_t width, int dtype, const float* gate, float* out,
                               void* workspace, size_t workspace_size, void* stream) {
  clear_error();
  if (int status = check_weight(dtype, hidden, width, o_weight)) return status;
  LR_REQUIRE(post_gradient && out, "Invalid gradient inputs");
  return weighted_rows(o_weight, dtype, hidden, width, 1, nullptr, nullptr, nullptr, post_gradient,
                       nullptr, gate, out, workspace, workspace_size, as_stream(stream));
}

extern "C" size_t lr_pre_gradient_layers_workspace_bytes(int64_t layers, int64_t hidden,
                                                         int64_t width) {
  if (layers <= 0) return 0;
  return static_cast<size_t>(layers) * lr_row_sum_workspace_bytes(1, hidden, width);
}

extern "C" int lr_pre_gradient_layers(const int64_t* layer_table, int64_t layers, int64_t hidden,
                                      int64_t width, int dtype, void* workspace,
                                      size_t workspace_size, void* stream) {
  clear_error();
  LR_REQUIRE(dtype == LR_DTYPE_BF16 || dtype == LR_DTYPE_F16 || dtype == LR_DTYPE_F32,
             "Weights must be float32, float16 or bfloat16");
  // The same row bounds as check_weight on the per-layer path; the weights' 16-byte alignment
  // cannot be checked here (their addresses are in device memory) and is the caller's to keep.
  LR_REQUIRE(hidden > 0 && width > 0 && width % 8 == 0 && width <= 8192,
             "Weight rows must be a multiple of 8 elements, at most 8192");
  LR_REQUIRE(layer_table && layers > 0 && layers < 65536, "Invalid layer table");
  LR_REQUIRE(workspace && workspace_size >= lr_pre_gradient_layers_workspace_bytes(layers, hidden, width) &&
                 reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
             "Row-sum workspace too small");
  const int64_t per_block = rows_per_block(hidden, width, 1);
  const int64_t blocks = ceil_div(hidden, per_block);
  RowSumArgs args{};
  args.vocab = hidden;
  args.dim = width;
  args.rows = 1;
  args.rows_per_block = per_block;
  args.partial = static_cast<float*>(workspace);
  args.layer_table = layer_table;
  const hipStream_t s = as_stream(stream);
  const size_t lds = static_cast<size_t>(per_block) * sizeof(float);
  int status = dispatch_weight(dtype, [&]<typename T>() {
    hipLaunchKernelGGL((row_sum_kernel<T, 1>),
                       dim3(static_cast<unsigned>(ceil_div(width, kRowSumColumns)),
                            static_cast<unsigned>(blocks), static_cast<unsigned>(layers)),
                       dim3(kRowSumThreads), lds, s, args);
    return check_launch("row_sum");
  });
  if (status) return status;
  return dispatch_weight(dtype, [&]<typename T>() {
    hipLaunchKernelGGL(row_sum_reduce_kernel<T>,
                       dim3(static_cast<unsigned>(ceil_div(width, kReduceColumns)), 1u,
                            static_cast<unsigned>(layers)),
                       dim3(kReduceThreads), 0, s, static_cast<const float*>(workspace), blocks,
                       int64_t{1}, width, static_cast<const T*>(nullptr), hidden, nullptr,
                       nullptr, nullptr, nullptr, layer_table);
    return check_launch("row_sum_reduce");
  });
}
