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
//   margin_stats_kernel  per logits row: target (given, or the first argmax), competitor max M,
//                        competitor sum S = sum_{v != t} exp(l_v - M), margin l_t - (M + log S).
//   row_sum_kernel       Z_blk[r, :] = sum_{v in blk} c[r, v] * W[v, :] over a block of rows of
//                        W, with c = softmax over the competitors (exp(l - M) / S, 0 at the
//                        target) or a given coefficient vector; one thread per 8 columns.
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
constexpr int kStatThreads = 1024;
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

// (value, index) pairs reduced across the block: larger value wins, ties to the lower index.
__device__ __forceinline__ void better(float& value, int64_t& index, float v2, int64_t i2) {
  if (v2 > value || (v2 == value && i2 < index)) {
    value = v2;
    index = i2;
  }
}

// grid: one block per logits row.
__global__ __launch_bounds__(kStatThreads) void margin_stats_kernel(
    const float* __restrict__ logits, int64_t vocab, const int64_t* __restrict__ targets_in,
    int64_t* __restrict__ targets_out, float* __restrict__ margins, float* __restrict__ stats) {
  __shared__ float red_v[kStatThreads / 64];
  __shared__ int64_t red_i[kStatThreads / 64];
  __shared__ int64_t target_s;
  __shared__ float max_s;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t r = blockIdx.x;
  const float* row = logits + r * vocab;
  int64_t target;
  if (targets_in) {
    target = targets_in[r];
  } else {  // torch.argmax: the first index of the largest value
    float best = -__builtin_huge_valf();
    int64_t at = vocab;
    for (int64_t v = tid; v < vocab; v += kStatThreads) better(best, at, row[v], v);
    for (int offset = 32; offset > 0; offset >>= 1)
      better(best, at, __shfl_xor(best, offset), __shfl_xor(at, offset));
    if (lane == 0) {
      red_v[wave] = best;
      red_i[wave] = at;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kStatThreads / 64; ++w) better(best, at, red_v[w], red_i[w]);
      target_s = at < vocab ? at : 0;
    }
    __syncthreads();
    target = target_s;
  }
  // Competitor max, then the competitor exp-sum against it.
  float mx = -__builtin_huge_valf();
  for (int64_t v = tid; v < vocab; v += kStatThreads)
    if (v != target) mx = fmaxf(mx, row[v]);
  for (int offset = 32; offset > 0; offset >>= 1) mx = fmaxf(mx, __shfl_xor(mx, offset));
  __syncthreads();
  if (lane == 0) red_v[wave] = mx;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kStatThreads / 64; ++w) mx = fmaxf(mx, red_v[w]);
    max_s = mx;
  }
  __syncthreads();
  mx = max_s;
  float sum = 0.f;
  for (int64_t v = tid; v < vocab; v += kStatThreads)
    if (v != target) sum += expf(row[v] - mx);
  for (int offset = 32; offset > 0; offset >>= 1) sum += __shfl_xor(sum, offset);
  __syncthreads();
  if (lane == 0) red_v[wave] = sum;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kStatThreads / 64; ++w) sum += red_v[w];
    const bool valid = target >= 0 && target < vocab;
    margins[r] = valid ? row[target] - (mx + logf(sum)) : __builtin_nanf("");
    stats[2 * r] = mx;
    stats[2 * r + 1] = sum;
    if (targets_out) targets_out[r] = target;
  }
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
  float* partial;             // [blocks, rows, dim]
};

// grid: ceil(vocab / rows_per_block) blocks of dim / 8 threads (<= 1024).
template <typename T, int RP>
__global__ __launch_bounds__(1024) void row_sum_kernel(RowSumArgs a) {
  extern __shared__ float coef[];  // [rows_per_block][RP]
  const int tid = threadIdx.x;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * a.rows_per_block;
  const int64_t count = a.vocab - v0 < a.rows_per_block ? a.vocab - v0 : a.rows_per_block;
  for (int64_t i = tid; i < a.rows_per_block * RP; i += blockDim.x) {
    const int64_t k = i / RP, r = i - k * RP;
    float c = 0.f;
    if (k < count && r < a.rows) {
      const int64_t v = v0 + k;
      if (a.logits) {
        c = v == a.targets[r] ? 0.f
                              : expf(a.logits[r * a.vocab + v] - a.stats[2 * r]) / a.stats[2 * r + 1];
      } else {
        c = a.coefficients[r * a.vocab + v];
      }
    }
    coef[i] = c;
  }
  __syncthreads();
  const T* weight = static_cast<const T*>(a.weight);
  const int64_t col = 8 * static_cast<int64_t>(tid);
  float acc[RP][8];
#pragma unroll
  for (int r = 0; r < RP; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  constexpr int kUnroll = 4;
  for (int64_t k = 0; k < count; k += kUnroll) {
    float w[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t v = v0 + (k + u < count ? k + u : count - 1);  // clamped; coefficient 0
      load8<T>(weight + v * a.dim + col, w[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (k + u >= count) break;
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const float c = coef[(k + u) * RP + r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(c, w[u][e], acc[r][e]);
      }
    }
  }
  for (int r = 0; r < RP && r < a.rows; ++r) {
    float* p = a.partial + (static_cast<int64_t>(blockIdx.x) * a.rows + r) * a.dim + col;
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
    const float* __restrict__ due, const float* __restrict__ gate, float* __restrict__ out) {
  constexpr int kGroups = kReduceThreads / kReduceColumns;
  __shared__ float sums[kGroups][kReduceColumns];
  const int tid = threadIdx.x, g = tid / kReduceColumns, c = tid - g * kReduceColumns;
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

int64_t rows_per_block(int64_t vocab) {
  const int64_t per = std::min<int64_t>(256, std::max<int64_t>(8, ceil_div(vocab, 512)));
  return ceil_div(per, 4) * 4;
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

extern "C" int lr_margin_stats(const float* logits, int64_t rows, int64_t vocab,
                               const int64_t* targets, int64_t* targets_out, float* margins,
                               float* stats, void* stream) {
  clear_error();
  LR_REQUIRE(rows > 0 && vocab > 1 && logits && margins && stats, "Invalid logits");
  hipLaunchKernelGGL(margin_stats_kernel, dim3(static_cast<unsigned>(rows)), dim3(kStatThreads), 0,
                     as_stream(stream), logits, vocab, targets, targets_out, margins, stats);
  return check_launch("margin_stats");
}

extern "C" size_t lr_row_sum_workspace_bytes(int64_t rows, int64_t vocab, int64_t dim) {
  if (rows <= 0 || vocab <= 0 || dim <= 0) return 0;
  const int64_t blocks = ceil_div(vocab, rows_per_block(vocab));
  return static_cast<size_t>(blocks) * static_cast<size_t>(std::min<int64_t>(rows, 8)) *
         static_cast<size_t>(dim) * sizeof(float);
}

namespace lr {
namespace {

int weighted_rows(const void* weight, int dtype, int64_t vocab, int64_t dim, int64_t rows,
                  const float* logits, const float* stats, const int64_t* targets,
                  const float* coefficients, const float* due, const float* gate, float* out,
                  void* workspace, size_t workspace_size, hipStream_t stream) {
  const int64_t per_block = rows_per_block(vocab);
  const int64_t blocks = ceil_div(vocab, per_block);
  LR_REQUIRE(workspace && workspace_size >= lr_row_sum_workspace_bytes(rows, vocab, dim),
             "Row-sum workspace too small");
  LR_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "Workspace must be 16-byte aligned");
  for (int64_t r0 = 0; r0 < rows; r0 += 8) {
    const int64_t here = std::min<int64_t>(8, rows - r0);
    const int rp = row_pass(here);
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
    const unsigned threads = static_cast<unsigned>(dim / 8);
    int status = dispatch_weight(dtype, [&]<typename T>() {
      auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), lds, stream,
                           args);
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
                         out + r0 * dim);
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
