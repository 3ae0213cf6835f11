// Op-level temporal scoring kernels with the reference's per-op contracts:
//   temporal_probabilities  csrc/scoring.cu:32-66   (masked, scaled, dtype-rounded softmax)
//   temporal_risk           csrc/scoring.cu:68-128  (min/max margin drop -> Bernoulli risk)
//   pool                    csrc/scoring.cu:190-203 (segmented sliding max)
//   decision_risk_scores    csrc/cache_legacy.cu:63-135 (legacy single-query scorer)
// Arithmetic follows the reference operation by operation (the library is built with
// -ffp-contract=off so no multiply-add is fused); reductions are wave64-native (butterfly
// within a wave, LDS across waves), so sums may differ from the reference's 256-lane tree in
// the last bits.

#include <cmath>

#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kRowThreads = 256;
constexpr int kWaves = kRowThreads / 64;

template <bool kMax>
__device__ __forceinline__ float wave_reduce(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    const float o = __shfl_xor(v, offset, 64);
    v = kMax ? fmaxf(v, o) : v + o;
  }
  return v;
}

// Block-wide reduction for 256 threads; every thread receives the result.
template <bool kMax>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
  v = wave_reduce<kMax>(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = kMax ? fmaxf(r, scratch[w]) : r + scratch[w];
  __syncthreads();
  return r;
}

template <typename T>
__device__ __forceinline__ float round_to(float x);
template <>
__device__ __forceinline__ float round_to<float>(float x) { return x; }
template <>
__device__ __forceinline__ float round_to<_Float16>(float x) { return static_cast<float>(static_cast<_Float16>(x)); }
template <>
__device__ __forceinline__ float round_to<__bf16>(float x) {
  return static_cast<float>(static_cast<__bf16>(x));
}

template <typename T>
__device__ __forceinline__ float load_as_float(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_as_float<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_as_float<double>(const double* p, int64_t i) {
  return static_cast<float>(p[i]);
}
template <>
__device__ __forceinline__ float load_as_float<_Float16>(const _Float16* p, int64_t i) {
  return static_cast<float>(p[i]);
}
template <>
__device__ __forceinline__ float load_as_float<__bf16>(const __bf16* p, int64_t i) {
  return static_cast<float>(p[i]);
}

// One 256-thread block per (query, group) row. Thread t owns positions t, t+256, ...; when a
// row fits in kCache per-thread registers the masked logits stay in registers across the
// three phases (max, exp-sum, normalise+project), otherwise they are re-derived from the
// logits (never from the output buffer).
template <typename T, int kCache>
__global__ __launch_bounds__(kRowThreads) void probabilities_kernel(
    const T* __restrict__ logits, const float* __restrict__ projected,
    const int64_t* __restrict__ query_positions, const float* __restrict__ key_positions,
    float* __restrict__ probabilities, float* __restrict__ output_projection, int64_t groups,
    int64_t length, float scale) {
  __shared__ float scratch[kWaves];
  const int64_t row = blockIdx.x;
  const int64_t group = row % groups;
  const int64_t query = row / groups;
  const float query_position = static_cast<float>(query_positions[query]);
  const T* in = logits + row * length;
  float* out = probabilities + row * length;
  const float* pv = projected + group * length;
  // Reference compares float key positions against the int64 query position promoted
  // to float (csrc/scoring.cu:46).
  auto masked = [&](int64_t t) -> float {
    const float rounded = round_to<T>(load_as_float<T>(in, t) * scale);
    return key_positions[t] <= query_position ? rounded : -INFINITY;
  };
  float cache[kCache > 0 ? kCache : 1];
  float maximum = -INFINITY;
  int i = 0;
  for (int64_t t = threadIdx.x; t < length; t += kRowThreads, ++i) {
    const float v = masked(t);
    if (kCache > 0) cache[i] = v;
    maximum = fmaxf(maximum, v);
  }
  maximum = block_reduce<true>(maximum, scratch);
  float denominator = 0.0f;
  i = 0;
  for (int64_t t = threadIdx.x; t < length; t += kRowThreads, ++i) {
    const float v = kCache > 0 ? cache[i] : masked(t);
    const float w = expf(v - maximum);
    if (kCache > 0) cache[i] = w;
    denominator += w;
  }
  denominator = block_reduce<false>(denominator, scratch);
  float projection = 0.0f;
  i = 0;
  for (int64_t t = threadIdx.x; t < length; t += kRowThreads, ++i) {
    const float w = kCache > 0 ? cache[i] : expf(masked(t) - maximum);
    const float p = w / denominator;
    out[t] = p;
    projection += p * pv[t];
  }
  projection = block_reduce<false>(projection, scratch);
  if (threadIdx.x == 0) output_projection[row] = projection;
}

__device__ __forceinline__ double softplus64(double v) { return v > 20.0 ? v : log1p(exp(v)); }

__device__ __forceinline__ double risk64(double margin, double probability, double base_softplus,
                                         float drop) {
  const double compared = margin - static_cast<double>(drop);
  return fmax(0.0, probability * (margin - compared) - base_softplus + softplus64(compared));
}

// 64 candidate lanes x 4 query lanes per block. Query lane q visits queries q, q+4, ...; the
// margin drop of one (query, candidate) sums the groups in order g = 0..G-1 exactly like the
// reference. Any non-finite drop makes the candidate's score NaN.
constexpr int kRiskCandidates = 64;
constexpr int kRiskQueryLanes = 4;

__global__ __launch_bounds__(kRiskCandidates* kRiskQueryLanes) void risk_kernel(
    const float* __restrict__ probabilities, const float* __restrict__ output_projection,
    const float* __restrict__ projected, const float* __restrict__ margin,
    float* __restrict__ result, int64_t window, int64_t groups, int64_t length, int64_t first,
    int64_t count, float epsilon) {
  __shared__ float minimums[kRiskQueryLanes][kRiskCandidates];
  __shared__ float maximums[kRiskQueryLanes][kRiskCandidates];
  __shared__ int bad[kRiskQueryLanes][kRiskCandidates];
  const int lane = threadIdx.x % kRiskCandidates;
  const int query_lane = threadIdx.x / kRiskCandidates;
  const int64_t candidate = static_cast<int64_t>(blockIdx.x) * kRiskCandidates + lane;
  const int64_t position = first + candidate;
  float minimum = INFINITY, maximum = -INFINITY;
  int nonfinite = 0;
  if (candidate < count) {
    for (int64_t query = query_lane; query < window; query += kRiskQueryLanes) {
      float drop = 0.0f;
      for (int64_t group = 0; group < groups; ++group) {
        const int64_t row = query * groups + group;
        const float p = probabilities[row * length + position];
        const float ratio = p / fmaxf(1.0f - p, epsilon);
        drop += ratio * (projected[group * length + position] - output_projection[row]);
      }
      if (!isfinite(drop)) {
        nonfinite = 1;
        break;
      }
      minimum = fminf(minimum, drop);
      maximum = fmaxf(maximum, drop);
    }
  }
  minimums[query_lane][lane] = minimum;
  maximums[query_lane][lane] = maximum;
  bad[query_lane][lane] = nonfinite;
  __syncthreads();
  if (query_lane == 0 && candidate < count) {
    for (int q = 1; q < kRiskQueryLanes; ++q) {
      minimum = fminf(minimum, minimums[q][lane]);
      maximum = fmaxf(maximum, maximums[q][lane]);
      nonfinite |= bad[q][lane];
    }
    if (nonfinite) {
      result[candidate] = NAN;
      return;
    }
    const double m = static_cast<double>(margin[0]);
    const double p = 1.0 / (1.0 + exp(-m));
    const double base = softplus64(m);
    result[candidate] = static_cast<float>(fmax(risk64(m, p, base, minimum), risk64(m, p, base, maximum)));
  }
}

// Sliding max of odd width inside each segment; NaN neighbours are ignored as by fmaxf and
// out-of-segment neighbours do not exist (csrc/scoring.cu:190-203). Block tile + halo in LDS.
// Workgroup (0, 0) also zeroes `clear[0, clear_words)` when given (the selection's counters, so
// that a following selection needs no launch of its own to reset them).
constexpr int kPoolThreads = 256;

__global__ __launch_bounds__(kPoolThreads) void pool_kernel(const float* __restrict__ scores,
                                                             int64_t total,
                                                             const int64_t* __restrict__ bounds,
                                                             float* __restrict__ output,
                                                             int half, int use_lds,
                                                             uint32_t* __restrict__ clear,
                                                             int clear_words) {
  extern __shared__ float tile[];
  if (clear != nullptr && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = threadIdx.x; i < clear_words; i += kPoolThreads) clear[i] = 0;
  const int64_t segment = blockIdx.y;
  int64_t begin = bounds[segment], end = bounds[segment + 1];
  if (begin < 0) begin = 0;
  if (end > total) end = total;
  const int64_t tile_start = begin + static_cast<int64_t>(blockIdx.x) * kPoolThreads;
  if (tile_start >= end) return;
  const int64_t position = tile_start + threadIdx.x;
  if (use_lds) {
    const int span = kPoolThreads + 2 * half;
    for (int i = threadIdx.x; i < span; i += kPoolThreads) {
      const int64_t p = tile_start - half + i;
      tile[i] = (p >= begin && p < end) ? scores[p] : -INFINITY;
    }
    __syncthreads();
    if (position >= end) return;
    float value = -INFINITY;
    for (int o = 0; o <= 2 * half; ++o) value = fmaxf(value, tile[threadIdx.x + o]);
    output[position] = value;
  } else {
    if (position >= end) return;
    float value = -INFINITY;
    for (int64_t o = -half; o <= half; ++o) {
      const int64_t n = position + o;
      if (n >= begin && n < end) value = fmaxf(value, scores[n]);
    }
    output[position] = value;
  }
}

__device__ __forceinline__ double stable_sigmoid(double v) {
  if (v >= 0.0) return 1.0 / (1.0 + exp(-v));
  const double e = exp(v);
  return e / (1.0 + e);
}

__device__ __forceinline__ double stable_softplus(double v) {
  if (v > 20.0) return v + log1p(exp(-v));
  return log1p(exp(v));
}

// One 256-thread block per candidate. The margin drop is a long mixed-sign sum whose
// cancellation amplifies any change of summation order, so this legacy op keeps the
// reference's order (csrc/cache_legacy.cu:98-121): thread t accumulates terms t, t+256, ...,
// then an LDS tree halves the 256 partials.
template <typename T>
__global__ __launch_bounds__(256) void decision_risk_kernel(
    float* __restrict__ scores, const float* __restrict__ probabilities,
    const T* __restrict__ values, const float* __restrict__ head_outputs,
    const float* __restrict__ gradients, int64_t groups, int64_t candidates, int64_t head_dim,
    double base_margin, float epsilon) {
  __shared__ float reduction[256];
  const int64_t candidate = blockIdx.x;
  float partial = 0.0f;
  const int64_t terms = groups * head_dim;
  for (int64_t index = threadIdx.x; index < terms; index += 256) {
    const int64_t group = index / head_dim;
    const int64_t d = index % head_dim;
    const float alpha = probabilities[group * candidates + candidate];
    const float denominator = fmaxf(1.0f - alpha, epsilon);
    const float value = load_as_float<T>(values, candidate * head_dim + d);
    const float local_delta = alpha / denominator * (value - head_outputs[group * head_dim + d]);
    partial += gradients[group * head_dim + d] * local_delta;
  }
  reduction[threadIdx.x] = partial;
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (threadIdx.x < stride) reduction[threadIdx.x] += reduction[threadIdx.x + stride];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double compared = base_margin - static_cast<double>(reduction[0]);
    const double probability = stable_sigmoid(base_margin);
    double kl = probability * (base_margin - compared) - stable_softplus(base_margin) +
                stable_softplus(compared);
    if (kl < 0.0) kl = 0.0;
    scores[candidate] = static_cast<float>(kl);
  }
}

template <typename T>
int launch_probabilities(const void* logits, const float* projected, const int64_t* qpos,
                         const float* kpos, int64_t window, int64_t groups, int64_t length,
                         float scale, float* probabilities, float* output_projection,
                         hipStream_t stream) {
  const int64_t rows = window * groups;
  const T* in = static_cast<const T*>(logits);
  if (length <= 256 * 16) {
    probabilities_kernel<T, 16><<<rows, kRowThreads, 0, stream>>>(
        in, projected, qpos, kpos, probabilities, output_projection, groups, length, scale);
  } else {
    probabilities_kernel<T, 0><<<rows, kRowThreads, 0, stream>>>(
        in, projected, qpos, kpos, probabilities, output_projection, groups, length, scale);
  }
  return check_launch("temporal_probabilities");
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_temporal_probabilities(const void* logits, int logits_dtype,
                                         const float* projected, const int64_t* query_positions,
                                         const float* key_positions, int64_t window,
                                         int64_t groups, int64_t length, float scale,
                                         float* probabilities, float* output_projection,
                                         void* stream) {
  clear_error();
  LR_REQUIRE(logits_dtype == LR_DTYPE_F32 || logits_dtype == LR_DTYPE_F16 ||
                 logits_dtype == LR_DTYPE_BF16,
             "Only FP32/FP16/BF16 scores are supported");
  LR_REQUIRE(window > 0 && groups > 0 && length > 0, "Empty attention dimensions");
  LR_REQUIRE(window * groups <= 2147483647LL, "Empty attention dimensions");
  LR_REQUIRE(logits && projected && query_positions && key_positions && probabilities &&
                 output_projection,
             "Expected contiguous CUDA tensor");
  const hipStream_t s = as_stream(stream);
  switch (logits_dtype) {
    case LR_DTYPE_F32:
      return launch_probabilities<float>(logits, projected, query_positions, key_positions, window,
                                         groups, length, scale, probabilities, output_projection, s);
    case LR_DTYPE_F16:
      return launch_probabilities<_Float16>(logits, projected, query_positions, key_positions, window,
                                          groups, length, scale, probabilities, output_projection, s);
    default:
      return launch_probabilities<__bf16>(logits, projected, query_positions, key_positions,
                                                   window, groups, length, scale, probabilities,
                                                   output_projection, s);
  }
}

extern "C" int lr_temporal_risk(const float* probabilities, const float* output_projection,
                                const float* projected, const float* margin, int64_t window,
                                int64_t groups, int64_t length, int64_t first, int64_t last,
                                double epsilon, float* result, void* stream) {
  clear_error();
  LR_REQUIRE(window > 0 && groups > 0 && first >= 0 && last > first && last <= length &&
                 epsilon > 0,
             "Invalid risk interval");
  LR_REQUIRE(probabilities && output_projection && projected && margin && result,
             "Expected contiguous CUDA tensor");
  const int64_t count = last - first;
  const int64_t blocks = ceil_div(count, kRiskCandidates);
  risk_kernel<<<blocks, kRiskCandidates * kRiskQueryLanes, 0, as_stream(stream)>>>(
      probabilities, output_projection, projected, margin, result, window, groups, length, first,
      count, static_cast<float>(epsilon));
  return check_launch("temporal_risk");
}

namespace lr {

int launch_pool(const float* scores, int64_t total, const int64_t* bounds, int64_t segments,
                int64_t max_count, int64_t width, float* out, uint32_t* clear, int clear_words,
                hipStream_t stream) {
  const int half = static_cast<int>(width / 2);
  const int use_lds = width <= 4097 ? 1 : 0;
  const size_t lds = use_lds ? (kPoolThreads + 2 * half) * sizeof(float) : 0;
  dim3 grid(static_cast<unsigned>(ceil_div(max_count, kPoolThreads)),
            static_cast<unsigned>(segments));
  pool_kernel<<<grid, kPoolThreads, lds, stream>>>(scores, total, bounds, out, half, use_lds,
                                                   clear, clear_words);
  return check_launch("pool");
}

}  // namespace lr

extern "C" int lr_pool(const float* scores, int64_t total, const int64_t* bounds,
                       int64_t segments, int64_t max_count, int64_t width, float* out,
                       void* stream) {
  clear_error();
  LR_REQUIRE(segments >= 1 && total >= 0, "Invalid pool layout");
  LR_REQUIRE(width > 0 && width % 2 == 1 && max_count > 0, "Invalid pool configuration");
  LR_REQUIRE(segments <= 65535, "Invalid pool layout");
  if (total == 0) return LR_OK;
  LR_REQUIRE(scores && bounds && out, "Expected contiguous CUDA tensor");
  return launch_pool(scores, total, bounds, segments, max_count, width, out, nullptr, 0,
                     as_stream(stream));
}

extern "C" int lr_decision_risk_scores(const float* probabilities, const void* values,
                                       int values_dtype, const float* head_outputs,
                                       const float* gradients, int64_t groups,
                                       int64_t candidates, int64_t head_dim, double base_margin,
                                       double epsilon, float* scores, void* stream) {
  clear_error();
  LR_REQUIRE(epsilon > 0.0 && epsilon < 1.0, "denominator_epsilon must be in (0,1)");
  LR_REQUIRE(groups >= 0 && candidates >= 0 && head_dim >= 0, "candidate count mismatch");
  LR_REQUIRE(values_dtype >= LR_DTYPE_F32 && values_dtype <= LR_DTYPE_BF16, "Invalid dtype");
  if (candidates == 0) return LR_OK;
  LR_REQUIRE(probabilities && values && head_outputs && gradients && scores,
             "probabilities must be CUDA");
  LR_REQUIRE(candidates <= 2147483647LL, "candidate count mismatch");
  const int64_t blocks = candidates;
  const hipStream_t s = as_stream(stream);
  const float eps = static_cast<float>(epsilon);
  switch (values_dtype) {
    case LR_DTYPE_F32:
      decision_risk_kernel<float><<<blocks, 256, 0, s>>>(
          scores, probabilities, static_cast<const float*>(values), head_outputs, gradients, groups,
          candidates, head_dim, base_margin, eps);
      break;
    case LR_DTYPE_F64:
      decision_risk_kernel<double><<<blocks, 256, 0, s>>>(
          scores, probabilities, static_cast<const double*>(values), head_outputs, gradients,
          groups, candidates, head_dim, base_margin, eps);
      break;
    case LR_DTYPE_F16:
      decision_risk_kernel<_Float16><<<blocks, 256, 0, s>>>(
          scores, probabilities, static_cast<const _Float16*>(values), head_outputs, gradients,
          groups, candidates, head_dim, base_margin, eps);
      break;
    default:
      decision_risk_kernel<__bf16><<<blocks, 256, 0, s>>>(
          scores, probabilities, static_cast<const __bf16*>(values), head_outputs,
          gradients, groups, candidates, head_dim, base_margin, eps);
      break;
  }
  return check_launch("decision_risk_scores");
}
