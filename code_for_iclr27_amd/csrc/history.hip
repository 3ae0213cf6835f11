// Device-resident query history: a doubled ring that keeps every layer's last `window` decode
// queries addressable as one strided [Hq, n, d] view, so the scorer reads the window in place.
//
// The reference keeps a deque of per-step [1, Hq, 1, d] tensors per layer and concatenates them
// at every audit (history.py:11-63). Here append k (0-based) writes its rows to ring row
// k mod W and to row k mod W + W of a [layers, Hq, 2W, d] buffer, and its position to the same
// two entries of a [2W] int64 array. After n appends the window is rows [s, s + min(n, W)) with
// s = n mod W once n >= W (else 0): always contiguous, oldest first.

#include <algorithm>

#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kHistoryThreads = 64;  // one wave: 8 workgroups per cfg1 layer, 256 per append

template <int G> struct HistoryGranule;
template <> struct HistoryGranule<16> { typedef unsigned type __attribute__((ext_vector_type(4))); };
template <> struct HistoryGranule<4> { using type = unsigned; };
template <> struct HistoryGranule<2> { using type = unsigned short; };

// Passed by value (1 KiB of kernel arguments): no pointer table to upload per append.
struct LayerPointers {
  const void* ptr[LR_HISTORY_MAX_LAYERS];
};

// grid: (ceil(row granules / threads), layers in this launch). Each granule of one layer's
// [Hq, d] query goes to both copies of its ring row.
template <int G>
__global__ __launch_bounds__(kHistoryThreads) void history_append_kernel(
    LayerPointers sources, int64_t layer_base, int64_t heads, int64_t row_granules,
    int64_t window, int64_t slot, unsigned char* __restrict__ ring, int64_t position,
    int64_t* __restrict__ ring_positions) {
  using T = typename HistoryGranule<G>::type;
  const int64_t layer = layer_base + blockIdx.y;
  const T* source = static_cast<const T*>(sources.ptr[blockIdx.y]);
  const int64_t per_layer = heads * row_granules;
  const int64_t head_stride = 2 * window * row_granules;  // granules between query heads
  T* base = reinterpret_cast<T*>(ring) + layer * heads * head_stride;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kHistoryThreads + threadIdx.x; i < per_layer;
       i += static_cast<int64_t>(gridDim.x) * kHistoryThreads) {
    const int64_t head = i / row_granules, granule = i - head * row_granules;
    const T value = source[i];
    T* row = base + head * head_stride + slot * row_granules + granule;
    row[0] = value;
    row[window * row_granules] = value;
  }
  if (layer == 0 && blockIdx.x == 0 && threadIdx.x == 0) {
    ring_positions[slot] = position;
    ring_positions[slot + window] = position;
  }
}

template <int G>
int launch_append(const void* const* layer_queries, int64_t layers, int64_t heads,
                  int64_t row_bytes, int64_t window, int64_t slot, void* ring, int64_t position,
                  int64_t* ring_positions, hipStream_t stream) {
  const int64_t row_granules = row_bytes / G;
  const int64_t per_layer = heads * row_granules;
  const int64_t blocks = std::min<int64_t>(ceil_div(per_layer, kHistoryThreads), 1024);
  for (int64_t base = 0; base < layers; base += LR_HISTORY_MAX_LAYERS) {
    const int64_t count = std::min<int64_t>(LR_HISTORY_MAX_LAYERS, layers - base);
    LayerPointers sources{};
    for (int64_t l = 0; l < count; ++l) sources.ptr[l] = layer_queries[base + l];
    hipLaunchKernelGGL(history_append_kernel<G>, dim3(blocks, count), dim3(kHistoryThreads), 0,
                       stream, sources, base, heads, row_granules, window, slot,
                       static_cast<unsigned char*>(ring), position, ring_positions);
    if (int status = check_launch("history_append")) return status;
  }
  return LR_OK;
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_history_append(const void* const* layer_queries, int64_t layers, int64_t heads,
                                 int64_t dim, int elem_bytes, int64_t window, int64_t slot,
                                 void* ring, int64_t position, int64_t* ring_positions,
                                 void* stream) {
  clear_error();
  LR_REQUIRE(layer_queries && ring && ring_positions, "Invalid query-history buffers");
  LR_REQUIRE(layers > 0 && heads > 0 && dim > 0 && window > 0, "Invalid query-history shape");
  LR_REQUIRE(elem_bytes == 2 || elem_bytes == 4, "Query history holds 16- or 32-bit queries");
  LR_REQUIRE(slot >= 0 && slot < window, "Query-history slot out of range");
  const int64_t row_bytes = dim * elem_bytes;
  uintptr_t alignment_bits = reinterpret_cast<uintptr_t>(ring) | static_cast<uintptr_t>(row_bytes);
  for (int64_t l = 0; l < layers; ++l) {
    LR_REQUIRE(layer_queries[l] != nullptr, "Invalid query-history buffers");
    alignment_bits |= reinterpret_cast<uintptr_t>(layer_queries[l]);
  }
  const hipStream_t s = as_stream(stream);
  if (alignment_bits % 16 == 0)
    return launch_append<16>(layer_queries, layers, heads, row_bytes, window, slot, ring, position,
                             ring_positions, s);
  if (alignment_bits % 4 == 0)
    return launch_append<4>(layer_queries, layers, heads, row_bytes, window, slot, ring, position,
                            ring_positions, s);
  return launch_append<2>(layer_queries, layers, heads, row_bytes, window, slot, ring, position,
                          ring_positions, s);
}
