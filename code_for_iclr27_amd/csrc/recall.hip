// Device side of the recall transport: one launch per eviction batch for the archive payload of
// every layer, one per search for the query means of every layer.
//
// The reference packs an eviction batch with one _C.pack launch per layer, each after two
// host->device index copies (src/lazy_recall/recall/transport.py:150-167), and forms the search
// queries with a view/float/mean and a copy per layer (transport.py:293-296). Here a batch is a
// list of (layer, head, row) descriptors over a per-layer pointer table, both uploaded in one
// copy, and each is a single launch whatever the layer count.
#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kRecallThreads = 256;

// One thread per 16-byte chunk of a payload row half (key or value): descriptors i = chunk
// index / (2 * chunks), half = which of K and V. The chunk-0 thread of the key half also writes
// the metadata row (layer, head, int64 position), as pack_kernel does (csrc/recall.cu:30-47).
__global__ __launch_bounds__(kRecallThreads) void pack_layers_kernel(
    const int64_t* __restrict__ layer_table, int64_t layers, const int64_t* __restrict__ rows,
    int64_t count, int64_t chunks, uint4* __restrict__ payload, int64_t* __restrict__ metadata) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kRecallThreads + threadIdx.x;
  const int64_t per_row = 2 * chunks;
  if (t >= count * per_row) return;
  const int64_t i = t / per_row;
  const int64_t within = t - i * per_row;
  const int half = within >= chunks ? 1 : 0;
  const int64_t chunk = within - half * chunks;
  const int64_t layer = rows[3 * i], head = rows[3 * i + 1], row = rows[3 * i + 2];
  if (layer < 0 || layer >= layers) return;
  const int64_t* entry = layer_table + 4 * layer;
  if (row < 0 || row >= entry[3]) return;
  const uint4* source = reinterpret_cast<const uint4*>(entry[half]) + row * chunks + chunk;
  payload[(2 * i + half) * chunks + chunk] = *source;
  if (half == 0 && chunk == 0) {
    const float position = reinterpret_cast<const float*>(entry[2])[row];
    metadata[3 * i] = layer;
    metadata[3 * i + 1] = head;
    metadata[3 * i + 2] = static_cast<int64_t>(position);
  }
}

// The eviction batch of a fused layout change (an audit's removals or an evict_prefix batch),
// packed straight from the removal sets the compaction reads, before the compaction: the
// record_evicted call of remove_positions (src/lazy_recall/cache.py:110-112) without the host
// round trip. Block (x, slot) packs part of head slot `slot`'s removed rows; the slot's first
// payload row is the number of rows removed from the slots before it (slot order is (layer,
// head) order, and each slot's positions ascend, so the payload is in the (layer, head,
// position) order record_evicted archives). Rows past `capacity` are not written.
__global__ __launch_bounds__(kRecallThreads) void pack_heads_kernel(
    const int64_t* __restrict__ head_table, int64_t heads_per_layer, const int64_t* __restrict__ quotas,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ positions, int64_t chunks,
    int64_t capacity, uint4* __restrict__ payload, int64_t* __restrict__ metadata) {
  __shared__ int64_t partial[kRecallThreads / 64];
  const int64_t slot = blockIdx.y;
  const int64_t* row = head_table + slot * LR_HEAD_WORDS;
  const int64_t segment = row[4];
  if (segment < 0) return;  // uniform across the block, before the barrier
  const int64_t n = quotas[segment];
  if (n <= 0) return;
  int64_t before = 0;
  for (int64_t k = threadIdx.x; k < slot; k += kRecallThreads) {
    const int64_t other = head_table[k * LR_HEAD_WORDS + 4];
    before += other >= 0 ? quotas[other] : 0;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) before += __shfl_xor(before, o, 64);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = before;
  __syncthreads();
  int64_t first = 0;
#pragma unroll
  for (int w = 0; w < kRecallThreads / 64; ++w) first += partial[w];
  const int64_t length = row[3];
  const int64_t layer = slot / heads_per_layer, head = slot - layer * heads_per_layer;
  const int64_t* removed = positions + offsets[segment];
  const int64_t per_row = 2 * chunks;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * kRecallThreads + threadIdx.x; t < n * per_row;
       t += static_cast<int64_t>(gridDim.x) * kRecallThreads) {
    const int64_t i = t / per_row;
    const int64_t within = t - i * per_row;
    const int half = within >= chunks ? 1 : 0;
    const int64_t chunk = within - half * chunks;
    const int64_t position = removed[i];
    const int64_t out = first + i;
    if (position < 0 || position >= length || out >= capacity) continue;
    const uint4* source = reinterpret_cast<const uint4*>(row[half]) + position * chunks + chunk;
    payload[(2 * out + half) * chunks + chunk] = *source;
    if (half == 0 && chunk == 0) {
      metadata[3 * out] = layer;
      metadata[3 * out + 1] = head;
      metadata[3 * out + 2] = static_cast<int64_t>(reinterpret_cast<const float*>(row[2])[position]);
    }
  }
}

template <typename T>
__device__ __forceinline__ float as_float(T v) { return static_cast<float>(v); }

// One workgroup per layer; thread e of a head's dim elements sums its G query heads in order.
template <typename T>
__global__ __launch_bounds__(kRecallThreads) void group_mean_kernel(
    const int64_t* __restrict__ query_table, int64_t heads, int64_t groups, int64_t dim,
    float* __restrict__ out) {
  const int64_t layer = blockIdx.x;
  const T* queries = reinterpret_cast<const T*>(query_table[2 * layer]);
  const int64_t stride = query_table[2 * layer + 1];
  const float divisor = static_cast<float>(groups);
  for (int64_t e = threadIdx.x; e < heads * dim; e += kRecallThreads) {
    const int64_t h = e / dim, k = e - h * dim;
    float sum = 0.0f;
    for (int64_t g = 0; g < groups; ++g) sum += as_float(queries[(h * groups + g) * stride + k]);
    out[layer * heads * dim + e] = sum / divisor;
  }
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_pack_layers(const int64_t* layer_table, int64_t layers, const int64_t* rows,
                              int64_t count, int64_t dim, void* payload, int64_t* metadata,
                              void* stream) {
  clear_error();
  LR_REQUIRE(layers > 0 && count >= 0 && dim > 0 && (dim * 2) % 16 == 0,
             "Invalid archive payload shape");
  if (count == 0) return LR_OK;
  LR_REQUIRE(layer_table && rows && payload && metadata, "Expected contiguous CUDA tensor");
  LR_REQUIRE(reinterpret_cast<uintptr_t>(payload) % 16 == 0, "Archive payload must be 16-byte aligned");
  const int64_t chunks = dim * 2 / 16;
  const int64_t threads = count * 2 * chunks;
  LR_REQUIRE(threads / kRecallThreads < kMaxGridX, "Archive batch too large");
  pack_layers_kernel<<<static_cast<unsigned>(ceil_div(threads, kRecallThreads)), kRecallThreads, 0,
                       as_stream(stream)>>>(layer_table, layers, rows, count, chunks,
                                            static_cast<uint4*>(payload), metadata);
  return check_launch("pack_layers");
}

extern "C" int lr_pack_heads(const int64_t* head_table, int64_t slots, int64_t heads_per_layer,
                             const int64_t* quotas, const int64_t* offsets,
                             const int64_t* positions, int64_t max_rows, int64_t dim,
                             int64_t capacity, void* payload, int64_t* metadata, void* stream) {
  clear_error();
  LR_REQUIRE(slots > 0 && slots <= 65535 && heads_per_layer > 0 && slots % heads_per_layer == 0,
             "Invalid head table");
  LR_REQUIRE(dim > 0 && (dim * 2) % 16 == 0 && max_rows >= 0 && capacity >= 0,
             "Invalid archive payload shape");
  if (max_rows == 0 || capacity == 0) return LR_OK;
  LR_REQUIRE(head_table && quotas && offsets && positions && payload && metadata,
             "Expected contiguous CUDA tensor");
  LR_REQUIRE(reinterpret_cast<uintptr_t>(payload) % 16 == 0, "Archive payload must be 16-byte aligned");
  const int64_t chunks = dim * 2 / 16;
  int64_t bx = ceil_div(max_rows * 2 * chunks, int64_t{kRecallThreads});
  if (bx > 64) bx = 64;  // the blocks of a slot stride over its rows
  const dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>(slots));
  pack_heads_kernel<<<grid, kRecallThreads, 0, as_stream(stream)>>>(
      head_table, heads_per_layer, quotas, offsets, positions, chunks, capacity,
      static_cast<uint4*>(payload), metadata);
  return check_launch("pack_heads");
}

extern "C" int lr_group_mean_queries(const int64_t* query_table, int64_t layers, int64_t heads,
                                     int64_t groups, int64_t dim, int dtype, float* out,
                                     void* stream) {
  clear_error();
  LR_REQUIRE(layers > 0 && layers < 65536 && heads > 0 && groups > 0 && dim > 0,
             "Invalid recall configuration");
  LR_REQUIRE(query_table && out, "Expected contiguous CUDA tensor");
  const dim3 grid(static_cast<unsigned>(layers));
  switch (dtype) {
    case LR_DTYPE_BF16:
      group_mean_kernel<__bf16><<<grid, kRecallThreads, 0, as_stream(stream)>>>(query_table, heads, groups, dim, out);
      break;
    case LR_DTYPE_F16:
      group_mean_kernel<_Float16><<<grid, kRecallThreads, 0, as_stream(stream)>>>(query_table, heads, groups, dim, out);
      break;
    case LR_DTYPE_F32:
      group_mean_kernel<float><<<grid, kRecallThreads, 0, as_stream(stream)>>>(query_table, heads, groups, dim, out);
      break;
    default:
      LR_REQUIRE(false, "Queries must be float32, float16 or bfloat16");
  }
  return check_launch("group_mean_queries");
}
