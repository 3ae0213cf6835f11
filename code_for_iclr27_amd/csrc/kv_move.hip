// Ragged KV data movement for gfx950: compaction, per-head append, recall merge, archive
// pack and multi-request batch append. Every kernel is a pure row gather, HBM-bound, so the
// design goal is full-width (16-byte) coalesced accesses and as few index computations per
// byte as possible:
//   - a "lane group" of power-of-two lanes moves one row, each lane a 16-byte granule (or the
//     widest granule the row size and pointers allow);
//   - each lane group walks R consecutive output rows, so per-row index work (a binary search
//     in compaction, a descriptor read in batch append) is amortised or incremental;
//   - every index read from device memory is bounds-checked before it is dereferenced.
#include <cstring>

#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kThreads = 256;
constexpr int kBatch = 4;  // rows a lane group copies with all their loads in flight together

struct RowLayout {
  int64_t row_bytes;  // bytes per row (dim * element size)
  int64_t chunks;     // granules per row
  int lanes_log2;     // log2(lanes per row group), lanes <= 64
  int rows_per_group; // consecutive rows walked by one lane group
};

inline int log2_ceil(int64_t v) {
  int l = 0;
  while ((int64_t{1} << l) < v) ++l;
  return l;
}

// Lane-group geometry: up to 64 lanes per row, enough lane groups to fill 256 CUs.
inline RowLayout make_layout(int64_t row_bytes, int granule, int64_t rows, int max_rows_per_group) {
  RowLayout layout;
  layout.row_bytes = row_bytes;
  layout.chunks = row_bytes / granule;
  layout.lanes_log2 = log2_ceil(layout.chunks < 64 ? layout.chunks : 64);
  const int64_t lanes = int64_t{1} << layout.lanes_log2;
  const int64_t target_groups = (int64_t{256} * 2048) / lanes;  // ~full residency on 256 CUs
  // whole batches of rows per lane group (the kernels copy kBatch rows at a time)
  int64_t r = ceil_div(ceil_div(rows, target_groups), kBatch) * kBatch;
  if (r < kBatch) r = kBatch;
  if (r > max_rows_per_group) r = max_rows_per_group;
  layout.rows_per_group = static_cast<int>(r);
  return layout;
}

inline int64_t blocks_for(const RowLayout& layout, int64_t rows) {
  const int64_t groups_per_block = kThreads >> layout.lanes_log2;
  const int64_t groups = ceil_div(rows, layout.rows_per_group);
  int64_t blocks = ceil_div(groups, groups_per_block);
  if (blocks < 1) blocks = 1;
  return blocks < kMaxGridX ? blocks : kMaxGridX;
}

template <int G> struct RawGranule;  // plain vector types: arrays of them stay in registers
template <> struct RawGranule<16> { typedef unsigned type __attribute__((ext_vector_type(4))); };
template <> struct RawGranule<8> { typedef unsigned type __attribute__((ext_vector_type(2))); };
template <> struct RawGranule<4> { using type = unsigned; };
template <> struct RawGranule<2> { using type = unsigned short; };
template <> struct RawGranule<1> { using type = unsigned char; };

// The same pointer in the global address space (lets the compiler emit global_* instead of
// flat_* memory instructions for pointers read from device tables).
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* global_ptr(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* global_ptr(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

// Lane-group coordinates shared by the row kernels.
struct GroupCoord {
  int lane, lanes, group, groups_per_block;
};

// Every row kernel runs with kThreads threads per block; the constant spares each kernel a
// dependent load of the block size at its start.
__device__ __forceinline__ GroupCoord group_coord(int lanes_log2) {
  GroupCoord g;
  g.lanes = 1 << lanes_log2;
  g.lane = threadIdx.x & (g.lanes - 1);
  g.group = threadIdx.x >> lanes_log2;
  g.groups_per_block = kThreads >> lanes_log2;
  return g;
}

// A lane group's batch of up to kBatch rows of one or two tensors (K and V). Every lane issues
// all its loads of the batch before any store: a load issued under a per-row branch would be
// waited for before the next one. Rows that are not copied read `src` = a readable fallback
// row and store nothing.
//
// Cache policy of the row copies (measured per kernel on gfx950): the all-layer kernels that
// move hundreds of MB run faster with nontemporal (`nt`) accesses, which stream past the
// caches (compaction and reinsertion: loads and stores; the all-layer append: stores only),
// while the per-layer drop-ins (one layer, tens of MB, often still in the 256 MB Infinity
// Cache) are slower with them and keep the default forms.
enum CopyPolicy : int { kCached = 0, kStreamStores = 2, kStreamAll = 3 };

template <bool kTwo>
struct RowBatch {
  const uint8_t* src[kBatch];
  uint8_t* dst[kBatch];
  const uint8_t* src2[kBatch];
  uint8_t* dst2[kBatch];
  bool ok[kBatch];
};

template <int P, typename V>
__device__ __forceinline__ V load_granule(const uint8_t* row, int64_t c) {
  const auto p = global_ptr(reinterpret_cast<const V*>(row)) + c;
  if constexpr ((P & 1) != 0) return __builtin_nontemporal_load(p);
  else return *p;
}

template <int P, typename V>
__device__ __forceinline__ void store_granule(uint8_t* row, int64_t c, V v) {
  const auto p = global_ptr(reinterpret_cast<V*>(row)) + c;
  if constexpr ((P & 2) != 0) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <int G, bool kTwo, int P = kCached>
__device__ __forceinline__ void copy_batch(const RowBatch<kTwo>& b, int64_t chunks, int lane,
                                           int lanes) {
  using V = typename RawGranule<G>::type;
  for (int64_t c = lane; c < chunks; c += lanes) {
    V x[kBatch], y[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      x[u] = load_granule<P, V>(b.src[u], c);
      if constexpr (kTwo) y[u] = load_granule<P, V>(b.src2[u], c);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (b.ok[u]) {
        store_granule<P, V>(b.dst[u], c, x[u]);
        if constexpr (kTwo) store_granule<P, V>(b.dst2[u], c, y[u]);
      }
    }
  }
}

// Granules [0, count) of one or two flat ranges (K and V), `U` granules per thread at a
// stride of the whole grid row (`first` = the thread's index in that row), every load of a
// round issued before its stores, each wave instruction on one contiguous span.
template <int U, int P, bool kTwo, typename V>
__device__ __forceinline__ void flat_copy(const V* src, V* dst, const V* src2, V* dst2,
                                          int64_t count, int64_t first, int64_t stride) {
  const auto s1 = global_ptr(src);
  const auto s2 = global_ptr(src2);
  const auto d1 = global_ptr(dst);
  const auto d2 = global_ptr(dst2);
  auto load = [](auto p) {
    if constexpr ((P & 1) != 0) return __builtin_nontemporal_load(p);
    else return *p;
  };
  auto store = [](auto p, V v) {
    if constexpr ((P & 2) != 0) __builtin_nontemporal_store(v, p);
    else *p = v;
  };
  const int64_t end = count;
  int64_t i = first;
  for (; i + (U - 1) * stride < end; i += U * stride) {
    V x[U], y[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      x[u] = load(s1 + i + u * stride);
      if constexpr (kTwo) y[u] = load(s2 + i + u * stride);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      store(d1 + i + u * stride, x[u]);
      if constexpr (kTwo) store(d2 + i + u * stride, y[u]);
    }
  }
  V x[U], y[U];  // the rest: fewer than U granules for this thread
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (i + u * stride < end) {
      x[u] = load(s1 + i + u * stride);
      if constexpr (kTwo) y[u] = load(s2 + i + u * stride);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (i + u * stride < end) {
      store(d1 + i + u * stride, x[u]);
      if constexpr (kTwo) store(d2 + i + u * stride, y[u]);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Compaction of one row range: output rows [d0, d0 + n) of a head of `length` rows minus the
// sorted removal list `removed` land at out_start + d0... Output d takes input d + j,
// j = #{i : removed[i] - i <= d} (the gather rule of csrc/scoring.cu:164-188). The block first
// maps each of its n <= kCompactRows output rows to its source by binary search over the
// removal list (staged in LDS when it fits), one row per thread, copying the positions on the
// way; then its lane groups copy the rows in batches. Called by every thread of the block (it
// has barriers).
constexpr int kCompactRows = 128;     // most output rows per block (measured faster than 256)
constexpr int kCompactStaged = 4096;  // removal entries staged in LDS (larger lists: global)
static_assert(kCompactRows <= kThreads, "one thread maps each output row of a block");

template <int G, int P>
__device__ __forceinline__ void compact_block(const uint8_t* keys, const uint8_t* values,
                                              const float* positions, int64_t length,
                                              const int64_t* removed, int64_t removed_count,
                                              int64_t d0, int n, int64_t out_start,
                                              const RowLayout& layout, uint8_t* out_keys,
                                              uint8_t* out_values, float* out_positions) {
  __shared__ int32_t staged[kCompactStaged];
  __shared__ int64_t source[kCompactRows];
  const bool in_lds = removed_count <= kCompactStaged;
  if (in_lds)
    for (int64_t i = threadIdx.x; i < removed_count; i += kThreads)
      staged[i] = static_cast<int32_t>(removed[i]);
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < n) {
    const int64_t d = d0 + threadIdx.x;
    int64_t lo = 0, hi = removed_count;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      const int64_t r = in_lds ? staged[mid] : removed[mid];
      if (r - mid <= d) lo = mid + 1;
      else hi = mid;
    }
    const int64_t src = d + lo;
    const bool valid = src < length;  // a malformed removal list can point past the head
    source[threadIdx.x] = valid ? src : -1;
    if (valid) out_positions[out_start + d] = positions[src];
  }
  __syncthreads();
  const GroupCoord gc = group_coord(layout.lanes_log2);
  const int64_t rb = layout.row_bytes;
  for (int r0 = gc.group; r0 < n; r0 += gc.groups_per_block * kBatch) {
    RowBatch<true> b;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int r = r0 + u * gc.groups_per_block;
      const int64_t src = r < n ? source[r] : -1;
      const int64_t from = src >= 0 ? src : 0;  // n > 0, so row 0 of the head exists
      b.ok[u] = src >= 0;
      b.src[u] = keys + from * rb;
      b.src2[u] = values + from * rb;
      b.dst[u] = out_keys + (out_start + d0 + r) * rb;
      b.dst2[u] = out_values + (out_start + d0 + r) * rb;
    }
    copy_batch<G, true, P>(b, layout.chunks, gc.lane, gc.lanes);
  }
}

// compact (csrc/scoring.cu:294-314): one flat [rows_in, dim] cache, block x = output rows
// [x * rows_per_block, ...), rows_per_block <= kCompactRows.
template <int G>
__global__ __launch_bounds__(kThreads) void compact_kernel(
    const uint8_t* __restrict__ keys, const uint8_t* __restrict__ values,
    const float* __restrict__ positions, const int64_t* __restrict__ removed,
    int64_t removed_count, int64_t rows_in, int64_t rows_out, int rows_per_block,
    RowLayout layout, uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions) {
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  if (d0 >= rows_out) return;  // uniform across the block
  const int n = static_cast<int>(rows_out - d0 < rows_per_block ? rows_out - d0 : rows_per_block);
  compact_block<G, kCached>(keys, values, positions, rows_in, removed, removed_count, d0, n, 0,
                            layout, out_keys, out_values, out_positions);
}

// ---------------------------------------------------------------------------------------
// Per-head ragged append (csrc/scoring.cu:130-162 and csrc/cache_legacy.cu:13-40): head h's
// old rows move from src_start(h) to dst_start(h) = src_start(h) + h * added, followed by
// `added` new rows. blockIdx.y = head; rows of a head are covered up to `covered_rows`.
template <int G, bool kWithPositions, int P>
__device__ __forceinline__ void head_append(
    const uint8_t* __restrict__ cache_keys, const uint8_t* __restrict__ cache_values,
    const float* __restrict__ positions, int64_t rows_in, const uint8_t* __restrict__ new_keys,
    const uint8_t* __restrict__ new_values, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ lengths_or_next, int lengths_are_cumulative, int64_t heads,
    int64_t added, int64_t covered_rows, int64_t logical_start, const RowLayout& layout,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int32_t* __restrict__ out_cumulative,
    int32_t* __restrict__ out_lengths) {
  constexpr bool kTwo = kWithPositions;  // the legacy single-tensor form has no values
  const GroupCoord gc = group_coord(layout.lanes_log2);
  const int64_t head = blockIdx.y;
  const int64_t old_start = starts[head];
  const int64_t old_length = lengths_are_cumulative ? lengths_or_next[head + 1] - old_start
                                                    : lengths_or_next[head];
  const int64_t new_start = old_start + head * added;
  if (out_cumulative != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    out_cumulative[head] = static_cast<int32_t>(new_start);
    out_lengths[head] = static_cast<int32_t>(old_length + added);
    if (head == heads - 1)
      out_cumulative[heads] = static_cast<int32_t>(lengths_or_next[heads] + heads * added);
  }
  int64_t total = old_length + added;
  if (total > covered_rows) total = covered_rows;
  const int64_t rows_out = rows_in + heads * added;
  const int64_t R = layout.rows_per_group;
  const int64_t rb = layout.row_bytes;
  for (int64_t first = (static_cast<int64_t>(blockIdx.x) * gc.groups_per_block + gc.group) * R;
       first < total;
       first += static_cast<int64_t>(gridDim.x) * gc.groups_per_block * R) {
    const int64_t end = first + R < total ? first + R : total;
    // skipped copies read the first new row, or with no new rows the first cache row (the
    // host returns early when there are neither)
    const uint8_t* fallback = added > 0 ? new_keys : cache_keys;
    const uint8_t* fallback2 = added > 0 ? new_values : cache_values;
    for (int64_t p0 = first; p0 < end; p0 += kBatch) {
      RowBatch<kTwo> b;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t p = p0 + u, dst = new_start + p;
        const bool old = p < old_length;
        const int64_t src = old ? old_start + p : head * added + (p - old_length);
        const bool ok = p < end && dst >= 0 && dst < rows_out && (!old || (src >= 0 && src < rows_in));
        b.ok[u] = ok;
        b.src[u] = !ok ? fallback : old ? cache_keys + src * rb : new_keys + src * rb;
        b.dst[u] = out_keys + dst * rb;
        if constexpr (kTwo) {
          b.src2[u] = !ok ? fallback2 : old ? cache_values + src * rb : new_values + src * rb;
          b.dst2[u] = out_values + dst * rb;
        }
      }
      float position[kBatch];
      if constexpr (kWithPositions) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int64_t p = p0 + u;
          const bool old = b.ok[u] && p < old_length;
          // rows without an old position read the first one (only when the cache has rows)
          const float loaded = rows_in > 0 ? positions[old ? old_start + p : 0] : 0.0f;
          position[u] = old ? loaded : static_cast<float>(logical_start + (p - old_length));
        }
      }
      copy_batch<G, kTwo, P>(b, layout.chunks, gc.lane, gc.lanes);
      if (kWithPositions && gc.lane == 0) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
          if (b.ok[u]) out_positions[new_start + p0 + u] = position[u];
      }
    }
  }
}

// The same append as flat copies: a head's old rows are one contiguous run in the cache and
// in the output (and its new rows one run in new_keys), so the rows the checks above admit form
// one interval per run, copied granule by granule with `U` granules per thread in flight. The
// positions and the output metadata follow the row form exactly.
template <int G, bool kWithPositions, int P, int U, int kBlock>
__device__ __forceinline__ void head_append_flat(
    const uint8_t* __restrict__ cache_keys, const uint8_t* __restrict__ cache_values,
    const float* __restrict__ positions, int64_t rows_in, const uint8_t* __restrict__ new_keys,
    const uint8_t* __restrict__ new_values, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ lengths_or_next, int lengths_are_cumulative, int64_t heads,
    int64_t added, int64_t covered_rows, int64_t logical_start, int64_t row_bytes,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int32_t* __restrict__ out_cumulative,
    int32_t* __restrict__ out_lengths) {
  constexpr bool kTwo = kWithPositions;  // the legacy single-tensor form has no values
  using V = typename RawGranule<G>::type;
  const int64_t head = blockIdx.y;
  const int64_t old_start = starts[head];
  const int64_t old_length = lengths_are_cumulative ? lengths_or_next[head + 1] - old_start
                                                    : lengths_or_next[head];
  const int64_t new_start = old_start + head * added;
  if (out_cumulative != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    out_cumulative[head] = static_cast<int32_t>(new_start);
    out_lengths[head] = static_cast<int32_t>(old_length + added);
    if (head == heads - 1)
      out_cumulative[heads] = static_cast<int32_t>(lengths_or_next[heads] + heads * added);
  }
  int64_t total = old_length + added;
  if (total > covered_rows) total = covered_rows;
  const int64_t rows_out = rows_in + heads * added;
  const int64_t rg = row_bytes / G;  // granules per row
  // the block size as a constant: blockDim would be one more dependent load at the start
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  // rows p with a destination in the output: [-new_start, rows_out - new_start)
  const int64_t dst_lo = -new_start, dst_hi = rows_out - new_start;
  // old rows: p < old_length with the source row inside the cache
  int64_t lo = max(max(int64_t{0}, dst_lo), -old_start);
  int64_t hi = min(min(old_length, total), min(dst_hi, rows_in - old_start));
  auto out_k = [&](int64_t p) { return reinterpret_cast<V*>(out_keys) + (new_start + p) * rg; };
  auto out_v = [&](int64_t p) {
    return kTwo ? reinterpret_cast<V*>(out_values) + (new_start + p) * rg : nullptr;
  };
  if (lo < hi)
    flat_copy<U, P, kTwo>(
        reinterpret_cast<const V*>(cache_keys) + (old_start + lo) * rg, out_k(lo),
        kTwo ? reinterpret_cast<const V*>(cache_values) + (old_start + lo) * rg : nullptr,
        out_v(lo), (hi - lo) * rg, first, stride);
  // new rows: p in [old_length, total), row head * added + (p - old_length) of the new rows
  lo = max(max(int64_t{0}, dst_lo), old_length);
  hi = min(total, dst_hi);
  if (lo < hi) {
    const int64_t row = head * added + (lo - old_length);
    flat_copy<1, P, kTwo>(reinterpret_cast<const V*>(new_keys) + row * rg, out_k(lo),
                          kTwo ? reinterpret_cast<const V*>(new_values) + row * rg : nullptr,
                          out_v(lo), (hi - lo) * rg, first, stride);
  }
  if constexpr (kWithPositions) {
    for (int64_t p = first; p < total; p += stride) {
      const int64_t dst = new_start + p;
      const bool old = p < old_length;
      const int64_t src = old_start + p;
      if (dst < 0 || dst >= rows_out || (old && (src < 0 || src >= rows_in))) continue;
      out_positions[dst] = old ? positions[src] : static_cast<float>(logical_start + (p - old_length));
    }
  }
}

// The per-layer appends (one layer, tens of MB: a single round of copies over the chip) in
// two-wave workgroups of two granules per thread and tensor (measured fastest of 64-256
// threads with 1-8 granules for a cfg1 layer).
constexpr int kAppendThreads = 128;
constexpr int kAppendLayerUnroll = 2;

template <int G, bool kWithPositions>
__global__ __launch_bounds__(kAppendThreads) void head_append_kernel(
    const uint8_t* __restrict__ cache_keys, const uint8_t* __restrict__ cache_values,
    const float* __restrict__ positions, int64_t rows_in, const uint8_t* __restrict__ new_keys,
    const uint8_t* __restrict__ new_values, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ lengths_or_next, int lengths_are_cumulative, int64_t heads,
    int64_t added, int64_t covered_rows, int64_t logical_start, int64_t row_bytes,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int32_t* __restrict__ out_cumulative,
    int32_t* __restrict__ out_lengths) {
  head_append_flat<G, kWithPositions, kCached, kAppendLayerUnroll, kAppendThreads>(
      cache_keys, cache_values, positions, rows_in, new_keys, new_values, starts, lengths_or_next,
      lengths_are_cumulative, heads, added, covered_rows, logical_start, row_bytes, out_keys,
      out_values, out_positions, out_cumulative, out_lengths);
}

// One decode step's append into every layer (blockIdx.z = layer): the per-layer append above
// with its arguments from a table of LR_APPEND_WORDS i64 per layer, all layers' outputs packed
// into one K, V and positions buffer (layer l from its output row [8]) and one [L, heads + 1]
// cumulative / [L, heads] lengths pair. The table comes from memory, or (up to
// kInlineLayers layers, their first kAppendRowWords words) in the launch's kernel arguments.
constexpr int kAppendRowWords = 9;  // the words of a table row the kernel reads
constexpr int kInlineLayers = 48;
struct InlineAppendTable {
  int64_t words[kInlineLayers * kAppendRowWords];
};

template <int G>
__device__ __forceinline__ void append_layer(const int64_t (&row)[kAppendRowWords], int64_t layer,
                                             int64_t heads, int64_t added, int64_t covered_rows,
                                             const RowLayout& layout, uint8_t* out_keys,
                                             uint8_t* out_values, float* out_positions,
                                             int32_t* out_cumulative, int32_t* out_lengths) {
  const int64_t first = row[8];
  const int32_t* cumulative = reinterpret_cast<const int32_t*>(row[4]);
  head_append<G, true, kStreamStores>(
      reinterpret_cast<const uint8_t*>(row[0]), reinterpret_cast<const uint8_t*>(row[1]),
      reinterpret_cast<const float*>(row[2]), row[3], reinterpret_cast<const uint8_t*>(row[5]),
      reinterpret_cast<const uint8_t*>(row[6]), cumulative, cumulative, 1, heads, added,
      covered_rows, row[7], layout, out_keys + first * layout.row_bytes,
      out_values + first * layout.row_bytes, out_positions + first,
      out_cumulative + layer * (heads + 1), out_lengths + layer * heads);
}

template <int G>
__global__ __launch_bounds__(kThreads) void append_layers_kernel(
    const int64_t* __restrict__ table, int64_t heads, int64_t added, int64_t covered_rows,
    RowLayout layout, uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int32_t* __restrict__ out_cumulative,
    int32_t* __restrict__ out_lengths) {
  const int64_t layer = blockIdx.z;
  int64_t row[kAppendRowWords];
#pragma unroll
  for (int i = 0; i < kAppendRowWords; ++i) row[i] = table[layer * LR_APPEND_WORDS + i];
  append_layer<G>(row, layer, heads, added, covered_rows, layout, out_keys, out_values,
                  out_positions, out_cumulative, out_lengths);
}

template <int G>
__global__ __launch_bounds__(kThreads) void append_layers_inline_kernel(
    const InlineAppendTable table, int64_t heads, int64_t added, int64_t covered_rows,
    RowLayout layout, uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int32_t* __restrict__ out_cumulative,
    int32_t* __restrict__ out_lengths) {
  const int64_t layer = blockIdx.z;
  int64_t row[kAppendRowWords];
#pragma unroll
  for (int i = 0; i < kAppendRowWords; ++i) row[i] = table.words[layer * kAppendRowWords + i];
  append_layer<G>(row, layer, heads, added, covered_rows, layout, out_keys, out_values,
                  out_positions, out_cumulative, out_lengths);
}

// ---------------------------------------------------------------------------------------
// Indexed gathers. kMode selects the index rule:
//   0 keep      (compact_flattened_kv, csrc/cache_legacy.cu:42-61): src = index[r]
//   1 merge     (csrc/recall.cu:7-28): index[r] >= 0 existing row, else recalled[-index[r]-1]
//   2 pack      (csrc/recall.cu:30-47): src = index[r], output interleaved [r, {K,V}]
enum GatherMode { kKeep = 0, kMerge = 1, kPack = 2 };

template <int G, int kMode>
__global__ __launch_bounds__(kThreads) void gather_kernel(
    const uint8_t* __restrict__ keys, const uint8_t* __restrict__ values,
    const float* __restrict__ positions, int64_t rows_in, const int64_t* __restrict__ index,
    int64_t rows_out, const uint8_t* __restrict__ recalled,
    const float* __restrict__ recalled_positions, int64_t recalled_rows,
    const int64_t* __restrict__ heads, int64_t layer, RowLayout layout,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int64_t* __restrict__ metadata) {
  const GroupCoord gc = group_coord(layout.lanes_log2);
  const int64_t R = layout.rows_per_group;
  const int64_t rb = layout.row_bytes;
  // a readable row for copies that are skipped; with none, no index can be valid
  const uint8_t* fallback = rows_in > 0 ? keys : recalled_rows > 0 ? recalled : nullptr;
  if (fallback == nullptr) return;
  const float* fallback_position = rows_in > 0 ? positions : recalled_positions;
  for (int64_t first = (static_cast<int64_t>(blockIdx.x) * gc.groups_per_block + gc.group) * R;
       first < rows_out;
       first += static_cast<int64_t>(gridDim.x) * gc.groups_per_block * R) {
    const int64_t end = first + R < rows_out ? first + R : rows_out;
    for (int64_t r0 = first; r0 < end; r0 += kBatch) {
      // every load of the batch is unconditional (clamped indices, fallback rows), so none is
      // waited for before the next is issued
      int64_t source[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) source[u] = index[r0 + u < end ? r0 + u : end - 1];
      RowBatch<true> b;
      const float* from_position[kBatch];
      int64_t head_of[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t r = r0 + u, src = source[u];
        const bool from_recalled = kMode == kMerge && src < 0 && src != INT64_MIN;
        const int64_t restored = from_recalled ? -src - 1 : 0;
        bool ok;
        if (from_recalled) {
          ok = restored < recalled_rows;
          b.src[u] = ok ? recalled + (2 * restored) * rb : fallback;
          b.src2[u] = ok ? recalled + (2 * restored + 1) * rb : fallback;
          from_position[u] = ok ? recalled_positions + restored : fallback_position;
        } else {
          ok = src >= 0 && src < rows_in;
          b.src[u] = ok ? keys + src * rb : fallback;
          b.src2[u] = ok ? values + src * rb : fallback;
          from_position[u] = ok ? positions + src : fallback_position;
        }
        b.ok[u] = ok && r < end;
        if (kMode == kPack) {
          b.dst[u] = out_keys + (2 * r) * rb;
          b.dst2[u] = out_keys + (2 * r + 1) * rb;
          head_of[u] = heads[r < end ? r : end - 1];
        } else {
          b.dst[u] = out_keys + r * rb;
          b.dst2[u] = out_values + r * rb;
        }
      }
      float position[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) position[u] = kMode == kKeep ? 0.0f : *from_position[u];
      copy_batch<G, true>(b, layout.chunks, gc.lane, gc.lanes);
      if (gc.lane == 0) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if (!b.ok[u]) continue;
          const int64_t r = r0 + u;
          if (kMode == kPack) {
            metadata[3 * r] = layer;
            metadata[3 * r + 1] = head_of[u];
            metadata[3 * r + 2] = static_cast<int64_t>(position[u]);
          } else if (kMode == kMerge) {
            out_positions[r] = position[u];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// batch_append (csrc/batch_append.cu:8-34): blockIdx.y = (request, head) segment with the
// reference's 7-word descriptor; the segment's old rows then its one new row are written
// contiguously from the destination row. The descriptor comes either from memory (a device or
// host-coherent array) or from the launch's kernel arguments (batches of up to
// kInlineSegments segments, read with scalar loads from the kernel-argument segment).
//
// A segment's old rows are contiguous in the source cache and in the output, so K and V are
// each one flat copy of old rows x row bytes: every thread moves kAppendUnroll granules of
// each at a stride of the segment's whole grid row, all loads issued before the stores, and
// every wave instruction touches one contiguous span. The new row and the positions follow.
constexpr int kInlineSegments = 64;
constexpr int kAppendUnroll = 8;
struct InlineDescriptors {
  int64_t words[kInlineSegments * 7];
};

template <int G>
__device__ __forceinline__ void batch_append_segment(
    const int64_t (&d)[7], int64_t segment, const uint8_t* __restrict__ new_keys,
    const uint8_t* __restrict__ new_values, int64_t max_rows, int64_t row_bytes,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions) {
  using T = typename RawGranule<G>::type;
  const int64_t source = d[3], old_length = d[4], destination = d[5], logical = d[6];
  int64_t total = old_length + 1;
  if (total > max_rows) total = max_rows;
  const int64_t old_rows = old_length < total ? old_length : total;
  const int64_t rg = row_bytes / G;  // granules per row
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  flat_copy<kAppendUnroll, kCached, true>(
      reinterpret_cast<const T*>(reinterpret_cast<const uint8_t*>(d[0]) + source * row_bytes),
      reinterpret_cast<T*>(out_keys + destination * row_bytes),
      reinterpret_cast<const T*>(reinterpret_cast<const uint8_t*>(d[1]) + source * row_bytes),
      reinterpret_cast<T*>(out_values + destination * row_bytes), old_rows * rg, first, stride);
  if (old_rows < total)  // the new row (only when the clamp left room for it)
    flat_copy<1, kCached, true>(
        reinterpret_cast<const T*>(new_keys + segment * row_bytes),
        reinterpret_cast<T*>(out_keys + (destination + old_rows) * row_bytes),
        reinterpret_cast<const T*>(new_values + segment * row_bytes),
        reinterpret_cast<T*>(out_values + (destination + old_rows) * row_bytes), rg, first, stride);
  const auto positions = global_ptr(reinterpret_cast<const float*>(d[2]));
  for (int64_t p = first; p < total; p += stride)
    out_positions[destination + p] = p < old_rows ? positions[source + p] : static_cast<float>(logical);
}

template <int G>
__global__ __launch_bounds__(kThreads) void batch_append_kernel(
    const int64_t* __restrict__ descriptors, const uint8_t* __restrict__ new_keys,
    const uint8_t* __restrict__ new_values, int64_t max_rows, int64_t row_bytes,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions) {
  const int64_t segment = blockIdx.y;
  int64_t d[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) d[i] = descriptors[segment * 7 + i];
  batch_append_segment<G>(d, segment, new_keys, new_values, max_rows, row_bytes, out_keys,
                          out_values, out_positions);
}

template <int G>
__global__ __launch_bounds__(kThreads) void batch_append_inline_kernel(
    const InlineDescriptors descriptors, const uint8_t* __restrict__ new_keys,
    const uint8_t* __restrict__ new_values, int64_t max_rows, int64_t row_bytes,
    uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions) {
  const int64_t segment = blockIdx.y;
  int64_t d[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) d[i] = descriptors.words[segment * 7 + i];
  batch_append_segment<G>(d, segment, new_keys, new_values, max_rows, row_bytes, out_keys,
                          out_values, out_positions);
}

// ---------------------------------------------------------------------------------------
// Audit-step compaction of every (layer, KV head) in one launch (the per-layer loop of
// cache.py:113-178). blockIdx.y = head slot; each head keeps its rows minus the sorted
// head-relative removal list of its score segment, and lands in one packed output at
// sum over earlier head slots of (length - quota), derived here from the quotas. Block x
// covers output rows [x * kCompactRows, ...) of its head.
template <int G>
__global__ __launch_bounds__(kThreads) void compact_heads_kernel(
    const int64_t* __restrict__ head_table, const int64_t* __restrict__ quotas,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ removed_positions,
    RowLayout layout, uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions, int64_t heads_per_layer, int32_t* __restrict__ head_lens,
    int32_t* __restrict__ cumulative) {
  __shared__ int64_t partial[kThreads / 64];
  const int64_t head = blockIdx.y;
  const int64_t* row = head_table + head * LR_HEAD_WORDS;
  const int64_t length = row[3], segment = row[4];
  const int64_t removed_count = segment >= 0 ? quotas[segment] : 0;
  const int64_t rows_out = length - removed_count;
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kCompactRows;
  if (head_lens != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    // the layer's new metadata (cache.py:171-177): this head's length and its end in the
    // layer's cumulative lengths; the layer's first head also writes the leading 0
    const int64_t layer = head / heads_per_layer, h = head - layer * heads_per_layer;
    int64_t end = 0;
    for (int64_t k = layer * heads_per_layer; k <= head; ++k) {
      const int64_t* other = head_table + k * LR_HEAD_WORDS;
      end += other[3] - (other[4] >= 0 ? quotas[other[4]] : 0);
    }
    head_lens[head] = static_cast<int32_t>(rows_out);
    cumulative[layer * (heads_per_layer + 1) + h + 1] = static_cast<int32_t>(end);
    if (h == 0) cumulative[layer * (heads_per_layer + 1)] = 0;
  }
  if (d0 >= rows_out) return;  // uniform across the block, before any barrier
  // output start of this head slot
  int64_t before = 0;
  for (int64_t h = threadIdx.x; h < head; h += kThreads) {
    const int64_t* other = head_table + h * LR_HEAD_WORDS;
    before += other[3] - (other[4] >= 0 ? quotas[other[4]] : 0);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) before += __shfl_xor(before, o, 64);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = before;
  __syncthreads();
  int64_t out_start = 0;
  for (int w = 0; w < kThreads / 64; ++w) out_start += partial[w];
  const int n = static_cast<int>(rows_out - d0 < kCompactRows ? rows_out - d0 : kCompactRows);
  compact_block<G, kStreamAll>(
      reinterpret_cast<const uint8_t*>(row[0]), reinterpret_cast<const uint8_t*>(row[1]),
      reinterpret_cast<const float*>(row[2]), length,
      segment >= 0 ? removed_positions + offsets[segment] : nullptr, removed_count, d0, n,
      out_start, layout, out_keys, out_values, out_positions);
}

// ---------------------------------------------------------------------------------------
// Reinsertion of recalled rows into every layer at once (insert_payload, src/lazy_recall/
// cache.py:201-253, with merge_plan, recall/planning.py:34-52, and _C.merge, csrc/recall.cu:
// 7-28). A head's resident positions ascend (the cache keeps them so), its recalled positions
// come in any order; the merged head holds both, ascending. Instead of a per-row source mapping
// the rows are scattered: resident row j of a head goes to j + (recalled positions below it),
// recalled row k (k-th smallest) to k + (resident positions below it). So the resident rows,
// almost every byte, need only the recalled positions, not the recalled payload, and can move
// while the payload is still being copied in.
//
// Reinsert table, LR_REINSERT_WORDS i64 per (layer, KV head) slot:
//   [0] keys ptr, [1] values ptr, [2] positions ptr (f32) of the head's first resident row,
//   [3] resident rows, [4] first entry of the head's recalled run, [5] recalled rows of the
//   head, [6] first output row of the merged head, [7] unused (0).
constexpr int kPlanRankMax = 1024;  // runs the plan sorts by rank counting (else bitonic)
constexpr int kReinsertMax = LR_REINSERT_MAX_PER_HEAD;  // recalled rows of one head (sorted in LDS)

// One workgroup per slot: its recalled entries sorted by position in LDS (bitonic), each one's
// insertion point among the resident positions (binary search), duplicates flagged (bit 1);
// writes the sorted run back with each entry's absolute output row, and each input entry's row
// within its merged head.
__global__ __launch_bounds__(kThreads) void reinsert_plan_kernel(
    const int64_t* __restrict__ table, const int64_t* __restrict__ grouped,
    int64_t* __restrict__ sorted_position, int64_t* __restrict__ sorted_source,
    int64_t* __restrict__ sorted_destination, int64_t* __restrict__ recalled_rows, int64_t count,
    int32_t* __restrict__ flag, int64_t heads_per_layer, int32_t* __restrict__ head_lens,
    int32_t* __restrict__ cumulative) {
  __shared__ int64_t key[kReinsertMax];
  __shared__ int64_t value[kReinsertMax];
  __shared__ __align__(16) uint64_t packed[kPlanRankMax + 2];
  const int64_t slot = blockIdx.x;
  const int64_t* entry = table + slot * LR_REINSERT_WORDS;
  const int64_t first = entry[4], r = entry[5];
  if (head_lens != nullptr && threadIdx.x < 64) {
    // the layer's new metadata (replace_head_lens after insert_payload, cache.py:246): this
    // head's merged length and its end in the layer's cumulative lengths, the heads up to this
    // one summed across the first wave (their table rows loaded at once)
    const int64_t layer = slot / heads_per_layer, h = slot - layer * heads_per_layer;
    int64_t part = 0;
    for (int64_t k = threadIdx.x; k <= h; k += 64) {
      const int64_t* row = table + (layer * heads_per_layer + k) * LR_REINSERT_WORDS;
      part += row[3] + row[5];
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) part += __shfl_xor(part, offset);
    if (threadIdx.x == 0) {
      head_lens[slot] = static_cast<int32_t>(entry[3] + r);
      cumulative[layer * (heads_per_layer + 1) + h + 1] = static_cast<int32_t>(part);
      if (h == 0) cumulative[layer * (heads_per_layer + 1)] = 0;
    }
  }
  if (r == 0) return;
  if (r > kReinsertMax) {
    if (threadIdx.x == 0) atomicOr(flag, 8);
    return;
  }
  int n2 = 1;
  while (n2 < r) n2 <<= 1;
  // Runs of up to kPlanRankMax entries whose (position, source) pairs pack into one u64 each
  // (position in [0, 2^31), source in [0, 2^32)) are sorted by rank counting: every entry
  // counts the smaller packed pairs in LDS, then moves to its rank. The pairs are unique (one
  // source per entry), so the ranks are a permutation. Other runs take the bitonic network.
  bool packable = true;
  for (int k = threadIdx.x; k < n2; k += kThreads) {
    const int64_t position = k < r ? grouped[first + k] : INT64_MAX;
    const int64_t source = k < r ? grouped[count + first + k] : -1;
    key[k] = position;
    value[k] = source;
    if (k < r && (position < 0 || position >= (int64_t{1} << 31) || source < 0 ||
                  source >= (int64_t{1} << 32)))
      packable = false;
  }
  packable = __syncthreads_and(packable) && r <= kPlanRankMax;
  if (packable) {
    for (int k = threadIdx.x; k < r; k += kThreads)
      packed[k] = (static_cast<uint64_t>(key[k]) << 32) | static_cast<uint64_t>(value[k]);
    if (threadIdx.x == 0 && (r & 1)) packed[r] = ~uint64_t{0};  // pads the last pair read
    __syncthreads();
    // E entries per thread (the fewest that cover the run), each ranked over all pairs
    auto rank_entries = [&]<int E>() {
      uint64_t mine[E];
      uint32_t rank[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int k = threadIdx.x + e * kThreads;
        mine[e] = k < r ? packed[k] : ~uint64_t{0};
        rank[e] = 0;
      }
      const int pairs = static_cast<int>((r + 1) >> 1);
#pragma unroll 8
      for (int j = 0; j < pairs; ++j) {
        const ulonglong2 c = reinterpret_cast<const ulonglong2*>(packed)[j];
#pragma unroll
        for (int e = 0; e < E; ++e) rank[e] += (c.x < mine[e]) + (c.y < mine[e]);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int k = threadIdx.x + e * kThreads;
        if (k < r) {
          key[rank[e]] = static_cast<int64_t>(mine[e] >> 32);
          value[rank[e]] = static_cast<int64_t>(mine[e] & 0xffffffffu);
        }
      }
    };
    if (r <= kThreads) rank_entries.template operator()<1>();
    else if (r <= 2 * kThreads) rank_entries.template operator()<2>();
    else rank_entries.template operator()<kPlanRankMax / kThreads>();
    __syncthreads();
  }
  for (int size = 2; size <= (packable ? 1 : n2); size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int k = threadIdx.x; k < n2; k += kThreads) {
        const int other = k ^ stride;
        if (other > k) {
          const bool ascending = (k & size) == 0;
          // ties (only between duplicates, which are refused) by source index
          const bool greater = key[k] > key[other] || (key[k] == key[other] && value[k] > value[other]);
          if (greater == ascending) {
            const int64_t tk = key[k], tv = value[k];
            key[k] = key[other];
            value[k] = value[other];
            key[other] = tk;
            value[other] = tv;
          }
        }
      }
      __syncthreads();
    }
  }
  const float* resident = reinterpret_cast<const float*>(entry[2]);
  const int64_t n = entry[3], out_first = entry[6];
  for (int k = threadIdx.x; k < r; k += kThreads) {
    const int64_t position = key[k];
    int64_t lo = 0, hi = n;  // resident positions below `position`
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (static_cast<int64_t>(resident[mid]) < position) lo = mid + 1;
      else hi = mid;
    }
    const bool duplicate = (lo < n && static_cast<int64_t>(resident[lo]) == position) ||
                           (k > 0 && key[k - 1] == position);
    if (duplicate) atomicOr(flag, 1);
    const int64_t row = lo + k;
    sorted_position[first + k] = position;
    sorted_source[first + k] = value[k];
    sorted_destination[first + k] = out_first + row;
    if (value[k] >= 0 && value[k] < count) recalled_rows[value[k]] = row;
  }
}

// Resident rows: block (x, slot) owns rows [x * kCompactRows, ...) of the slot's head; each
// thread finds its row's destination by binary search over the head's sorted recalled
// positions (staged in LDS), then lane groups copy the rows in batches.
template <int G>
__global__ __launch_bounds__(kThreads) void reinsert_resident_kernel(
    const int64_t* __restrict__ table, const int64_t* __restrict__ sorted_position,
    RowLayout layout, uint8_t* __restrict__ out_keys, uint8_t* __restrict__ out_values,
    float* __restrict__ out_positions) {
  __shared__ int32_t recalled[kReinsertMax];  // positions are below 2^31 (host-checked)
  __shared__ int64_t destination[kCompactRows];
  const int64_t* entry = table + static_cast<int64_t>(blockIdx.y) * LR_REINSERT_WORDS;
  const int64_t n = entry[3];
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kCompactRows;
  if (d0 >= n) return;  // uniform
  const int64_t first = entry[4], r = entry[5] < kReinsertMax ? entry[5] : kReinsertMax;
  for (int64_t k = threadIdx.x; k < r; k += kThreads)
    recalled[k] = static_cast<int32_t>(sorted_position[first + k]);
  __syncthreads();
  const int rows = static_cast<int>(n - d0 < kCompactRows ? n - d0 : kCompactRows);
  const float* positions = reinterpret_cast<const float*>(entry[2]);
  if (static_cast<int>(threadIdx.x) < rows) {
    const int64_t j = d0 + threadIdx.x;
    const float p = positions[j];
    const int64_t key = static_cast<int64_t>(p);
    int64_t lo = 0, hi = r;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (recalled[mid] < key) lo = mid + 1;
      else hi = mid;
    }
    const int64_t to = entry[6] + j + lo;
    destination[threadIdx.x] = to;
    out_positions[to] = p;
  }
  __syncthreads();
  const GroupCoord gc = group_coord(layout.lanes_log2);
  const int64_t rb = layout.row_bytes;
  const uint8_t* keys = reinterpret_cast<const uint8_t*>(entry[0]);
  const uint8_t* values = reinterpret_cast<const uint8_t*>(entry[1]);
  for (int r0 = gc.group; r0 < rows; r0 += gc.groups_per_block * kBatch) {
    RowBatch<true> b;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int row = r0 + u * gc.groups_per_block;
      const bool ok = row < rows;
      const int64_t from = ok ? d0 + row : d0;
      b.ok[u] = ok;
      b.src[u] = keys + from * rb;
      b.src2[u] = values + from * rb;
      const int64_t to = ok ? destination[row] : 0;
      b.dst[u] = out_keys + to * rb;
      b.dst2[u] = out_values + to * rb;
    }
    copy_batch<G, true, kStreamAll>(b, layout.chunks, gc.lane, gc.lanes);
  }
}

// Device grouping of a reinsertion whose identities (metadata [count, 3] i64: layer, head,
// position) are already in device memory, so that the host never walks them (the reference's
// merge_plan runs on the host per layer, src/lazy_recall/recall/planning.py:34-52). The host
// uploads the reinsert table with words [4..7] zero; then:
//   count: each valid identity adds one to its slot's word [5] (invalid ones set flag bit 2);
//   table: one workgroup turns the counts into each slot's first recalled entry [4] and first
//          output row [6] (exclusive prefixes, slot order), clears the cursor [7], copies the
//          counts to host-coherent memory for the host's layout, and flags (bit 3) a slot past
//          LR_REINSERT_MAX_PER_HEAD;
//   group: each valid identity takes the next place of its slot's run (a cursor atomic; the
//          order inside a run does not matter, the plan sorts each run by position).
__device__ __forceinline__ bool recall_identity(const int64_t* metadata, int64_t i, int64_t layers,
                                                int64_t heads, int64_t* slot, int64_t* position) {
  const int64_t layer = metadata[3 * i], head = metadata[3 * i + 1], p = metadata[3 * i + 2];
  const bool valid = layer >= 0 && layer < layers && head >= 0 && head < heads && p >= 0 &&
                     p < (int64_t{1} << 31);
  *slot = layer * heads + head;
  *position = p;
  return valid;
}

// A workgroup's identities usually fall in a few slots (a transport batch comes grouped by
// slot), so each workgroup first counts in LDS and then adds one total per slot it saw: a
// few hundred global atomics instead of one per identity on a few hundred counters.
constexpr int kGroupSlotsLds = 4096;  // slots counted in LDS (more: one global atomic each)

__global__ __launch_bounds__(kThreads) void reinsert_count_kernel(
    const int64_t* __restrict__ metadata, int64_t count, int64_t layers, int64_t heads,
    int64_t* __restrict__ table, int32_t* __restrict__ flag) {
  __shared__ uint32_t local[kGroupSlotsLds];
  const int64_t slots = layers * heads;
  const bool in_lds = slots <= kGroupSlotsLds;
  if (in_lds)
    for (int64_t k = threadIdx.x; k < slots; k += kThreads) local[k] = 0;
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < count) {
    int64_t slot, position;
    if (!recall_identity(metadata, i, layers, heads, &slot, &position)) {
      atomicOr(flag, 4);
    } else if (in_lds) {
      atomicAdd(&local[slot], 1u);
    } else {
      atomicAdd(reinterpret_cast<unsigned long long*>(table + slot * LR_REINSERT_WORDS + 5), 1ull);
    }
  }
  __syncthreads();
  if (in_lds)
    for (int64_t k = threadIdx.x; k < slots; k += kThreads)
      if (local[k] != 0)
        atomicAdd(reinterpret_cast<unsigned long long*>(table + k * LR_REINSERT_WORDS + 5),
                  static_cast<unsigned long long>(local[k]));
}

__global__ __launch_bounds__(1024) void reinsert_table_kernel(int64_t* __restrict__ table,
                                                              int64_t slots,
                                                              int64_t* __restrict__ host_counts,
                                                              int32_t* __restrict__ flag) {
  __shared__ int64_t wave_sums[16][2];
  int64_t carry_run = 0, carry_rows = 0;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int64_t base = 0; base < slots; base += 1024) {
    const int64_t slot = base + threadIdx.x;
    int64_t* entry = table + slot * LR_REINSERT_WORDS;
    const int64_t r = slot < slots ? entry[5] : 0, n = slot < slots ? entry[3] : 0;
    // inclusive wave scans of (r, n + r), then the waves' totals
    int64_t run = r, rows = n + r;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t a = __shfl_up(run, o, 64), b = __shfl_up(rows, o, 64);
      if (lane >= o) run += a, rows += b;
    }
    if (lane == 63) wave_sums[wave][0] = run, wave_sums[wave][1] = rows;
    __syncthreads();
    int64_t before_run = carry_run, before_rows = carry_rows;
    for (int w = 0; w < wave; ++w) before_run += wave_sums[w][0], before_rows += wave_sums[w][1];
    for (int w = 0; w < 16; ++w) carry_run += wave_sums[w][0], carry_rows += wave_sums[w][1];
    if (slot < slots) {
      entry[4] = before_run + run - r;
      entry[6] = before_rows + rows - (n + r);
      entry[7] = 0;
      if (host_counts != nullptr) host_counts[slot] = r;
      if (r > LR_REINSERT_MAX_PER_HEAD) atomicOr(flag, 8);
    }
    __syncthreads();  // wave_sums is rewritten by the next round
  }
}

// Grouping: each workgroup takes, per slot it saw, one range of that slot's run with a
// single global atomic (its LDS count), then places its identities inside the range by LDS
// atomics.
__global__ __launch_bounds__(kThreads) void reinsert_group_kernel(
    const int64_t* __restrict__ metadata, int64_t count, int64_t layers, int64_t heads,
    int64_t* __restrict__ table, int64_t* __restrict__ grouped) {
  __shared__ uint32_t local[kGroupSlotsLds];
  __shared__ int64_t base[kGroupSlotsLds];
  const int64_t slots = layers * heads;
  const bool in_lds = slots <= kGroupSlotsLds;
  if (in_lds)
    for (int64_t k = threadIdx.x; k < slots; k += kThreads) local[k] = 0;
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  int64_t slot = 0, position = 0;
  const bool valid = i < count && recall_identity(metadata, i, layers, heads, &slot, &position);
  uint32_t rank = 0;
  if (valid && in_lds) rank = atomicAdd(&local[slot], 1u);
  __syncthreads();
  if (in_lds)
    for (int64_t k = threadIdx.x; k < slots; k += kThreads)
      if (local[k] != 0)
        base[k] = static_cast<int64_t>(atomicAdd(
            reinterpret_cast<unsigned long long*>(table + k * LR_REINSERT_WORDS + 7),
            static_cast<unsigned long long>(local[k])));
  __syncthreads();
  if (!valid) return;
  int64_t* entry = table + slot * LR_REINSERT_WORDS;
  const int64_t at = in_lds ? base[slot] + rank
                            : static_cast<int64_t>(atomicAdd(
                                  reinterpret_cast<unsigned long long*>(entry + 7), 1ull));
  if (at >= entry[5]) return;  // cannot happen: the count saw the same identities
  grouped[entry[4] + at] = position;
  grouped[count + entry[4] + at] = i;
}

// Recalled rows: sorted entry q copies payload row sorted_source[q] (key half, value half) to
// output row sorted_destination[q], with its position.
template <int G>
__global__ __launch_bounds__(kThreads) void reinsert_recalled_kernel(
    const int64_t* __restrict__ sorted_position, const int64_t* __restrict__ sorted_source,
    const int64_t* __restrict__ sorted_destination, int64_t count, int64_t out_rows,
    const uint8_t* __restrict__ payload, RowLayout layout, uint8_t* __restrict__ out_keys,
    uint8_t* __restrict__ out_values, float* __restrict__ out_positions) {
  const GroupCoord gc = group_coord(layout.lanes_log2);
  const int64_t rb = layout.row_bytes;
  for (int64_t q0 = (static_cast<int64_t>(blockIdx.x) * gc.groups_per_block + gc.group) * kBatch;
       q0 < count; q0 += static_cast<int64_t>(gridDim.x) * gc.groups_per_block * kBatch) {
    RowBatch<true> b;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t q = q0 + u;
      const int64_t source = q < count ? sorted_source[q] : -1;
      const int64_t to = q < count ? sorted_destination[q] : -1;
      const bool ok = source >= 0 && source < count && to >= 0 && to < out_rows;
      b.ok[u] = ok;
      b.src[u] = payload + (ok ? 2 * source : 0) * rb;
      b.src2[u] = payload + (ok ? 2 * source + 1 : 0) * rb;
      b.dst[u] = out_keys + (ok ? to : 0) * rb;
      b.dst2[u] = out_values + (ok ? to : 0) * rb;
      if (ok && gc.lane == 0) out_positions[to] = static_cast<float>(sorted_position[q]);
    }
    copy_batch<G, true>(b, layout.chunks, gc.lane, gc.lanes);
  }
}

inline const uint8_t* bytes(const void* p) { return static_cast<const uint8_t*>(p); }
inline uint8_t* bytes(void* p) { return static_cast<uint8_t*>(p); }

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_compact(const void* keys, const void* values, const float* positions,
                          int64_t rows, int64_t dim, int elem_bytes, const int64_t* removed,
                          int64_t removed_count, void* out_keys, void* out_values,
                          float* out_positions, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes), "Invalid KV layout");
  LR_REQUIRE(rows >= 0 && dim > 0, "Invalid KV layout");
  LR_REQUIRE(removed_count >= 0 && removed_count <= rows, "Invalid removals");
  const int64_t rows_out = rows - removed_count;
  if (rows_out == 0) return LR_OK;
  LR_REQUIRE(keys && values && positions && out_keys && out_values && out_positions,
             "Expected contiguous CUDA tensor");
  LR_REQUIRE(removed_count == 0 || removed != nullptr, "Invalid removals");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {keys, values, out_keys, out_values});
  LR_REQUIRE(rows < (int64_t{1} << 31), "Invalid KV layout");
  const RowLayout layout = make_layout(row_bytes, g, rows_out, 8);
  // enough blocks to spread one layer over the CUs: 32..kCompactRows rows per block
  int64_t per_block = ceil_div(ceil_div(rows_out, 1024), 32) * 32;
  if (per_block > kCompactRows) per_block = kCompactRows;
  const int64_t blocks = ceil_div(rows_out, per_block);
  LR_REQUIRE(blocks < kMaxGridX, "Invalid KV layout");
  return dispatch_granule(g, [&]<int G>() {
    compact_kernel<G><<<blocks, kThreads, 0, as_stream(stream)>>>(
        bytes(keys), bytes(values), positions, removed, removed_count, rows, rows_out,
        static_cast<int>(per_block), layout,
        bytes(out_keys), bytes(out_values), out_positions);
    return check_launch("compact");
  });
}

namespace {

// Workgroups per head for the per-layer appends: one round of kAppendLayerUnroll granules per
// thread over `rows` rows of `granules_per_row` granules.
int64_t append_blocks(int64_t rows, int64_t granules_per_row) {
  int64_t bx = ceil_div(rows * granules_per_row, int64_t{kAppendThreads} * kAppendLayerUnroll);
  if (bx < 1) bx = 1;
  return bx < 65535 ? bx : 65535;
}

}  // namespace

extern "C" int lr_append(const void* keys, const void* values, const float* positions,
                         int64_t rows, const void* new_keys, const void* new_values,
                         const int32_t* cumulative, int64_t heads, int64_t added, int64_t dim,
                         int elem_bytes, int64_t logical_start, int64_t max_length,
                         void* out_keys, void* out_values, float* out_positions,
                         int32_t* out_cumulative, int32_t* out_lengths, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && rows >= 0 && dim > 0, "Invalid KV layout");
  LR_REQUIRE(heads > 0 && added > 0 && max_length >= 0, "Invalid appended shape");
  LR_REQUIRE(heads <= 65535, "Invalid appended shape");
  LR_REQUIRE(new_keys && new_values && cumulative && out_keys && out_values && out_positions &&
                 out_cumulative && out_lengths,
             "Expected contiguous CUDA tensor");
  LR_REQUIRE(rows == 0 || (keys && values && positions), "Expected contiguous CUDA tensor");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {keys, values, new_keys, new_values, out_keys, out_values});
  const int64_t covered = max_length + added;
  const int64_t bx = append_blocks(covered, row_bytes / g);
  dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>(heads));
  return dispatch_granule(g, [&]<int G>() {
    head_append_kernel<G, true><<<grid, kAppendThreads, 0, as_stream(stream)>>>(
        bytes(keys), bytes(values), positions, rows, bytes(new_keys), bytes(new_values),
        cumulative, cumulative, 1, heads, added, covered, logical_start, row_bytes,
        bytes(out_keys), bytes(out_values), out_positions, out_cumulative, out_lengths);
    return check_launch("append");
  });
}

extern "C" int lr_append_flattened_cache(const void* cache, int64_t rows, const void* states,
                                         int64_t total_heads, int64_t new_length, int64_t dim,
                                         int elem_bytes, const int32_t* head_lens,
                                         const int32_t* cu_head_lens, void* out, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && rows >= 0 && dim > 0, "head_dim mismatch");
  LR_REQUIRE(total_heads >= 0 && new_length >= 0 && total_heads <= 65535, "head count mismatch");
  if (total_heads == 0 || (rows == 0 && new_length == 0)) return LR_OK;
  LR_REQUIRE(states && head_lens && cu_head_lens && out, "states must be contiguous CUDA");
  LR_REQUIRE(rows == 0 || cache, "cache must be CUDA");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {cache, states, out});
  // Rows per head are bounded by the whole cache plus the new rows; the grid covers the mean
  // head (its threads stride over longer ones).
  const int64_t covered = rows + new_length;
  const int64_t per_head = ceil_div(rows + total_heads * new_length, total_heads);
  const int64_t bx = append_blocks(per_head, row_bytes / g);
  dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>(total_heads));
  return dispatch_granule(g, [&]<int G>() {
    head_append_kernel<G, false><<<grid, kAppendThreads, 0, as_stream(stream)>>>(
        bytes(cache), nullptr, nullptr, rows, bytes(states), nullptr, cu_head_lens, head_lens, 0,
        total_heads, new_length, covered, 0, row_bytes, bytes(out), nullptr, nullptr, nullptr,
        nullptr);
    return check_launch("append_flattened_cache");
  });
}

extern "C" int lr_compact_flattened_kv(const void* keys, const void* values, int64_t rows,
                                       int64_t dim, int elem_bytes,
                                       const int64_t* keep_indices, int64_t keep_count,
                                       void* out_keys, void* out_values, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && rows >= 0 && dim > 0, "K/V shape mismatch");
  LR_REQUIRE(keep_count >= 0, "keep_indices must be rank one");
  if (keep_count == 0) return LR_OK;
  LR_REQUIRE(keys && values && keep_indices && out_keys && out_values,
             "keep_indices must be contiguous CUDA");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {keys, values, out_keys, out_values});
  const RowLayout layout = make_layout(row_bytes, g, keep_count, 8);
  const int64_t blocks = blocks_for(layout, keep_count);
  return dispatch_granule(g, [&]<int G>() {
    gather_kernel<G, kKeep><<<blocks, kThreads, 0, as_stream(stream)>>>(
        bytes(keys), bytes(values), nullptr, rows, keep_indices, keep_count, nullptr, nullptr, 0,
        nullptr, 0, layout, bytes(out_keys), bytes(out_values), nullptr, nullptr);
    return check_launch("compact_flattened_kv");
  });
}

extern "C" int lr_merge(const void* keys, const void* values, const float* positions,
                        int64_t rows, const void* recalled, const float* recalled_positions,
                        int64_t recalled_rows, const int64_t* mapping, int64_t out_rows,
                        int64_t dim, int elem_bytes, void* out_keys, void* out_values,
                        float* out_positions, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && rows >= 0 && dim > 0, "Invalid K/V shape");
  LR_REQUIRE(recalled_rows >= 0 && out_rows >= 0, "Invalid recalled shape");
  if (out_rows == 0) return LR_OK;
  LR_REQUIRE(mapping && out_keys && out_values && out_positions, "Expected contiguous CUDA tensor");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {keys, values, recalled, out_keys, out_values});
  // one batch per lane group: each batch waits for its mapping entries, so more, shorter lane
  // groups keep more rows in flight (measured faster than two or four batches per group)
  const RowLayout layout = make_layout(row_bytes, g, out_rows, kBatch);
  const int64_t blocks = blocks_for(layout, out_rows);
  return dispatch_granule(g, [&]<int G>() {
    gather_kernel<G, kMerge><<<blocks, kThreads, 0, as_stream(stream)>>>(
        bytes(keys), bytes(values), positions, rows, mapping, out_rows, bytes(recalled),
        recalled_positions, recalled_rows, nullptr, 0, layout, bytes(out_keys),
        bytes(out_values), out_positions, nullptr);
    return check_launch("merge");
  });
}

extern "C" int lr_pack(const void* keys, const void* values, const float* positions,
                       int64_t rows, const int64_t* indices, const int64_t* heads, int64_t count,
                       int64_t dim, int elem_bytes, int64_t layer, void* payload,
                       int64_t* metadata, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && rows >= 0 && dim > 0, "Invalid K/V shape");
  LR_REQUIRE(count >= 0, "Invalid gather indices");
  if (count == 0) return LR_OK;
  LR_REQUIRE(keys && values && positions && indices && heads && payload && metadata,
             "Expected contiguous CUDA tensor");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {keys, values, payload});
  const RowLayout layout = make_layout(row_bytes, g, count, 8);
  const int64_t blocks = blocks_for(layout, count);
  return dispatch_granule(g, [&]<int G>() {
    gather_kernel<G, kPack><<<blocks, kThreads, 0, as_stream(stream)>>>(
        bytes(keys), bytes(values), positions, rows, indices, count, nullptr, nullptr, 0, heads,
        layer, layout, bytes(payload), nullptr, nullptr, metadata);
    return check_launch("pack");
  });
}

namespace {

// The checks and launch shape shared by both batch_append entry points; `launch` gets the
// granule, the row layout and the grid.
template <typename Launch>
int batch_append_launch(int64_t segments, const void* new_keys, const void* new_values,
                        int64_t dim, int elem_bytes, int64_t max_rows, void* out_keys,
                        void* out_values, float* out_positions, Launch&& launch) {
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && dim > 0, "Only batched one-token append is supported");
  LR_REQUIRE(segments > 0 && segments <= 65535, "Request metadata mismatch");
  LR_REQUIRE(max_rows >= 1, "Invalid head length");
  LR_REQUIRE(new_keys && new_values && out_keys && out_values && out_positions,
             "Contiguous CUDA states required");
  const int64_t row_bytes = dim * elem_bytes;
  // Descriptor pointers are required to share the alignment of the row size (a whole
  // number of rows from a 16-byte aligned allocation), so only the row size and the
  // pointers seen here bound the granule.
  const int g = granule_for(row_bytes, {new_keys, new_values, out_keys, out_values});
  // workgroups per segment: one pass of kAppendUnroll granules per thread over the longest
  // segment's old rows
  int64_t bx = ceil_div(ceil_div(max_rows * row_bytes, g), int64_t{kThreads} * kAppendUnroll);
  if (bx < 1) bx = 1;
  const dim3 grid(static_cast<unsigned>(bx < 65535 ? bx : 65535), static_cast<unsigned>(segments));
  return dispatch_granule(g, [&]<int G>() { return launch.template operator()<G>(row_bytes, grid); });
}

}  // namespace

extern "C" int lr_batch_append(const int64_t* descriptors, int64_t segments,
                               const void* new_keys, const void* new_values, int64_t dim,
                               int elem_bytes, int64_t max_rows, void* out_keys,
                               void* out_values, float* out_positions, void* stream) {
  clear_error();
  LR_REQUIRE(descriptors != nullptr, "Contiguous CUDA states required");
  return batch_append_launch(
      segments, new_keys, new_values, dim, elem_bytes, max_rows, out_keys, out_values,
      out_positions, [&]<int G>(int64_t row_bytes, dim3 grid) {
        batch_append_kernel<G><<<grid, kThreads, 0, as_stream(stream)>>>(
            descriptors, bytes(new_keys), bytes(new_values), max_rows, row_bytes,
            bytes(out_keys), bytes(out_values), out_positions);
        return check_launch("batch_append");
      });
}

extern "C" int lr_batch_append_host(const int64_t* host_descriptors, int64_t segments,
                                    const void* new_keys, const void* new_values, int64_t dim,
                                    int elem_bytes, int64_t max_rows, void* out_keys,
                                    void* out_values, float* out_positions, void* stream) {
  clear_error();
  LR_REQUIRE(host_descriptors != nullptr, "Request metadata mismatch");
  LR_REQUIRE(segments <= kInlineSegments, "Too many segments for descriptors in the launch");
  InlineDescriptors words{};
  if (segments > 0)
    std::memcpy(words.words, host_descriptors, static_cast<size_t>(segments) * 7 * sizeof(int64_t));
  return batch_append_launch(
      segments, new_keys, new_values, dim, elem_bytes, max_rows, out_keys, out_values,
      out_positions, [&]<int G>(int64_t row_bytes, dim3 grid) {
        batch_append_inline_kernel<G><<<grid, kThreads, 0, as_stream(stream)>>>(
            words, bytes(new_keys), bytes(new_values), max_rows, row_bytes, bytes(out_keys),
            bytes(out_values), out_positions);
        return check_launch("batch_append");
      });
}

extern "C" int lr_compact_heads_layout(const int64_t* head_table, int64_t heads,
                                       const int64_t* quotas, const int64_t* offsets,
                                       const int64_t* removed_positions, int64_t dim,
                                       int elem_bytes, int64_t max_length, int64_t total_out_rows,
                                       void* out_keys, void* out_values, float* out_positions,
                                       int64_t heads_per_layer, int32_t* head_lens,
                                       int32_t* cumulative, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && dim > 0, "Invalid KV layout");
  LR_REQUIRE(heads > 0 && heads <= 65535 && max_length >= 0, "Invalid head table");
  const bool layout_out = head_lens != nullptr;
  LR_REQUIRE(!layout_out || (cumulative != nullptr && heads_per_layer > 0 &&
                             heads % heads_per_layer == 0),
             "Invalid head table");
  if (!layout_out && (total_out_rows == 0 || max_length == 0)) return LR_OK;
  LR_REQUIRE(head_table && quotas && offsets && removed_positions &&
                 (total_out_rows == 0 || (out_keys && out_values && out_positions)),
             "Expected contiguous CUDA tensor");
  LR_REQUIRE(total_out_rows < (int64_t{1} << 31) || !layout_out,
             "Cumulative lengths exceed int32");
  const int64_t row_bytes = dim * elem_bytes;
  // Head rows are whole rows of 256-byte aligned allocations; the outputs bound the granule.
  const int g = total_out_rows > 0 ? granule_for(row_bytes, {out_keys, out_values})
                                   : granule_for(row_bytes, {});
  LR_REQUIRE(max_length < (int64_t{1} << 31), "Invalid head table");
  const RowLayout layout = make_layout(row_bytes, g, total_out_rows > 0 ? total_out_rows : 1, 8);
  int64_t bx = ceil_div(max_length, kCompactRows);
  if (bx < 1) bx = 1;  // block 0 of every head writes the layout
  LR_REQUIRE(bx <= 65535, "Invalid head table");
  dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>(heads));
  return dispatch_granule(g, [&]<int G>() {
    compact_heads_kernel<G><<<grid, kThreads, 0, as_stream(stream)>>>(
        head_table, quotas, offsets, removed_positions, layout, bytes(out_keys),
        bytes(out_values), out_positions, layout_out ? heads_per_layer : 1, head_lens,
        cumulative);
    return check_launch("compact_heads");
  });
}

extern "C" int lr_compact_heads(const int64_t* head_table, int64_t heads, const int64_t* quotas,
                                const int64_t* offsets, const int64_t* removed_positions,
                                int64_t dim, int elem_bytes, int64_t max_length,
                                int64_t total_out_rows, void* out_keys, void* out_values,
                                float* out_positions, void* stream) {
  return lr_compact_heads_layout(head_table, heads, quotas, offsets, removed_positions, dim,
                                 elem_bytes, max_length, total_out_rows, out_keys, out_values,
                                 out_positions, 0, nullptr, nullptr, stream);
}

extern "C" int lr_reinsert_plan_layout(const int64_t* table, int64_t slots,
                                       const int64_t* grouped, int64_t count, int64_t* workspace,
                                       int64_t* recalled_rows, int32_t* flag,
                                       int64_t heads_per_layer, int32_t* head_lens,
                                       int32_t* cumulative, void* stream) {
  clear_error();
  LR_REQUIRE(slots > 0 && slots <= (int64_t{1} << 31) - 1 && count >= 0 &&
                 count < (int64_t{1} << 40),
             "Invalid reinsert layout");
  LR_REQUIRE(table && flag && (count == 0 || (grouped && workspace && recalled_rows)),
             "Expected contiguous CUDA tensor");
  const bool layout_out = head_lens != nullptr;
  LR_REQUIRE(!layout_out || (cumulative != nullptr && heads_per_layer > 0 &&
                             slots % heads_per_layer == 0),
             "Invalid reinsert layout");
  if (count == 0 && !layout_out) return LR_OK;
  reinsert_plan_kernel<<<static_cast<unsigned>(slots), kThreads, 0, as_stream(stream)>>>(
      table, grouped, workspace, workspace + count, workspace + 2 * count, recalled_rows, count,
      flag, layout_out ? heads_per_layer : 1, head_lens, cumulative);
  return check_launch("reinsert_plan");
}

extern "C" int lr_reinsert_plan(const int64_t* table, int64_t slots, const int64_t* grouped,
                                int64_t count, int64_t* workspace, int64_t* recalled_rows,
                                int32_t* flag, void* stream) {
  return lr_reinsert_plan_layout(table, slots, grouped, count, workspace, recalled_rows, flag, 0,
                                 nullptr, nullptr, stream);
}

extern "C" int lr_reinsert_group(int64_t* table, int64_t slots, int64_t heads,
                                 const int64_t* metadata, int64_t count, int64_t* grouped,
                                 int64_t* host_counts, int32_t* flag, void* stream) {
  clear_error();
  LR_REQUIRE(slots > 0 && slots <= (int64_t{1} << 31) - 1 && heads > 0 && slots % heads == 0 &&
                 count >= 0 && count < (int64_t{1} << 40),
             "Invalid reinsert layout");
  LR_REQUIRE(table && flag && (count == 0 || (metadata && grouped)),
             "Expected contiguous CUDA tensor");
  const hipStream_t s = as_stream(stream);
  const unsigned blocks = static_cast<unsigned>(ceil_div(count, int64_t{kThreads}));
  if (count > 0) {
    reinsert_count_kernel<<<blocks, kThreads, 0, s>>>(metadata, count, slots / heads, heads,
                                                      table, flag);
    if (int rc = check_launch("reinsert_count")) return rc;
  }
  reinsert_table_kernel<<<1, 1024, 0, s>>>(table, slots, host_counts, flag);
  if (int rc = check_launch("reinsert_table")) return rc;
  if (count > 0) {
    reinsert_group_kernel<<<blocks, kThreads, 0, s>>>(metadata, count, slots / heads, heads, table,
                                                      grouped);
    return check_launch("reinsert_group");
  }
  return LR_OK;
}

extern "C" int lr_reinsert_resident(const int64_t* table, int64_t slots, const int64_t* workspace,
                                    int64_t count, int64_t max_length, int64_t dim,
                                    int elem_bytes, int64_t out_rows, void* out_keys,
                                    void* out_values, float* out_positions, void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && dim > 0, "Invalid KV layout");
  LR_REQUIRE(slots > 0 && slots <= 65535 && max_length >= 0 && count >= 0, "Invalid reinsert layout");
  if (out_rows == 0 || max_length == 0) return LR_OK;
  LR_REQUIRE(table && out_keys && out_values && out_positions && (count == 0 || workspace),
             "Expected contiguous CUDA tensor");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {out_keys, out_values});
  LR_REQUIRE(max_length < (int64_t{1} << 31), "Invalid reinsert layout");
  const RowLayout layout = make_layout(row_bytes, g, out_rows, 8);
  const int64_t bx = ceil_div(max_length, kCompactRows);
  LR_REQUIRE(bx <= 65535, "Invalid reinsert layout");
  dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>(slots));
  return dispatch_granule(g, [&]<int G>() {
    reinsert_resident_kernel<G><<<grid, kThreads, 0, as_stream(stream)>>>(
        table, workspace, layout, bytes(out_keys), bytes(out_values), out_positions);
    return check_launch("reinsert_resident");
  });
}

extern "C" int lr_reinsert_recalled(const int64_t* workspace, int64_t count, const void* payload,
                                    int64_t dim, int elem_bytes, int64_t out_rows,
                                    void* out_keys, void* out_values, float* out_positions,
                                    void* stream) {
  clear_error();
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && dim > 0 && count >= 0 && out_rows >= 0,
             "Invalid KV layout");
  if (count == 0 || out_rows == 0) return LR_OK;
  LR_REQUIRE(workspace && payload && out_keys && out_values && out_positions,
             "Expected contiguous CUDA tensor");
  const int64_t row_bytes = dim * elem_bytes;
  const int g = granule_for(row_bytes, {payload, out_keys, out_values});
  const RowLayout layout = make_layout(row_bytes, g, count, kBatch);
  const int64_t groups_per_block = kThreads >> layout.lanes_log2;
  int64_t blocks = ceil_div(ceil_div(count, kBatch), groups_per_block);
  if (blocks > kMaxGridX) blocks = kMaxGridX;
  return dispatch_granule(g, [&]<int G>() {
    reinsert_recalled_kernel<G><<<static_cast<unsigned>(blocks), kThreads, 0, as_stream(stream)>>>(
        workspace, workspace + count, workspace + 2 * count, count, out_rows, bytes(payload),
        layout, bytes(out_keys), bytes(out_values), out_positions);
    return check_launch("reinsert_recalled");
  });
}

namespace {

// The checks and launch shape shared by both append_layers entry points; `launch` gets the
// granule, the row layout and the grid.
template <typename Launch>
int append_layers_launch(int64_t layers, int64_t heads, int64_t added, int64_t dim,
                         int elem_bytes, int64_t max_length, void* out_keys, void* out_values,
                         float* out_positions, int32_t* out_cumulative, int32_t* out_lengths,
                         Launch&& launch) {
  LR_REQUIRE(valid_elem_bytes(elem_bytes) && dim > 0, "Invalid KV layout");
  LR_REQUIRE(layers > 0 && layers <= 65535 && heads > 0 && heads <= 65535 && added > 0 &&
                 max_length >= 0,
             "Invalid appended shape");
  LR_REQUIRE(out_keys && out_values && out_positions && out_cumulative && out_lengths,
             "Expected contiguous CUDA tensor");
  const int64_t row_bytes = dim * elem_bytes;
  // every layer's rows are whole rows of its (16-byte aligned) allocation; the outputs bound
  // the granule
  const int g = granule_for(row_bytes, {out_keys, out_values});
  const int64_t covered = max_length + added;
  const RowLayout layout = make_layout(row_bytes, g, covered * heads * layers, 8);
  int64_t bx = ceil_div(ceil_div(covered, layout.rows_per_group), kThreads >> layout.lanes_log2);
  if (bx < 1) bx = 1;
  const dim3 grid(static_cast<unsigned>(bx < 65535 ? bx : 65535), static_cast<unsigned>(heads),
                  static_cast<unsigned>(layers));
  return dispatch_granule(
      g, [&]<int G>() { return launch.template operator()<G>(covered, layout, grid); });
}

}  // namespace

extern "C" int lr_append_layers(const int64_t* table, int64_t layers, int64_t heads,
                                int64_t added, int64_t dim, int elem_bytes, int64_t max_length,
                                void* out_keys, void* out_values, float* out_positions,
                                int32_t* out_cumulative, int32_t* out_lengths, void* stream) {
  clear_error();
  LR_REQUIRE(table != nullptr, "Expected contiguous CUDA tensor");
  return append_layers_launch(
      layers, heads, added, dim, elem_bytes, max_length, out_keys, out_values, out_positions,
      out_cumulative, out_lengths,
      [&]<int G>(int64_t covered, const RowLayout& layout, dim3 grid) {
        append_layers_kernel<G><<<grid, kThreads, 0, as_stream(stream)>>>(
            table, heads, added, covered, layout, bytes(out_keys), bytes(out_values),
            out_positions, out_cumulative, out_lengths);
        return check_launch("append_layers");
      });
}

extern "C" int lr_append_layers_host(const int64_t* host_table, int64_t layers, int64_t heads,
                                     int64_t added, int64_t dim, int elem_bytes,
                                     int64_t max_length, void* out_keys, void* out_values,
                                     float* out_positions, int32_t* out_cumulative,
                                     int32_t* out_lengths, void* stream) {
  clear_error();
  LR_REQUIRE(host_table != nullptr, "Invalid appended shape");
  LR_REQUIRE(layers <= kInlineLayers, "Too many layers for a table in the launch");
  InlineAppendTable words{};
  for (int64_t l = 0; l < layers; ++l)
    for (int i = 0; i < kAppendRowWords; ++i)
      words.words[l * kAppendRowWords + i] = host_table[l * LR_APPEND_WORDS + i];
  return append_layers_launch(
      layers, heads, added, dim, elem_bytes, max_length, out_keys, out_values, out_positions,
      out_cumulative, out_lengths,
      [&]<int G>(int64_t covered, const RowLayout& layout, dim3 grid) {
        append_layers_inline_kernel<G><<<grid, kThreads, 0, as_stream(stream)>>>(
            words, heads, added, covered, layout, bytes(out_keys), bytes(out_values),
            out_positions, out_cumulative, out_lengths);
        return check_launch("append_layers");
      });
}
