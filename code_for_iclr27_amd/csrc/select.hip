// Device-side allocation-preserving selection (src/lazy_recall/selection.py:52-88):
//   1. global bottom-`count` of the raw scores (ties: lower index first) -> per-segment quotas;
//   2. per segment, bottom-quota of the pooled scores (ties: lower index first);
//   3. the refined picks of each segment fill that segment's slots of the global order
//      (transplant, selection.py:42-49).
// The reference runs a global torch.topk, a host searchsorted/bincount, one torch.topk launch
// plus a device->host copy per segment and a numpy transplant. Here everything stays on the
// device: a multi-block radix select finds the global threshold, one workgroup per segment
// does its counting, ordered compaction, radix select and stable radix sorts in LDS, and a
// final stable sort orders the slots. Scores are compared through an order-preserving uint32
// key (-0.0 and +0.0 are one key; NaN sorts last).
#include <utility>

#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kSegThreads = 256;   // per-segment workgroups

__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;  // -0.0 == +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

__device__ __forceinline__ uint32_t atomic_load_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct SelectState {
  uint32_t prefix, mask, remaining, less, done, pad[3];
};

// ---------------------------------------------------------------------------------------
// Workgroup primitives. BLOCK threads, BLOCK / 64 waves.

// Exclusive prefix of per-thread counts in thread order; returns the thread's offset and
// writes the block total to *total (LDS). One call = two barriers.
template <int BLOCK>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t value, uint32_t* wave_sums,
                                                         uint32_t* total) {
  constexpr int W = BLOCK / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t inclusive = value;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t n = __shfl_up(inclusive, o, 64);
    if (lane >= o) inclusive += n;
  }
  if (lane == 63) wave_sums[wave] = inclusive;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const uint32_t v = wave_sums[w];
    if (w < wave) before += v;
    all += v;
  }
  __syncthreads();
  if (threadIdx.x == 0) *total = all;
  return before + inclusive - value;
}

template <int BLOCK>
struct SortLds {
  uint32_t hist[256];
  uint32_t base[256];
  uint32_t wave_counts[BLOCK / 64][256];
  uint32_t wave_sums[BLOCK / 64];
  uint32_t scalars[8];
};

// Stable rank of each lane's 8-bit digit among earlier lanes of the wave with the same digit;
// `count` receives how many active lanes share it; the lowest such lane is the leader.
__device__ __forceinline__ void wave_match_digit(uint32_t digit, bool active, uint32_t* rank,
                                                 uint32_t* count, bool* leader) {
  uint64_t peers = __ballot(active);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const uint64_t m = __ballot(active && ((digit >> b) & 1u));
    peers &= ((digit >> b) & 1u) ? m : ~m;
  }
  *rank = __popcll(peers & lanemask_lt());
  *count = __popcll(peers);
  *leader = active && *rank == 0;
}

// Stable LSD radix sort of n (key, value) pairs by key, 8 bits per pass, ping-ponging between
// (keys, values) and (tmp_keys, tmp_values). Result ends in (keys, values). All BLOCK threads
// of the workgroup must call it.
template <int BLOCK>
__device__ void block_radix_sort(uint32_t* keys, uint32_t* values, uint32_t* tmp_keys,
                                 uint32_t* tmp_values, uint32_t n, SortLds<BLOCK>& lds) {
  constexpr int W = BLOCK / 64;
  const int wave = threadIdx.x >> 6;
  uint32_t* src_k = keys;
  uint32_t* src_v = values;
  uint32_t* dst_k = tmp_keys;
  uint32_t* dst_v = tmp_values;
  for (int shift = 0; shift < 32; shift += 8) {
    for (int i = threadIdx.x; i < 256; i += BLOCK) lds.hist[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += BLOCK) atomicAdd(&lds.hist[(src_k[i] >> shift) & 255u], 1u);
    __syncthreads();
    if (threadIdx.x < 64) {  // exclusive scan of 256 bins by one wave (4 bins per lane)
      const int lane = threadIdx.x;
      uint32_t c[4], s = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = lds.hist[4 * lane + j];
        s += c[j];
      }
      uint32_t inc = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
      }
      uint32_t run = inc - s;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lds.base[4 * lane + j] = run;
        run += c[j];
      }
      // a pass where every key has the same digit moves nothing: flag it
      bool single = false;
#pragma unroll
      for (int j = 0; j < 4; ++j) single |= c[j] == n;
      lds.scalars[0] = __any(single) ? 1u : 0u;
    }
    for (int i = threadIdx.x; i < W * 256; i += BLOCK) (&lds.wave_counts[0][0])[i] = 0;
    __syncthreads();
    if (lds.scalars[0]) {
      __syncthreads();
      continue;  // identity permutation: keep the buffers as they are
    }
    for (uint32_t chunk = 0; chunk < n; chunk += BLOCK) {
      const uint32_t i = chunk + threadIdx.x;
      const bool active = i < n;
      const uint32_t key = active ? src_k[i] : 0u;
      const uint32_t value = active ? src_v[i] : 0u;
      const uint32_t digit = (key >> shift) & 255u;
      uint32_t rank, count;
      bool leader;
      wave_match_digit(digit, active, &rank, &count, &leader);
      if (leader) lds.wave_counts[wave][digit] = count;
      __syncthreads();
      if (active) {
        uint32_t offset = lds.base[digit] + rank;
        for (int w = 0; w < wave; ++w) offset += lds.wave_counts[w][digit];
        dst_k[offset] = key;
        dst_v[offset] = value;
      }
      __syncthreads();
      for (int d = threadIdx.x; d < 256; d += BLOCK) {
        uint32_t add = 0;
        for (int w = 0; w < W; ++w) {
          add += lds.wave_counts[w][d];
          lds.wave_counts[w][d] = 0;
        }
        lds.base[d] += add;
      }
      __syncthreads();
    }
    uint32_t* t = src_k; src_k = dst_k; dst_k = t;
    t = src_v; src_v = dst_v; dst_v = t;
    __threadfence_block();
    __syncthreads();
  }
  if (src_k != keys) {  // an odd number of moving passes left the result in tmp
    for (uint32_t i = threadIdx.x; i < n; i += BLOCK) {
      keys[i] = src_k[i];
      values[i] = src_v[i];
    }
    __syncthreads();
  }
}

// k-th smallest key (1-based rank `k`) among the n keys produced by key_at(i). Returns
// threshold key, count of keys strictly below it, and how many threshold-equal keys to take.
template <int BLOCK, typename KeyAt>
__device__ void block_radix_select(uint32_t n, uint32_t k, KeyAt key_at, SortLds<BLOCK>& lds,
                                   uint32_t* threshold, uint32_t* less, uint32_t* take_equal) {
  uint32_t prefix = 0, mask = 0, remaining = k, below = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += BLOCK) lds.hist[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += BLOCK) {
      const uint32_t key = key_at(i);
      if ((key & mask) == prefix) atomicAdd(&lds.hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      uint32_t c[4], s = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = lds.hist[4 * lane + j];
        s += c[j];
      }
      uint32_t inc = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
      }
      uint32_t run = inc - s;
      // the lane whose 4 bins contain the crossing of `remaining` finishes the pass
      if (run < remaining && inc >= remaining) {
        uint32_t digit = 4 * lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (run + c[j] >= remaining) {
            digit = 4 * lane + j;
            break;
          }
          run += c[j];
        }
        lds.scalars[0] = digit;
        lds.scalars[1] = run;
      }
    }
    __syncthreads();
    const uint32_t digit = lds.scalars[0], skipped = lds.scalars[1];
    prefix |= digit << shift;
    mask |= 255u << shift;
    remaining -= skipped;
    below += skipped;
    __syncthreads();
  }
  *threshold = prefix;
  *less = below;
  *take_equal = remaining;
}

// Ordered (stable) compaction helper: returns the rank of this thread's element among the
// selected elements of its chunk plus everything selected before the chunk (*running, LDS).
template <int BLOCK>
__device__ __forceinline__ uint32_t block_ordered_rank(bool selected, SortLds<BLOCK>& lds,
                                                       uint32_t* running) {
  const uint32_t offset = block_exclusive_scan<BLOCK>(selected ? 1u : 0u, lds.wave_sums, &lds.scalars[2]);
  const uint32_t base = *running;
  __syncthreads();
  if (threadIdx.x == 0) *running = base + lds.scalars[2];
  __syncthreads();
  return base + offset;
}

// ---------------------------------------------------------------------------------------
// Global threshold: 3 passes (11 + 11 + 10 bits) over all raw scores. Each pass is a
// per-block histogram of the keys that match the prefix found so far, written without atomics,
// then one workgroup sums the block histograms and extends the prefix by the digit where the
// running count reaches the remaining rank.
constexpr int kHistBlocks = 128;

__global__ __launch_bounds__(256) void select_init_kernel(SelectState* state, uint32_t count) {
  if (threadIdx.x == 0) {
    state->prefix = 0;
    state->mask = 0;
    state->remaining = count;
    state->less = 0;
    state->done = 0;
  }
}

template <int BITS, int SHIFT>
__global__ __launch_bounds__(256) void select_block_histogram_kernel(
    const float* __restrict__ scores, int64_t n, int64_t chunk,
    const SelectState* __restrict__ state, uint32_t* __restrict__ block_hist) {
  constexpr int BINS = 1 << BITS;
  __shared__ uint32_t local[BINS];
  for (int i = threadIdx.x; i < BINS; i += 256) local[i] = 0;
  __syncthreads();
  const uint32_t prefix = state->prefix, mask = state->mask;
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t end = begin + chunk < n ? begin + chunk : n;
  // chunk is a multiple of 1024 and scores is 16-byte aligned: float4 loads, 4 in flight
  for (int64_t base = begin + threadIdx.x * 4; base < end; base += 256 * 4 * 4) {
    float4 q[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t at = base + u * 256 * 4;
      if (at + 3 < end) {
        q[u] = *reinterpret_cast<const float4*>(scores + at);
      } else {
        q[u].x = at < end ? scores[at] : NAN;
        q[u].y = at + 1 < end ? scores[at + 1] : NAN;
        q[u].z = at + 2 < end ? scores[at + 2] : NAN;
        q[u].w = at + 3 < end ? scores[at + 3] : NAN;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t at = base + u * 256 * 4;
      const float v[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (at + j < end) {
          const uint32_t key = float_key(v[j]);
          if ((key & mask) == prefix) atomicAdd(&local[(key >> SHIFT) & (BINS - 1)], 1u);
        }
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < BINS; i += 256) block_hist[static_cast<int64_t>(blockIdx.x) * BINS + i] = local[i];
}

template <int BITS, int SHIFT>
__global__ __launch_bounds__(1024) void select_reduce_kernel(const uint32_t* __restrict__ block_hist,
                                                             int blocks, SelectState* state) {
  constexpr int BINS = 1 << BITS;
  constexpr int PER = BINS / 1024 > 0 ? BINS / 1024 : 1;
  __shared__ uint32_t wave_sums[16];
  __shared__ uint32_t total;
  uint32_t c[PER], sum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int bin = threadIdx.x * PER + j;
    uint32_t acc = 0;
    if (bin < BINS)
      for (int b = 0; b < blocks; ++b) acc += block_hist[static_cast<int64_t>(b) * BINS + bin];
    c[j] = acc;
    sum += acc;
  }
  const uint32_t before = block_exclusive_scan<1024>(sum, wave_sums, &total);
  const uint32_t remaining = state->remaining;
  __syncthreads();
  if (before < remaining && before + sum >= remaining) {
    uint32_t run = before;
    int digit = threadIdx.x * PER + PER - 1;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (run + c[j] >= remaining) {
        digit = threadIdx.x * PER + j;
        break;
      }
      run += c[j];
    }
    state->prefix |= static_cast<uint32_t>(digit) << SHIFT;
    state->mask |= static_cast<uint32_t>(BINS - 1) << SHIFT;
    state->less += run;
    state->remaining = remaining - run;
  }
}

// Per segment: how many raw keys are below / equal to the global threshold.
__global__ __launch_bounds__(kSegThreads) void segment_count_kernel(
    const float* __restrict__ scores, const int64_t* __restrict__ ends,
    const SelectState* __restrict__ state, uint32_t* __restrict__ seg_less,
    uint32_t* __restrict__ seg_equal) {
  __shared__ uint32_t sums[2][kSegThreads / 64];
  const int64_t s = blockIdx.x;
  const int64_t begin = s == 0 ? 0 : ends[s - 1], end = ends[s];
  const uint32_t threshold = state->prefix;
  uint32_t less = 0, equal = 0;
  for (int64_t i = begin + threadIdx.x; i < end; i += kSegThreads) {
    const uint32_t key = float_key(scores[i]);
    less += key < threshold;
    equal += key == threshold;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    less += __shfl_xor(less, o, 64);
    equal += __shfl_xor(equal, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    sums[0][threadIdx.x >> 6] = less;
    sums[1][threadIdx.x >> 6] = equal;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = 0, b = 0;
    for (int w = 0; w < kSegThreads / 64; ++w) {
      a += sums[0][w];
      b += sums[1][w];
    }
    seg_less[s] = a;
    seg_equal[s] = b;
  }
}

// One workgroup: per-segment quotas (threshold-equal keys are granted in index order, i.e.
// segment order) and their exclusive prefix.
__global__ __launch_bounds__(1024) void segment_plan_kernel(
    const uint32_t* __restrict__ seg_less, const uint32_t* __restrict__ seg_equal,
    const SelectState* __restrict__ state, int64_t segments, uint32_t* __restrict__ take_equal,
    int64_t* __restrict__ quotas, int64_t* __restrict__ offsets) {
  __shared__ uint32_t wave_sums[16];
  __shared__ uint32_t totals[2];
  __shared__ uint32_t carry[2];
  if (threadIdx.x == 0) carry[0] = carry[1] = 0;
  __syncthreads();
  const uint32_t need = state->remaining;
  for (int64_t base = 0; base < segments; base += 1024) {
    const int64_t s = base + threadIdx.x;
    const uint32_t eq = s < segments ? seg_equal[s] : 0;
    const uint32_t eq_before = carry[0] + block_exclusive_scan<1024>(eq, wave_sums, &totals[0]);
    uint32_t take = 0;
    if (need > eq_before) take = need - eq_before < eq ? need - eq_before : eq;
    const uint32_t quota = s < segments ? seg_less[s] + take : 0;
    const uint32_t quota_before = carry[1] + block_exclusive_scan<1024>(quota, wave_sums, &totals[1]);
    if (s < segments) {
      take_equal[s] = take;
      quotas[s] = quota;
      offsets[s] = quota_before;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      carry[0] += totals[0];
      carry[1] += totals[1];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) offsets[segments] = carry[1];
}

// One workgroup per segment with a non-zero quota:
//   raw picks (index order) -> raw run sorted by raw key     (slot order inside the segment)
//   pooled bottom-quota     -> removal positions (ascending) and refined picks sorted by
//                              pooled key                    (what fills the segment's slots)
__global__ __launch_bounds__(kSegThreads) void segment_select_kernel(
    const float* __restrict__ raw, const float* __restrict__ pooled,
    const int64_t* __restrict__ ends, const int64_t* __restrict__ position_starts,
    const SelectState* __restrict__ state, const uint32_t* __restrict__ take_equal,
    const int64_t* __restrict__ quotas, const int64_t* __restrict__ offsets,
    uint8_t* __restrict__ raw_flags, uint32_t* __restrict__ run_keys,
    uint32_t* __restrict__ run_slots, uint32_t* __restrict__ refined_keys,
    uint32_t* __restrict__ refined_local, uint32_t* __restrict__ tmp_keys,
    uint32_t* __restrict__ tmp_values, int64_t* __restrict__ removed_positions,
    int64_t* __restrict__ changed, uint32_t* __restrict__ segment_of) {
  __shared__ SortLds<kSegThreads> lds;
  __shared__ uint32_t running[2];
  const int64_t s = blockIdx.x;
  const uint32_t quota = static_cast<uint32_t>(quotas[s]);
  if (quota == 0) {
    if (threadIdx.x == 0) changed[s] = 0;
    return;
  }
  const int64_t begin = s == 0 ? 0 : ends[s - 1], end = ends[s];
  const uint32_t n = static_cast<uint32_t>(end - begin);
  const int64_t offset = offsets[s];
  const uint32_t threshold = state->prefix, take = take_equal[s];
  const int64_t position_start = position_starts[s];
  if (threadIdx.x == 0) running[0] = running[1] = 0;
  __syncthreads();
  // raw picks in index order
  for (uint32_t chunk = 0; chunk < n; chunk += kSegThreads) {
    const uint32_t i = chunk + threadIdx.x;
    const bool active = i < n;
    const uint32_t key = active ? float_key(raw[begin + i]) : 0xffffffffu;
    const bool equal = active && key == threshold;
    const uint32_t equal_rank = block_ordered_rank<kSegThreads>(equal, lds, &running[1]);
    const bool picked = active && (key < threshold || (equal && equal_rank < take));
    const uint32_t rank = block_ordered_rank<kSegThreads>(picked, lds, &running[0]);
    if (active) raw_flags[begin + i] = picked;
    if (picked) {
      run_keys[offset + rank] = key;
      run_slots[offset + rank] = 0u;
    }
  }
  __threadfence_block();
  __syncthreads();
  block_radix_sort<kSegThreads>(run_keys + offset, run_slots + offset, tmp_keys + offset,
                                tmp_values + offset, quota, lds);
  // Slot payload for the global sort: position in the concatenated runs, i.e. segment offset
  // plus the rank in this segment's (key, index) order.
  for (uint32_t i = threadIdx.x; i < quota; i += kSegThreads) {
    run_slots[offset + i] = static_cast<uint32_t>(offset + i);
    segment_of[offset + i] = static_cast<uint32_t>(s);
  }
  __syncthreads();
  // refined picks: bottom-quota of the pooled scores
  uint32_t pthreshold, pless, ptake;
  block_radix_select<kSegThreads>(
      n, quota, [&](uint32_t i) { return float_key(pooled[begin + i]); }, lds, &pthreshold,
      &pless, &ptake);
  if (threadIdx.x == 0) running[0] = running[1] = 0;
  __syncthreads();
  uint32_t moved = 0;
  for (uint32_t chunk = 0; chunk < n; chunk += kSegThreads) {
    const uint32_t i = chunk + threadIdx.x;
    const bool active = i < n;
    const uint32_t key = active ? float_key(pooled[begin + i]) : 0xffffffffu;
    const bool equal = active && key == pthreshold;
    const uint32_t equal_rank = block_ordered_rank<kSegThreads>(equal, lds, &running[1]);
    const bool picked = active && (key < pthreshold || (equal && equal_rank < ptake));
    const uint32_t rank = block_ordered_rank<kSegThreads>(picked, lds, &running[0]);
    if (picked) {
      refined_keys[offset + rank] = key;
      refined_local[offset + rank] = i;
      removed_positions[offset + rank] = position_start + i;
      moved += raw_flags[begin + i] ? 0u : 1u;
    }
  }
  __threadfence_block();
  __syncthreads();
  const uint32_t moved_total =
      block_exclusive_scan<kSegThreads>(moved, lds.wave_sums, &lds.scalars[3]);
  (void)moved_total;
  __syncthreads();
  if (threadIdx.x == 0) changed[s] = lds.scalars[3];
  block_radix_sort<kSegThreads>(refined_keys + offset, refined_local + offset, tmp_keys + offset,
                                tmp_values + offset, quota, lds);
}

// Global slot order by merging the per-segment runs. Runs are concatenated in segment
// (= index) order and each is sorted by (key, index); at level l, blocks of 2^l consecutive
// segments are merged pairwise. An element of a left block lands at its own rank plus the
// number of partner keys strictly below it, a right-block element at its rank plus the
// partner keys below or equal (left elements have the lower indices), so the merge is stable
// and the final order is the (key, index) order of torch.topk(largest=False, sorted=True).
__global__ __launch_bounds__(256) void merge_level_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ slots_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ slots_out,
    const uint32_t* __restrict__ segment_of, const int64_t* __restrict__ offsets,
    int64_t segments, int level, int64_t count) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= count) return;
  const int64_t block = segment_of[p] >> level;
  const int64_t pair_first = (block >> 1) << (level + 1);
  const int64_t mid_segment = pair_first + (int64_t{1} << level);
  const int64_t end_segment = pair_first + (int64_t{2} << level);
  const int64_t pair_begin = offsets[pair_first];
  const int64_t mid = offsets[mid_segment < segments ? mid_segment : segments];
  const int64_t pair_end = offsets[end_segment < segments ? end_segment : segments];
  const uint32_t key = keys_in[p];
  int64_t rank, lo, hi;
  if (p < mid) {  // left block: partner = [mid, pair_end), count keys < key
    rank = p - pair_begin;
    lo = mid;
    hi = pair_end;
    while (lo < hi) {
      const int64_t m = (lo + hi) >> 1;
      if (keys_in[m] < key) lo = m + 1;
      else hi = m;
    }
    rank += lo - mid;
  } else {  // right block: partner = [pair_begin, mid), count keys <= key
    rank = p - mid;
    lo = pair_begin;
    hi = mid;
    while (lo < hi) {
      const int64_t m = (lo + hi) >> 1;
      if (keys_in[m] <= key) lo = m + 1;
      else hi = m;
    }
    rank += lo - pair_begin;
  }
  keys_out[pair_begin + rank] = key;
  slots_out[pair_begin + rank] = slots_in[p];
}

// Slot j of the global order: its raw value, its segment, and the refined position that the
// transplant gives it (the r-th slot of a segment takes that segment's r-th refined pick).
__global__ __launch_bounds__(256) void emit_kernel(
    const uint32_t* __restrict__ sorted_keys, const uint32_t* __restrict__ sorted_slots,
    const int64_t* __restrict__ offsets, int64_t segments,
    const int64_t* __restrict__ position_starts, const uint32_t* __restrict__ refined_local,
    int64_t count, float* __restrict__ out_values, int64_t* __restrict__ out_segments,
    int64_t* __restrict__ out_positions) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (j >= count) return;
  const int64_t slot = sorted_slots[j];
  int64_t lo = 0, hi = segments;  // last segment with offsets[s] <= slot
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (offsets[mid] <= slot) lo = mid;
    else hi = mid;
  }
  // skip empty segments sharing the same offset
  while (lo + 1 < segments && offsets[lo + 1] <= slot) ++lo;
  out_values[j] = key_float(sorted_keys[j]);
  out_segments[j] = lo;
  out_positions[j] = position_starts[lo] + refined_local[slot];
}

inline size_t align256(size_t v) { return (v + 255) & ~size_t{255}; }

struct SelectWorkspace {
  SelectState* state;
  uint32_t* hist;
  uint32_t* seg_less;
  uint32_t* seg_equal;
  uint32_t* take_equal;
  uint8_t* raw_flags;
  uint32_t *run_keys, *run_slots, *refined_keys, *refined_local, *tmp_keys, *tmp_values;
  uint32_t* segment_of;
  size_t bytes;
};

inline SelectWorkspace carve(void* base, int64_t total, int64_t segments, int64_t count) {
  SelectWorkspace w;
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  w.state = reinterpret_cast<SelectState*>(take(sizeof(SelectState)));
  w.hist = reinterpret_cast<uint32_t*>(take(size_t{kHistBlocks} * 2048 * 4));
  w.seg_less = reinterpret_cast<uint32_t*>(take(segments * 4));
  w.seg_equal = reinterpret_cast<uint32_t*>(take(segments * 4));
  w.take_equal = reinterpret_cast<uint32_t*>(take(segments * 4));
  w.raw_flags = reinterpret_cast<uint8_t*>(take(total));
  w.run_keys = reinterpret_cast<uint32_t*>(take(count * 4));
  w.run_slots = reinterpret_cast<uint32_t*>(take(count * 4));
  w.refined_keys = reinterpret_cast<uint32_t*>(take(count * 4));
  w.refined_local = reinterpret_cast<uint32_t*>(take(count * 4));
  w.tmp_keys = reinterpret_cast<uint32_t*>(take(count * 4));
  w.tmp_values = reinterpret_cast<uint32_t*>(take(count * 4));
  w.segment_of = reinterpret_cast<uint32_t*>(take(count * 4));
  w.bytes = off;
  return w;
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" size_t lr_select_workspace_bytes(int64_t total, int64_t segments, int64_t count) {
  if (total < 0 || segments < 0 || count < 0) return 0;
  return carve(nullptr, total, segments, count).bytes;
}

extern "C" int lr_select_refine(const float* raw, const float* pooled, int64_t total,
                                const int64_t* segment_ends, const int64_t* position_starts,
                                int64_t segments, int64_t count, void* workspace,
                                size_t workspace_bytes, float* out_values,
                                int64_t* out_segments, int64_t* out_positions, int64_t* quotas,
                                int64_t* offsets, int64_t* removed_positions, int64_t* changed,
                                void* stream) {
  clear_error();
  LR_REQUIRE(total > 0 && segments > 0, "Invalid segment bounds");
  LR_REQUIRE(count > 0 && count <= total, "Selection count must lie in [1, total]");
  LR_REQUIRE(total < (int64_t{1} << 31), "Score table too large");
  LR_REQUIRE(raw && pooled && segment_ends && position_starts && workspace && out_values &&
                 out_segments && out_positions && quotas && offsets && removed_positions && changed,
             "Expected contiguous CUDA tensor");
  const SelectWorkspace w = carve(workspace, total, segments, count);
  LR_REQUIRE(workspace_bytes >= w.bytes, "Workspace too small");
  const hipStream_t s = as_stream(stream);
  const uint32_t k = static_cast<uint32_t>(count);
  LR_REQUIRE((reinterpret_cast<uintptr_t>(raw) & 15) == 0, "Score table must be 16-byte aligned");
  select_init_kernel<<<1, 64, 0, s>>>(w.state, k);
  if (int rc = check_launch("select_init")) return rc;
  const int64_t chunk = ceil_div(ceil_div(total, kHistBlocks), 1024) * 1024;
  const int blocks = static_cast<int>(ceil_div(total, chunk));
  select_block_histogram_kernel<11, 21><<<blocks, 256, 0, s>>>(raw, total, chunk, w.state, w.hist);
  select_reduce_kernel<11, 21><<<1, 1024, 0, s>>>(w.hist, blocks, w.state);
  select_block_histogram_kernel<11, 10><<<blocks, 256, 0, s>>>(raw, total, chunk, w.state, w.hist);
  select_reduce_kernel<11, 10><<<1, 1024, 0, s>>>(w.hist, blocks, w.state);
  select_block_histogram_kernel<10, 0><<<blocks, 256, 0, s>>>(raw, total, chunk, w.state, w.hist);
  select_reduce_kernel<10, 0><<<1, 1024, 0, s>>>(w.hist, blocks, w.state);
  if (int rc = check_launch("select_histogram")) return rc;
  segment_count_kernel<<<segments, kSegThreads, 0, s>>>(raw, segment_ends, w.state, w.seg_less,
                                                        w.seg_equal);
  segment_plan_kernel<<<1, 1024, 0, s>>>(w.seg_less, w.seg_equal, w.state, segments,
                                         w.take_equal, quotas, offsets);
  if (int rc = check_launch("segment_plan")) return rc;
  segment_select_kernel<<<segments, kSegThreads, 0, s>>>(
      raw, pooled, segment_ends, position_starts, w.state, w.take_equal, quotas, offsets,
      w.raw_flags, w.run_keys, w.run_slots, w.refined_keys, w.refined_local, w.tmp_keys,
      w.tmp_values, removed_positions, changed, w.segment_of);
  if (int rc = check_launch("segment_select")) return rc;
  uint32_t* keys = w.run_keys;
  uint32_t* slots = w.run_slots;
  uint32_t* alt_keys = w.tmp_keys;
  uint32_t* alt_slots = w.tmp_values;
  for (int level = 0; (int64_t{1} << level) < segments; ++level) {
    merge_level_kernel<<<ceil_div(count, 256), 256, 0, s>>>(keys, slots, alt_keys, alt_slots,
                                                            w.segment_of, offsets, segments,
                                                            level, count);
    std::swap(keys, alt_keys);
    std::swap(slots, alt_slots);
  }
  if (int rc = check_launch("merge_level")) return rc;
  emit_kernel<<<ceil_div(count, 256), 256, 0, s>>>(keys, slots, offsets, segments,
                                                   position_starts, w.refined_local, count,
                                                   out_values, out_segments, out_positions);
  return check_launch("select_emit");
}
