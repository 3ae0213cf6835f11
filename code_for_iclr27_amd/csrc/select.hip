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
// key (-0.0 and +0.0 are one key; every NaN, whatever its sign and payload, is one key above
// +inf, so NaNs sort last and among themselves by index, as numpy and torch.topk order them).
#include <utility>

#include <rocprim/device/device_radix_sort.hpp>

#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kSegThreads = 256;   // per-segment workgroups
constexpr int kLoadBatch = 8;      // global loads per thread issued together
constexpr int kPickThreads = 512;  // segment_pick workgroups (measured faster than 256:
                                   // cfg1 selection 50 -> 47 us, cfg4 108 -> 79 us)

__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;  // -0.0 == +0.0
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // any NaN
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

// Exclusive scan of a pair of per-thread counts in thread order. Returns each count's offset and
// the block totals in registers. Two barriers; `wave_sums` may be reused after the call.
template <int BLOCK>
__device__ __forceinline__ void block_scan_pair(uint32_t a, uint32_t b, uint32_t (*wave_sums)[2],
                                                uint32_t& before_a, uint32_t& before_b,
                                                uint32_t& total_a, uint32_t& total_b) {
  constexpr int W = BLOCK / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t ia = a, ib = b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t na = __shfl_up(ia, o, 64), nb = __shfl_up(ib, o, 64);
    if (lane >= o) {
      ia += na;
      ib += nb;
    }
  }
  if (lane == 63) {
    wave_sums[wave][0] = ia;
    wave_sums[wave][1] = ib;
  }
  __syncthreads();
  uint32_t ba = 0, bb = 0, ta = 0, tb = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const uint32_t va = wave_sums[w][0], vb = wave_sums[w][1];
    if (w < wave) {
      ba += va;
      bb += vb;
    }
    ta += va;
    tb += vb;
  }
  __syncthreads();
  before_a = ba + ia - a;
  before_b = bb + ib - b;
  total_a = ta;
  total_b = tb;
}

// Digit of a radix-select pass: the bin of `hist` (BINS bins, global or LDS) holding the
// `remaining`-th key (1-based) and the number of keys in lower bins. The histogram must hold
// at least `remaining` keys. All BLOCK threads call it; the result is uniform.
template <int BINS, int BLOCK>
__device__ __forceinline__ void find_digit(const uint32_t* hist, uint32_t remaining,
                                           uint32_t (*wave_sums)[2], uint32_t* found,
                                           uint32_t& digit, uint32_t& below) {
  constexpr int PER = BINS / BLOCK;
  static_assert(PER >= 1 && BINS % BLOCK == 0, "bins per thread");
  if (threadIdx.x == 0) {
    found[0] = BINS - 1;
    found[1] = 0;
  }
  uint32_t c[PER], sum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    c[j] = hist[threadIdx.x * PER + j];
    sum += c[j];
  }
  uint32_t before, unused_b, total, unused_t;
  block_scan_pair<BLOCK>(sum, 0u, wave_sums, before, unused_b, total, unused_t);
  if (before < remaining && before + sum >= remaining) {
    uint32_t run = before, d = threadIdx.x * PER + PER - 1;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (run + c[j] >= remaining) {
        d = threadIdx.x * PER + j;
        break;
      }
      run += c[j];
    }
    found[0] = d;
    found[1] = run;
  }
  __syncthreads();
  digit = found[0];
  below = found[1];
  __syncthreads();
}

// ---------------------------------------------------------------------------------------
// Global threshold: the count-th smallest raw key, by three radix-select passes over all raw
// scores (digits of 11, 11 and 10 bits, most significant first). Pass p histograms, per
// workgroup in LDS, the keys that match the prefix found so far and adds the non-empty bins to
// one global histogram with atomics. The next kernel finds pass p's digit itself, in every
// workgroup (a scan of 2048 bins), so no launch is spent on reductions. states[p] is the
// selection state before pass p; only workgroup 0 of the kernel that derives it writes it.
// Passes 0 and 1 are kernels of their own; the last pass runs inside the per-segment counting
// (segment_count_kernel). The three histograms and the ticket counter are one block of
// kClearWords words that must be zero before pass 0: select_clear_kernel zeroes it, or the
// pool launch of lr_pool_select_refine_sets does.
constexpr int kHistBlocks = 256;
constexpr int kHistStride = 2048;  // words per pass histogram
constexpr int kClearWords = 3 * kHistStride + 1;  // histograms, then the ticket

struct PassShape {
  int bits, shift;
};
__host__ __device__ constexpr PassShape pass_shape(int pass) {
  return pass == 0 ? PassShape{11, 21} : pass == 1 ? PassShape{11, 10} : PassShape{10, 0};
}

__global__ __launch_bounds__(256) void select_clear_kernel(uint32_t* __restrict__ words) {
  for (int i = threadIdx.x; i < kClearWords; i += 256) words[i] = 0;
}

// Extends `st` (the state before pass `pass`) by that pass's digit, read from its histogram.
// All BLOCK threads of the workgroup call it.
template <int PASS, int BLOCK>
__device__ __forceinline__ SelectState extend_state(SelectState st, const uint32_t* __restrict__ hist,
                                                    uint32_t (*wave_sums)[2], uint32_t* found) {
  constexpr PassShape shape = pass_shape(PASS);
  uint32_t digit, below;
  find_digit<1 << shape.bits, BLOCK>(hist + PASS * kHistStride, st.remaining, wave_sums, found,
                                     digit, below);
  st.prefix |= digit << shape.shift;
  st.mask |= ((1u << shape.bits) - 1u) << shape.shift;
  st.less += below;
  st.remaining -= below;
  return st;
}

template <int PASS>
__global__ __launch_bounds__(256) void select_pass_kernel(const float* __restrict__ scores,
                                                          int64_t n, int64_t chunk,
                                                          uint32_t count,
                                                          SelectState* __restrict__ states,
                                                          uint32_t* __restrict__ hist) {
  static_assert(PASS == 0 || PASS == 1, "the last pass runs in segment_count_kernel");
  constexpr PassShape shape = pass_shape(PASS);
  constexpr int BINS = 1 << shape.bits;
  __shared__ uint32_t local[BINS];
  __shared__ uint32_t wave_sums[4][2];
  __shared__ uint32_t found[2];
  SelectState st{};
  if constexpr (PASS == 0) {
    st.remaining = count;  // nothing fixed yet: the count-th smallest of all keys
  } else {
    st = extend_state<PASS - 1, 256>(states[PASS - 1], hist, wave_sums, found);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) states[PASS] = st;
  for (int i = threadIdx.x; i < BINS; i += 256) local[i] = 0;
  __syncthreads();
  const uint32_t prefix = st.prefix, mask = st.mask;
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
        q[u].x = at < end ? scores[at] : 0.0f;
        q[u].y = at + 1 < end ? scores[at + 1] : 0.0f;
        q[u].z = at + 2 < end ? scores[at + 2] : 0.0f;
        q[u].w = at + 3 < end ? scores[at + 3] : 0.0f;
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
          if ((key & mask) == prefix) atomicAdd(&local[(key >> shape.shift) & (BINS - 1)], 1u);
        }
      }
    }
  }
  __syncthreads();
  uint32_t* global_hist = hist + PASS * kHistStride;
  for (int i = threadIdx.x; i < BINS; i += 256) {
    const uint32_t c = local[i];
    if (c) atomicAdd(&global_hist[i], c);
  }
}

// Per segment: how many raw keys lie below / at the global threshold, with the threshold's
// last digit found on the way. Every workgroup derives the threshold's 22-bit prefix from the
// second pass histogram (workgroup 0 publishes it as states[2]), counts its segment's keys
// below that prefix and histograms, in LDS, the last 10 bits of the keys that share it. A
// workgroup whose segment holds such keys adds them to the last pass histogram and keeps that
// LDS histogram's exclusive prefix in its row of `low_prefix` (kLowRow words). The last
// workgroup to finish (a ticket counter, no waiting) finds the last digit from the complete
// histogram, publishes states[3] = {threshold, all-ones mask, threshold-equal keys to take, keys
// below}, turns every segment's counts into keys below / equal to the threshold, and plans the
// per-segment quotas: the threshold-equal keys are granted in index order, i.e. segment order,
// and the quotas' exclusive prefix gives each segment's offset.
constexpr int kLowBins = 1 << pass_shape(2).bits;
constexpr int kLowRow = kLowBins + 1;  // exclusive prefix of the LDS histogram, then its total

__global__ __launch_bounds__(kSegThreads) void segment_count_kernel(
    const float* __restrict__ scores, const int64_t* __restrict__ ends,
    SelectState* __restrict__ states, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ seg_less, uint32_t* __restrict__ seg_equal,
    uint32_t* __restrict__ low_prefix, uint32_t* __restrict__ ticket, int64_t segments,
    uint32_t* __restrict__ take_equal, int64_t* __restrict__ quotas, int64_t* __restrict__ offsets,
    int64_t* __restrict__ host_info, const int32_t* __restrict__ nonfinite) {
  constexpr int PER = kLowBins / kSegThreads;
  static_assert(kLowBins % kSegThreads == 0, "low bins per thread");
  __shared__ uint32_t wave_sums[kSegThreads / 64][2];
  __shared__ uint32_t found[2];
  __shared__ uint32_t low[kLowBins];
  __shared__ bool last;
  for (int i = threadIdx.x; i < kLowBins; i += kSegThreads) low[i] = 0;
  // (extend_state ends with a barrier, which also publishes the zeroed histogram)
  const SelectState st = extend_state<1, kSegThreads>(states[1], hist, wave_sums, found);
  if (blockIdx.x == 0 && threadIdx.x == 0) states[2] = st;
  const int64_t s = blockIdx.x;
  const int64_t begin = s == 0 ? 0 : ends[s - 1], end = ends[s];
  // st.prefix has its last 10 bits clear: key < st.prefix exactly when the key's first 22 bits
  // lie below the threshold's
  uint32_t less = 0, matched = 0;
  // kLoadBatch loads per thread in flight at once (a loop of single loads pays the memory
  // latency once per element)
  for (int64_t base = begin + threadIdx.x; base < end; base += kSegThreads * kLoadBatch) {
    float v[kLoadBatch];
#pragma unroll
    for (int u = 0; u < kLoadBatch; ++u) {
      const int64_t i = base + u * kSegThreads;
      v[u] = i < end ? scores[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kLoadBatch; ++u) {
      if (base + u * kSegThreads < end) {
        const uint32_t key = float_key(v[u]);
        less += key < st.prefix;
        if ((key & st.mask) == st.prefix) {
          ++matched;
          atomicAdd(&low[key & (kLowBins - 1)], 1u);
        }
      }
    }
  }
  uint32_t bl, bm, total_less, total_matched;
  block_scan_pair<kSegThreads>(less, matched, wave_sums, bl, bm, total_less, total_matched);
  if (total_matched != 0) {  // uniform; the scan's barriers published the LDS histogram
    uint32_t c[PER], sum = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      c[j] = low[threadIdx.x * PER + j];
      sum += c[j];
      if (c[j] != 0) atomicAdd(&hist[2 * kHistStride + threadIdx.x * PER + j], c[j]);
    }
    uint32_t before, unused_b, unused_total, unused_t;
    block_scan_pair<kSegThreads>(sum, 0u, wave_sums, before, unused_b, unused_total, unused_t);
    uint32_t* row = low_prefix + s * kLowRow;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      row[threadIdx.x * PER + j] = before;
      before += c[j];
    }
    if (threadIdx.x == kSegThreads - 1) row[kLowBins] = before;
  }
  // The workgroup barrier orders every wave's histogram additions and row stores before wave
  // 0's device-scope release fence, which makes them visible device-wide before the ticket is
  // taken. One release per workgroup (it writes back the XCD's L2); only the last workgroup
  // acquires (which invalidates its XCD's L2), so the others' cached inputs survive.
  __syncthreads();
  if (threadIdx.x == 0) {
    seg_less[s] = total_less;
    seg_equal[s] = total_matched;  // non-zero exactly when the segment's row was written
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    last = atomicAdd(ticket, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;  // uniform across the workgroup
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const SelectState fin = extend_state<2, kSegThreads>(st, hist, wave_sums, found);
  if (threadIdx.x == 0) states[3] = fin;
  const uint32_t digit = fin.prefix & (kLowBins - 1);
  const uint32_t need = fin.remaining;
  uint32_t carry_equal = 0, carry_quota = 0;
  for (int64_t base = 0; base < segments; base += kSegThreads) {
    const int64_t t = base + threadIdx.x;
    uint32_t lt = 0, eq = 0;
    if (t < segments) {
      lt = seg_less[t];
      if (seg_equal[t] != 0) {
        const uint32_t* row = low_prefix + t * kLowRow;
        const uint32_t below = row[digit], through = row[digit + 1];
        lt += below;
        eq = through - below;
      }
    }
    uint32_t eq_before, unused, eq_total, unused_total;
    block_scan_pair<kSegThreads>(eq, 0u, wave_sums, eq_before, unused, eq_total, unused_total);
    eq_before += carry_equal;
    uint32_t take = 0;
    if (need > eq_before) take = need - eq_before < eq ? need - eq_before : eq;
    const uint32_t quota = t < segments ? lt + take : 0;
    uint32_t quota_before, quota_total;
    block_scan_pair<kSegThreads>(quota, 0u, wave_sums, quota_before, unused, quota_total, unused_total);
    quota_before += carry_quota;
    if (t < segments) {
      take_equal[t] = take;
      quotas[t] = quota;
      offsets[t] = quota_before;
      if (host_info != nullptr) host_info[t] = quota;
    }
    carry_equal += eq_total;
    carry_quota += quota_total;
  }
  if (threadIdx.x == 0) {
    offsets[segments] = carry_quota;
    if (host_info != nullptr) host_info[segments] = nonfinite != nullptr ? *nonfinite : 0;
  }
}

// Radix select inside one workgroup: the k-th smallest (1-based) of the n keys key_at(i), by
// three LDS-histogram passes (11, 11, 10 bits). Returns the key and how many keys equal to it
// belong to the bottom k. Each thread reads kLoadBatch keys before it counts them, so keys in
// global memory are read with that many loads in flight.
template <typename KeyAt>
__device__ __forceinline__ void block_select(uint32_t n, uint32_t k, KeyAt key_at, uint32_t* hist,
                                             uint32_t (*wave_sums)[2], uint32_t* found,
                                             uint32_t& threshold, uint32_t& take_equal) {
  SelectState st{};
  st.remaining = k;
  auto pass = [&](auto pass_index) {
    constexpr PassShape shape = pass_shape(decltype(pass_index)::value);
    constexpr int BINS = 1 << shape.bits;
    for (int i = threadIdx.x; i < BINS; i += kPickThreads) hist[i] = 0;
    __syncthreads();
    for (uint32_t base = threadIdx.x; base < n; base += kPickThreads * kLoadBatch) {
      uint32_t keys[kLoadBatch];
#pragma unroll
      for (int u = 0; u < kLoadBatch; ++u) {
        const uint32_t i = base + u * kPickThreads;
        keys[u] = i < n ? key_at(i) : 0u;
      }
#pragma unroll
      for (int u = 0; u < kLoadBatch; ++u)
        if (base + u * kPickThreads < n && (keys[u] & st.mask) == st.prefix)
          atomicAdd(&hist[(keys[u] >> shape.shift) & (BINS - 1)], 1u);
    }
    __syncthreads();
    uint32_t digit, below;
    find_digit<BINS, kPickThreads>(hist, st.remaining, wave_sums, found, digit, below);
    st.prefix |= digit << shape.shift;
    st.mask |= static_cast<uint32_t>(BINS - 1) << shape.shift;
    st.remaining -= below;
  };
  pass(std::integral_constant<int, 0>{});
  pass(std::integral_constant<int, 1>{});
  pass(std::integral_constant<int, 2>{});
  threshold = st.prefix;
  take_equal = st.remaining;
}

// ---------------------------------------------------------------------------------------
// Removal sets. One workgroup per segment with a non-zero quota:
//   raw picks:    key < T, or key == T among the first take_equal such keys in index order;
//   pooled picks: the same rule against the segment's own pooled threshold (bottom-quota).
// Writes the raw picks' keys (index order, for the queue), the pooled picks (index order:
// removal positions ascending, their keys and local indexes for the queue), and the count of
// pooled picks that are not raw picks. The segment's keys go through LDS in chunks of
// kPickStaged (read with coalesced loads, kLoadBatch per thread in flight); a segment of one
// chunk is read once for every pass. Within a chunk each thread owns one contiguous run, so the
// ordered (index-order) compaction costs one block scan per chunk, and the counts of earlier
// chunks carry over.
constexpr uint32_t kPickStaged = 4096;

// Keys [c0, c0 + m) of both score arrays of a segment into LDS. All threads call it.
__device__ __forceinline__ void stage_pick_keys(const float* __restrict__ raw,
                                                const float* __restrict__ pooled, int64_t begin,
                                                uint32_t c0, uint32_t m, uint32_t* raw_keys,
                                                uint32_t* pooled_keys) {
  for (uint32_t base = threadIdx.x; base < m; base += kPickThreads * kLoadBatch) {
    float r[kLoadBatch], q[kLoadBatch];
#pragma unroll
    for (int u = 0; u < kLoadBatch; ++u) {
      const uint32_t i = base + u * kPickThreads;
      r[u] = i < m ? raw[begin + c0 + i] : 0.0f;
      q[u] = i < m ? pooled[begin + c0 + i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kLoadBatch; ++u) {
      const uint32_t i = base + u * kPickThreads;
      if (i < m) {
        raw_keys[i] = float_key(r[u]);
        pooled_keys[i] = float_key(q[u]);
      }
    }
  }
}

__global__ __launch_bounds__(kPickThreads) void segment_pick_kernel(
    const float* __restrict__ raw, const float* __restrict__ pooled,
    const int64_t* __restrict__ ends, const int64_t* __restrict__ position_starts,
    const SelectState* __restrict__ states, const uint32_t* __restrict__ take_equal,
    const int64_t* __restrict__ quotas, const int64_t* __restrict__ offsets,
    uint32_t* __restrict__ run_keys, uint32_t* __restrict__ refined_keys,
    uint32_t* __restrict__ refined_local, int64_t* __restrict__ removed_positions,
    int64_t* __restrict__ changed) {
  __shared__ uint32_t raw_keys[kPickStaged];
  __shared__ uint32_t pooled_keys[kPickStaged];
  __shared__ uint32_t hist[2048];
  __shared__ uint32_t wave_sums[kPickThreads / 64][2];
  __shared__ uint32_t found[2];
  const int64_t s = blockIdx.x;
  const uint32_t quota = static_cast<uint32_t>(quotas[s]);
  if (quota == 0) {
    if (threadIdx.x == 0) changed[s] = 0;
    return;
  }
  const int64_t begin = s == 0 ? 0 : ends[s - 1], end = ends[s];
  const uint32_t n = static_cast<uint32_t>(end - begin);
  const int64_t offset = offsets[s];
  const int64_t position_start = position_starts[s];
  const bool single = n <= kPickStaged;  // uniform: one chunk, staged once for every pass
  if (single) {
    stage_pick_keys(raw, pooled, begin, 0, n, raw_keys, pooled_keys);
    __syncthreads();
  }
  // The thread's run [lo, hi) of a chunk of m keys.
  auto run_of = [](uint32_t m, uint32_t& lo, uint32_t& hi) {
    const uint32_t per = (m + kPickThreads - 1) / kPickThreads;
    lo = min(m, threadIdx.x * per);
    hi = min(m, lo + per);
  };
  // The run's keys (at most kRunMax) into registers with every LDS read issued at once, read
  // once for both passes over the run (a loop of dependent-latency reads otherwise).
  constexpr uint32_t kRunMax = kPickStaged / kPickThreads;
  static_assert(kPickStaged % kPickThreads == 0, "whole runs per chunk");
  auto load_run = [](const uint32_t* keys, uint32_t lo, uint32_t m, uint32_t (&out)[kRunMax]) {
#pragma unroll
    for (uint32_t k = 0; k < kRunMax; ++k) out[k] = keys[min(lo + k, m - 1)];
  };

  // raw picks in index order
  const uint32_t threshold = states[3].prefix, take = take_equal[s];
  {
    uint32_t carry_equal = 0, carry_rank = 0;
    for (uint32_t c0 = 0; c0 < n; c0 += kPickStaged) {
      const uint32_t m = min(n - c0, kPickStaged);
      if (!single) {
        __syncthreads();  // the previous chunk's readers are done
        stage_pick_keys(raw, pooled, begin, c0, m, raw_keys, pooled_keys);
        __syncthreads();
      }
      uint32_t lo, hi;
      run_of(m, lo, hi);
      uint32_t rk[kRunMax];
      load_run(raw_keys, lo, m, rk);
      uint32_t lt = 0, eq = 0;
#pragma unroll
      for (uint32_t k = 0; k < kRunMax; ++k) {
        if (lo + k < hi) {
          lt += rk[k] < threshold;
          eq += rk[k] == threshold;
        }
      }
      uint32_t lt_before, eq_before, lt_total, eq_total;
      block_scan_pair<kPickThreads>(lt, eq, wave_sums, lt_before, eq_before, lt_total, eq_total);
      const uint32_t take_left = take > carry_equal ? take - carry_equal : 0u;
      uint32_t rank = carry_rank + lt_before + min(take_left, eq_before);
      uint32_t seen = eq_before;
#pragma unroll
      for (uint32_t k = 0; k < kRunMax; ++k) {
        if (lo + k < hi) {
          const uint32_t key = rk[k];
          bool picked = key < threshold;
          if (key == threshold) picked = seen++ < take_left;
          if (picked) run_keys[offset + rank++] = key;
        }
      }
      carry_rank += lt_total + min(take_left, eq_total);
      carry_equal += eq_total;
    }
  }

  // pooled picks: bottom-quota of the segment's pooled keys, in index order
  uint32_t pthreshold, ptake;
  if (single) {
    block_select(n, quota, [&](uint32_t i) { return pooled_keys[i]; }, hist, wave_sums, found,
                 pthreshold, ptake);
  } else {
    block_select(n, quota, [&](uint32_t i) { return float_key(pooled[begin + i]); }, hist,
                 wave_sums, found, pthreshold, ptake);
  }
  uint32_t moved = 0;
  {
    uint32_t carry_equal = 0, carry_rank = 0, carry_raw_equal = 0;
    for (uint32_t c0 = 0; c0 < n; c0 += kPickStaged) {
      const uint32_t m = min(n - c0, kPickStaged);
      if (!single) {
        __syncthreads();
        stage_pick_keys(raw, pooled, begin, c0, m, raw_keys, pooled_keys);
        __syncthreads();
      }
      uint32_t lo, hi;
      run_of(m, lo, hi);
      uint32_t rk[kRunMax], pk[kRunMax];
      load_run(raw_keys, lo, m, rk);
      load_run(pooled_keys, lo, m, pk);
      uint32_t lt = 0, eq = 0, raw_eq = 0;
#pragma unroll
      for (uint32_t k = 0; k < kRunMax; ++k) {
        if (lo + k < hi) {
          lt += pk[k] < pthreshold;
          eq += pk[k] == pthreshold;
          raw_eq += rk[k] == threshold;
        }
      }
      uint32_t lt_before, eq_before, lt_total, eq_total;
      block_scan_pair<kPickThreads>(lt, eq, wave_sums, lt_before, eq_before, lt_total, eq_total);
      uint32_t raw_eq_before, unused, raw_eq_total, unused_total;
      block_scan_pair<kPickThreads>(raw_eq, 0u, wave_sums, raw_eq_before, unused, raw_eq_total,
                                    unused_total);
      const uint32_t take_left = ptake > carry_equal ? ptake - carry_equal : 0u;
      const uint32_t raw_take_left = take > carry_raw_equal ? take - carry_raw_equal : 0u;
      uint32_t rank = carry_rank + lt_before + min(take_left, eq_before);
      uint32_t seen = eq_before, raw_seen = raw_eq_before;
#pragma unroll
      for (uint32_t k = 0; k < kRunMax; ++k) {
        if (lo + k >= hi) continue;
        const uint32_t i = lo + k;
        // the raw rule again, in index order, tells whether slot i was a raw pick
        const uint32_t rkey = rk[k];
        bool raw_picked = rkey < threshold;
        if (rkey == threshold) raw_picked = raw_seen++ < raw_take_left;
        const uint32_t key = pk[k];
        bool picked = key < pthreshold;
        if (key == pthreshold) picked = seen++ < take_left;
        if (picked) {
          refined_keys[offset + rank] = key;
          refined_local[offset + rank] = c0 + i;
          removed_positions[offset + rank] = position_start + c0 + i;
          ++rank;
          moved += raw_picked ? 0u : 1u;
        }
      }
      carry_rank += lt_total + min(take_left, eq_total);
      carry_equal += eq_total;
      carry_raw_equal += raw_eq_total;
    }
  }
  uint32_t moved_before, unused, moved_total, unused_total;
  block_scan_pair<kPickThreads>(moved, 0u, wave_sums, moved_before, unused, moved_total, unused_total);
  if (threadIdx.x == 0) changed[s] = moved_total;
}

// ---------------------------------------------------------------------------------------
// Queue order. Per segment, both pick lists are put in (key, index) order: the raw picks give
// the segment's slots, the pooled picks what fills them (transplant). Slot j of the global
// order is then the j-th smallest raw pick over all segments, by (key, index), and takes the
// pooled pick of its segment at its rank within that segment.
//
// Up to kOrderMaxRuns segments and kOrderMaxCount picks (buckets of 512 picks on average), the
// global order is a bucketed merge of the sorted runs (three launches):
//   1. order_splitters_kernel: `samples` raw picks at a fixed stride of the concatenated
//      index-order lists, as (key << 32 | list position) composites. Composites are unique and
//      their order is the final (key, index) order. Each workgroup counts the rank of
//      kSplitterSamples of them among all samples in LDS; the sample of rank
//      ((b + 1) * samples) / buckets - 1 is splitter b, so the splitters cut the picks into
//      `buckets` ranges.
//   2. segment_sort_kernel: sorts each segment's two lists in LDS, then binary-searches every
//      splitter in the sorted raw list: bucket_pos[b][s] = how many of segment s's picks lie
//      at or below splitter b.
//   3. order_bucket_kernel (one workgroup per bucket): gathers its bucket's picks (a
//      contiguous range of every segment's sorted run), sorts them in LDS, and writes each one
//      at (picks below the bucket) + (rank within it), with its segment and transplanted
//      position. A bucket larger than LDS holds is sorted in global memory instead.
// More segments or picks than that: the runs are sorted the same way and rocPRIM's device radix
// sort orders the concatenation, then emit_kernel writes the slots.
//
// Per-segment sorts, by list length n:
//   n <= kRankSortMax: both lists at once, one half of the workgroup each; each entry's rank
//     (entries whose (key << 32 | index) composite is smaller: a smaller key, or an equal key
//     at a lower index) is counted by one, two or four lanes over interleaved parts of the
//     list in LDS and summed across them;
//   n <= kBitonicMax: a bitonic network over (key << 32 | index) pairs in LDS, one list after
//     the other;
//   longer lists: the block radix sort in global memory.
// Every sort keeps equal keys in index order.
constexpr int kSortThreads = 1024;       // segment_sort and splitter workgroups
constexpr uint32_t kRankSortMax = kSortThreads / 2;
constexpr uint32_t kBitonicMax = 4096;
constexpr int64_t kOrderMaxRuns = 1024;  // segments the bucketed order takes (LDS run tables)
constexpr uint32_t kOrderSamples = 2048;
constexpr int64_t kOrderBucketTarget = 128;  // mean picks per bucket
constexpr uint32_t kOrderMaxBuckets = 1024;
constexpr int64_t kOrderMaxCount = int64_t{kOrderMaxBuckets} * 512;
constexpr int kBucketThreads = 512;
constexpr uint32_t kBucketCap = 4096;  // bucket entries sorted in LDS

struct OrderShape {
  bool bucketed;
  uint32_t samples, stride, buckets;
};

// samples >= buckets, so the splitters (sorted samples at indexes ((b + 1) * samples) / buckets
// - 1) are distinct and increasing.
inline OrderShape order_shape(int64_t segments, int64_t count) {
  OrderShape o{};
  o.bucketed = segments <= kOrderMaxRuns && count > 0 && count <= kOrderMaxCount;
  if (!o.bucketed) return o;
  o.samples = static_cast<uint32_t>(count < kOrderSamples ? count : kOrderSamples);
  o.stride = static_cast<uint32_t>(count / o.samples);
  int64_t b = ceil_div(count, kOrderBucketTarget);
  if (b > kOrderMaxBuckets) b = kOrderMaxBuckets;
  if (b > o.samples) b = o.samples;
  o.buckets = static_cast<uint32_t>(b < 1 ? 1 : b);
  return o;
}

constexpr uint32_t kSplitterSamples = 64;  // samples ranked per splitter workgroup

struct RankLds {
  alignas(16) uint64_t composite[2][kRankSortMax];  // (key << 32 | index), padded with ~0
  uint32_t values[kRankSortMax];
  uint64_t sorted[kRankSortMax];  // the raw list's (key << 32 | offset + index) at their ranks
};

union SegmentSortLds {
  RankLds rank;
  struct {
    uint64_t pairs[kBitonicMax];
    uint32_t local[kBitonicMax];
  } bitonic;
  SortLds<kSortThreads> radix;
};

// Both lists of a segment (n <= kRankSortMax each) sorted by (key, index) in place: threads
// [0, kRankSortMax) rank the raw keys, the rest the pooled picks (keys, with their local
// indexes). With `composites`, the raw list's (key << 32 | offset + index) are left at their
// ranks in lds.sorted.
__device__ __forceinline__ void rank_sort_lists(uint32_t* raw_keys, uint32_t* pooled_keys,
                                                uint32_t* pooled_local, uint32_t n,
                                                uint32_t offset, bool composites,
                                                RankLds& lds) {
  const uint32_t list = threadIdx.x / kRankSortMax, t = threadIdx.x % kRankSortMax;
  const uint32_t n2 = (n + 1) & ~1u;
  uint64_t* lc = lds.composite[list];
  const uint32_t* src = list == 0 ? raw_keys : pooled_keys;
  for (uint32_t i = t; i < n2; i += kRankSortMax) {
    lc[i] = i < n ? (static_cast<uint64_t>(src[i]) << 32) | i : ~0ull;
    if (list == 1 && i < n) lds.values[i] = pooled_local[i];
  }
  __syncthreads();
  // lanes per entry (uniform): every lane of a group runs the same trip count
  const uint32_t lanes = n <= kRankSortMax / 4 ? 4u : n <= kRankSortMax / 2 ? 2u : 1u;
  const uint32_t i = t / lanes, part = t % lanes;
  const uint64_t mine = i < n ? lc[i] : ~0ull;
  uint32_t rank = 0;
  // composites are unique; the padding (~0) is never below a real one. Unrolled so that
  // several LDS reads are in flight (the loop is bound by their latency, not by VALU issue).
#pragma unroll 8
  for (uint32_t j = 2 * part; j < n2; j += 2 * lanes) {
    const ulonglong2 c2 = *reinterpret_cast<const ulonglong2*>(lc + j);
    rank += c2.x < mine;
    rank += c2.y < mine;
  }
  if (lanes >= 2) rank += __shfl_xor(rank, 1, 64);
  if (lanes == 4) rank += __shfl_xor(rank, 2, 64);
  if (part == 0 && i < n) {
    const uint32_t key = static_cast<uint32_t>(mine >> 32);
    if (list == 0) {
      raw_keys[rank] = key;
      if (composites) lds.sorted[rank] = mine + offset;
    } else {
      pooled_keys[rank] = key;
      pooled_local[rank] = lds.values[i];
    }
  }
  __syncthreads();
}

// Ascending sort of a[0, n2), n2 a power of two, by all BLOCK threads.
template <int BLOCK>
__device__ __forceinline__ void bitonic_sort_lds(uint64_t* a, uint32_t n2) {
  for (uint32_t size = 2; size <= n2; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (uint32_t t = threadIdx.x; t < n2 / 2; t += BLOCK) {
        const uint32_t i = 2 * t - (t & (stride - 1));  // lower element of pair t
        const uint64_t x = a[i], y = a[i + stride];
        if ((x > y) == ((i & size) == 0)) {
          a[i] = y;
          a[i + stride] = x;
        }
      }
      __syncthreads();
    }
  }
}

// bucket_pos[b * segments + s] for splitter b = threadIdx.x (its value in `split`): the number
// of entries r of the sorted run with composite(r) <= split (binary search).
template <typename CompositeAt>
__device__ __forceinline__ void partition_run(uint32_t n, CompositeAt composite, uint64_t split,
                                              uint32_t buckets, int64_t s, int64_t segments,
                                              uint32_t* __restrict__ bucket_pos) {
  const uint32_t b = threadIdx.x;
  if (b + 1 >= buckets) return;
  uint32_t lo = 0, hi = n;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (composite(mid) <= split) lo = mid + 1;
    else hi = mid;
  }
  bucket_pos[b * segments + s] = lo;
}

// One workgroup per segment. In the bucketed order (buckets > 0) it also partitions the sorted
// raw run by the buckets - 1 splitters; otherwise it writes each slot's position in the
// concatenated runs for the device radix sort.
__global__ __launch_bounds__(kSortThreads) void segment_sort_kernel(
    const int64_t* __restrict__ quotas, const int64_t* __restrict__ offsets,
    uint32_t* __restrict__ run_keys, uint32_t* __restrict__ run_slots,
    uint32_t* __restrict__ refined_keys, uint32_t* __restrict__ refined_local,
    uint32_t* __restrict__ tmp_keys, uint32_t* __restrict__ tmp_values,
    const uint64_t* __restrict__ splitters, uint32_t buckets, uint32_t* __restrict__ bucket_pos,
    int64_t segments) {
  static_assert(kOrderMaxBuckets <= kSortThreads, "one splitter per thread");
  __shared__ SegmentSortLds lds;
  const int64_t s = blockIdx.x;
  const bool order = buckets > 0;  // the bucketed order (buckets == 1: no splitters)
  // independent loads, issued together: thread b's splitter, the segment's list
  const uint64_t split = threadIdx.x + 1 < buckets ? splitters[threadIdx.x] : 0ull;
  const uint32_t quota = static_cast<uint32_t>(quotas[s]);
  const uint32_t offset = static_cast<uint32_t>(offsets[s]);
  if (quota == 0) {
    if (threadIdx.x + 1 < buckets) bucket_pos[threadIdx.x * segments + s] = 0u;
    return;
  }
  uint32_t* keys = run_keys + offset;
  if (quota <= kRankSortMax) {
    rank_sort_lists(keys, refined_keys + offset, refined_local + offset, quota, offset, order,
                    lds.rank);
    if (order)
      partition_run(quota, [&](uint32_t r) { return lds.rank.sorted[r]; }, split, buckets, s,
                    segments, bucket_pos);
  } else if (quota <= kBitonicMax) {
    uint32_t n2 = 1;
    while (n2 < quota) n2 <<= 1;
    uint64_t* pairs = lds.bitonic.pairs;
    for (uint32_t i = threadIdx.x; i < n2; i += kSortThreads)
      pairs[i] = i < quota ? (static_cast<uint64_t>(keys[i]) << 32) | i : ~0ull;
    __syncthreads();
    bitonic_sort_lds<kSortThreads>(pairs, n2);
    for (uint32_t i = threadIdx.x; i < quota; i += kSortThreads)
      keys[i] = static_cast<uint32_t>(pairs[i] >> 32);
    if (order)
      partition_run(quota, [&](uint32_t r) { return pairs[r] + offset; }, split, buckets, s,
                    segments, bucket_pos);
    __syncthreads();  // the raw list's readers are done with the LDS
    for (uint32_t i = threadIdx.x; i < n2; i += kSortThreads) {
      pairs[i] = i < quota ? (static_cast<uint64_t>(refined_keys[offset + i]) << 32) | i : ~0ull;
      if (i < quota) lds.bitonic.local[i] = refined_local[offset + i];
    }
    __syncthreads();
    bitonic_sort_lds<kSortThreads>(pairs, n2);
    for (uint32_t i = threadIdx.x; i < quota; i += kSortThreads) {
      const uint64_t pair = pairs[i];
      refined_keys[offset + i] = static_cast<uint32_t>(pair >> 32);
      refined_local[offset + i] = lds.bitonic.local[static_cast<uint32_t>(pair)];
    }
  } else {
    // payload: each raw pick's index in the segment's list
    for (uint32_t i = threadIdx.x; i < quota; i += kSortThreads) run_slots[offset + i] = i;
    __syncthreads();
    block_radix_sort<kSortThreads>(keys, run_slots + offset, tmp_keys + offset,
                                   tmp_values + offset, quota, lds.radix);
    if (order) {
      const uint32_t* index = run_slots + offset;
      partition_run(quota,
                    [&](uint32_t r) {
                      return (static_cast<uint64_t>(keys[r]) << 32) | (offset + index[r]);
                    },
                    split, buckets, s, segments, bucket_pos);
    }
    block_radix_sort<kSortThreads>(refined_keys + offset, refined_local + offset,
                                   tmp_keys + offset, tmp_values + offset, quota, lds.radix);
  }
  if (!order) {
    __syncthreads();
    // slot payload for the device radix sort: position in the concatenated runs
    for (uint32_t i = threadIdx.x; i < quota; i += kSortThreads) run_slots[offset + i] = offset + i;
  }
}

// Splitters of the bucketed order from the index-order raw picks (before segment_sort sorts
// them): sample j is the pick at list position j * stride. Workgroup w ranks samples
// [w * kSplitterSamples, ...), each by kSortThreads / kSplitterSamples lanes over interleaved
// parts of all samples in LDS.
__global__ __launch_bounds__(kSortThreads) void order_splitters_kernel(
    const uint32_t* __restrict__ run_keys, uint32_t samples, uint32_t stride, uint32_t buckets,
    uint64_t* __restrict__ splitters) {
  constexpr uint32_t kLanes = kSortThreads / kSplitterSamples;
  static_assert(kLanes <= 64 && 64 % kLanes == 0, "a sample's lanes share a wave");
  __shared__ uint64_t all[kOrderSamples];
  for (uint32_t j = threadIdx.x; j < samples; j += kSortThreads) {
    const uint32_t at = j * stride;
    all[j] = (static_cast<uint64_t>(run_keys[at]) << 32) | at;
  }
  __syncthreads();
  const uint32_t j = blockIdx.x * kSplitterSamples + threadIdx.x / kLanes;
  const uint32_t part = threadIdx.x % kLanes;
  const uint64_t mine = j < samples ? all[j] : ~0ull;
  uint32_t rank = 0;
#pragma unroll 8
  for (uint32_t k = part; k < samples; k += kLanes) rank += all[k] < mine;
#pragma unroll
  for (uint32_t o = 1; o < kLanes; o <<= 1) rank += __shfl_xor(rank, o, 64);
  if (part != 0 || j >= samples) return;
  // splitter b is the sample of rank ((b + 1) * samples) / buckets - 1; samples >= buckets, so
  // at most one b maps to a rank: the least m = b + 1 with (m * samples) / buckets > rank
  const uint64_t m = ((static_cast<uint64_t>(rank) + 1) * buckets + samples - 1) / samples;
  if (m >= 1 && m < buckets && (m * samples) / buckets - 1 == rank) splitters[m - 1] = mine;
}

struct BucketLds {
  uint32_t lo[kOrderMaxRuns];         // the bucket's first entry in each sorted run
  uint32_t start[kOrderMaxRuns + 1];  // exclusive prefix of the runs' shares
  uint32_t offset[kOrderMaxRuns];     // each run's position in the concatenation
  uint32_t wave_sums[kBucketThreads / 64][2];
  union alignas(16) {
    uint64_t pairs[kBucketCap];
    SortLds<kBucketThreads> radix;
  };
};

// Bucket b: the picks above splitter b - 1 and at or below splitter b (composite order). Each
// gathered entry e carries (key << 32 | e); e runs over the segments in order and within a run
// in sorted order, so for equal keys e order is index order and (key, e) order is the final
// order. Entries of buckets larger than kBucketCap go through spill_* (global, disjoint
// ranges per bucket) and the block radix sort.
__global__ __launch_bounds__(kBucketThreads) void order_bucket_kernel(
    const uint32_t* __restrict__ run_keys, const int64_t* __restrict__ quotas,
    const int64_t* __restrict__ offsets, const uint32_t* __restrict__ bucket_pos,
    int64_t segments, uint32_t buckets, const int64_t* __restrict__ position_starts,
    const uint32_t* __restrict__ refined_local, uint32_t* __restrict__ spill_keys,
    uint32_t* __restrict__ spill_entries, uint32_t* __restrict__ spill_keys2,
    uint32_t* __restrict__ spill_entries2, float* __restrict__ out_values,
    int64_t* __restrict__ out_segments, int64_t* __restrict__ out_positions) {
  __shared__ BucketLds lds;
  const uint32_t b = blockIdx.x;
  const int S = static_cast<int>(segments);
  constexpr int kPer = (kOrderMaxRuns + kBucketThreads - 1) / kBucketThreads;
  // each thread's runs [first, first + kPer): shares in this bucket, and picks below it
  const int first = threadIdx.x * kPer;
  uint32_t share[kPer], share_sum = 0, below_sum = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int s = first + k;
    share[k] = 0;
    if (s < S) {
      const uint32_t lo = b == 0 ? 0u : bucket_pos[static_cast<int64_t>(b - 1) * S + s];
      const uint32_t hi = b + 1 == buckets ? static_cast<uint32_t>(quotas[s])
                                           : bucket_pos[static_cast<int64_t>(b) * S + s];
      lds.lo[s] = lo;
      lds.offset[s] = static_cast<uint32_t>(offsets[s]);
      share[k] = hi - lo;
      share_sum += hi - lo;
      below_sum += lo;
    }
  }
  uint32_t before, unused, size, base;
  block_scan_pair<kBucketThreads>(share_sum, below_sum, lds.wave_sums, before, unused, size, base);
  if (size == 0) return;  // uniform
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int s = first + k;
    if (s < S) lds.start[s] = before;
    before += share[k];
  }
  if (threadIdx.x == 0) lds.start[S] = size;
  __syncthreads();
  // the run holding entry e: the last s with start[s] <= e (that run is not empty)
  auto run_of = [&](uint32_t e) {
    int lo = 0, hi = S;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (lds.start[mid] <= e) lo = mid;
      else hi = mid;
    }
    return lo;
  };
  // entry e's segment and its slot in the concatenated sorted runs
  auto locate = [&](uint32_t e, int& seg, uint32_t& slot) {
    seg = run_of(e);
    slot = lds.offset[seg] + lds.lo[seg] + (e - lds.start[seg]);
  };
  auto emit = [&](uint32_t r, uint32_t key, uint32_t e) {
    int seg;
    uint32_t slot;
    locate(e, seg, slot);
    const int64_t j = static_cast<int64_t>(base) + r;
    out_values[j] = key_float(key);
    out_segments[j] = seg;
    out_positions[j] = position_starts[seg] + refined_local[slot];
  };
  auto key_of = [&](uint32_t e) {
    int seg;
    uint32_t slot;
    locate(e, seg, slot);
    return run_keys[slot];
  };
  if (size <= kBucketCap) {
    uint64_t* pairs = lds.pairs;
    if (size <= kBucketThreads) {
      // one entry per thread, its outputs loaded with its key; rank among the bucket's
      // (unique) composites
      const uint32_t e = threadIdx.x, n2 = (size + 1) & ~1u;
      uint64_t mine = ~0ull;
      int seg = 0;
      int64_t position = 0;
      if (e < size) {
        uint32_t slot;
        locate(e, seg, slot);
        mine = (static_cast<uint64_t>(run_keys[slot]) << 32) | e;
        position = position_starts[seg] + refined_local[slot];
      }
      if (e < n2) pairs[e] = mine;
      __syncthreads();
      if (e < size) {
        uint32_t rank = 0;
#pragma unroll 8
        for (uint32_t k = 0; k < n2; k += 2) {
          const ulonglong2 c2 = *reinterpret_cast<const ulonglong2*>(pairs + k);
          rank += c2.x < mine;
          rank += c2.y < mine;
        }
        const int64_t j = static_cast<int64_t>(base) + rank;
        out_values[j] = key_float(static_cast<uint32_t>(mine >> 32));
        out_segments[j] = seg;
        out_positions[j] = position;
      }
      return;
    }
    uint32_t n2 = 1;
    while (n2 < size) n2 <<= 1;
    for (uint32_t e = threadIdx.x; e < n2; e += kBucketThreads)
      pairs[e] = e < size ? (static_cast<uint64_t>(key_of(e)) << 32) | e : ~0ull;
    __syncthreads();
    bitonic_sort_lds<kBucketThreads>(pairs, n2);
    for (uint32_t r = threadIdx.x; r < size; r += kBucketThreads)
      emit(r, static_cast<uint32_t>(pairs[r] >> 32), static_cast<uint32_t>(pairs[r]));
    return;
  }
  uint32_t* keys = spill_keys + base;
  uint32_t* entries = spill_entries + base;
  for (uint32_t e = threadIdx.x; e < size; e += kBucketThreads) {
    keys[e] = key_of(e);
    entries[e] = e;
  }
  __threadfence_block();
  __syncthreads();
  // stable by key over entries in e order: (key, e) order
  block_radix_sort<kBucketThreads>(keys, entries, spill_keys2 + base, spill_entries2 + base, size,
                                   lds.radix);
  for (uint32_t r = threadIdx.x; r < size; r += kBucketThreads) emit(r, keys[r], entries[r]);
}

// Global slot order for more than kOrderMaxRuns segments: the runs are concatenated in segment
// (= index) order and each is sorted by (key, index), so a stable radix sort of the
// concatenation by key alone gives the (key, index) order of torch.topk(largest=False,
// sorted=True). It is rocPRIM's device radix sort (a plain library sort of `count` key/slot
// pairs).
size_t order_sort_bytes(int64_t segments, int64_t count) {
  size_t bytes = 0;
  if (count > 0 && !order_shape(segments, count).bucketed)
    (void)rocprim::radix_sort_pairs(nullptr, bytes, static_cast<const uint32_t*>(nullptr),
                                    static_cast<uint32_t*>(nullptr),
                                    static_cast<const uint32_t*>(nullptr),
                                    static_cast<uint32_t*>(nullptr), static_cast<size_t>(count));
  return bytes;
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
  SelectState* states;  // [4]: before each threshold pass, then final
  uint32_t* hist;       // [3][kHistStride], then the ticket: kClearWords words zeroed per call
  uint32_t* ticket;     // workgroups of segment_count that have finished
  uint32_t* seg_less;
  uint32_t* seg_equal;
  uint32_t* low_prefix;  // [segments][kLowRow]
  uint32_t* take_equal;
  uint32_t *run_keys, *run_slots, *refined_keys, *refined_local, *tmp_keys, *tmp_values;
  OrderShape order;
  uint64_t* splitters;   // [buckets - 1]
  uint32_t* bucket_pos;  // [buckets - 1][segments]
  uint32_t *spill_keys, *spill_entries;  // ping-pong of an oversized bucket's global sort
  void* sort_storage;  // rocPRIM's temporary storage for the global order
  size_t sort_bytes;
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
  w.states = reinterpret_cast<SelectState*>(take(4 * sizeof(SelectState)));
  w.hist = reinterpret_cast<uint32_t*>(take(size_t{kClearWords} * 4));
  w.ticket = w.hist == nullptr ? nullptr : w.hist + 3 * kHistStride;
  w.seg_less = reinterpret_cast<uint32_t*>(take(segments * 4));
  w.seg_equal = reinterpret_cast<uint32_t*>(take(segments * 4));
  w.low_prefix = reinterpret_cast<uint32_t*>(take(static_cast<size_t>(segments) * kLowRow * 4));
  w.take_equal = reinterpret_cast<uint32_t*>(take(segments * 4));
  w.run_keys = reinterpret_cast<uint32_t*>(take(count * 4));
  w.run_slots = reinterpret_cast<uint32_t*>(take(count * 4));
  w.refined_keys = reinterpret_cast<uint32_t*>(take(count * 4));
  w.refined_local = reinterpret_cast<uint32_t*>(take(count * 4));
  w.tmp_keys = reinterpret_cast<uint32_t*>(take(count * 4));
  w.tmp_values = reinterpret_cast<uint32_t*>(take(count * 4));
  w.order = order_shape(segments, count);
  const size_t cuts = w.order.bucketed ? w.order.buckets - 1 : 0;
  w.splitters = reinterpret_cast<uint64_t*>(take(cuts * 8));
  w.bucket_pos = reinterpret_cast<uint32_t*>(take(cuts * segments * 4));
  w.spill_keys = reinterpret_cast<uint32_t*>(take(w.order.bucketed ? count * 4 : 0));
  w.spill_entries = reinterpret_cast<uint32_t*>(take(w.order.bucketed ? count * 4 : 0));
  w.sort_bytes = order_sort_bytes(segments, count);
  w.sort_storage = take(w.sort_bytes);
  w.bytes = off;
  return w;
}

// `cleared`: the caller's launch on the same stream has already zeroed w.hist[0, kClearWords).
int launch_sets(const float* raw, const float* pooled, int64_t total, const int64_t* segment_ends,
                const int64_t* position_starts, int64_t segments, int64_t count,
                const SelectWorkspace& w, int64_t* quotas, int64_t* offsets,
                int64_t* removed_positions, int64_t* changed, int64_t* host_info,
                const int32_t* nonfinite, bool cleared, hipStream_t s) {
  if (!cleared) {
    select_clear_kernel<<<1, 256, 0, s>>>(w.hist);
    if (int rc = check_launch("select_clear")) return rc;
  }
  const int64_t chunk = ceil_div(ceil_div(total, kHistBlocks), 1024) * 1024;
  const int blocks = static_cast<int>(ceil_div(total, chunk));
  const uint32_t k = static_cast<uint32_t>(count);
  select_pass_kernel<0><<<blocks, 256, 0, s>>>(raw, total, chunk, k, w.states, w.hist);
  select_pass_kernel<1><<<blocks, 256, 0, s>>>(raw, total, chunk, k, w.states, w.hist);
  if (int rc = check_launch("select_pass")) return rc;
  segment_count_kernel<<<segments, kSegThreads, 0, s>>>(raw, segment_ends, w.states, w.hist,
                                                        w.seg_less, w.seg_equal, w.low_prefix,
                                                        w.ticket, segments, w.take_equal, quotas,
                                                        offsets, host_info, nonfinite);
  if (int rc = check_launch("segment_count")) return rc;
  segment_pick_kernel<<<segments, kPickThreads, 0, s>>>(
      raw, pooled, segment_ends, position_starts, w.states, w.take_equal, quotas, offsets,
      w.run_keys, w.refined_keys, w.refined_local, removed_positions, changed);
  return check_launch("segment_pick");
}

// The queue order from the removal sets' pick lists (see the queue-order section above).
int launch_queue(const int64_t* position_starts, int64_t segments, int64_t count,
                 const SelectWorkspace& w, const int64_t* quotas, const int64_t* offsets,
                 float* out_values, int64_t* out_segments, int64_t* out_positions,
                 hipStream_t s) {
  const OrderShape& o = w.order;
  if (o.bucketed) {
    if (o.buckets > 1) {
      const unsigned groups = static_cast<unsigned>(ceil_div(o.samples, kSplitterSamples));
      order_splitters_kernel<<<groups, kSortThreads, 0, s>>>(w.run_keys, o.samples, o.stride,
                                                             o.buckets, w.splitters);
      if (int rc = check_launch("order_splitters")) return rc;
    }
    segment_sort_kernel<<<segments, kSortThreads, 0, s>>>(
        quotas, offsets, w.run_keys, w.run_slots, w.refined_keys, w.refined_local, w.tmp_keys,
        w.tmp_values, w.splitters, o.buckets, w.bucket_pos, segments);
    if (int rc = check_launch("segment_sort")) return rc;
    order_bucket_kernel<<<o.buckets, kBucketThreads, 0, s>>>(
        w.run_keys, quotas, offsets, w.bucket_pos, segments, o.buckets, position_starts,
        w.refined_local, w.tmp_keys, w.tmp_values, w.spill_keys, w.spill_entries, out_values,
        out_segments, out_positions);
    return check_launch("order_bucket");
  }
  segment_sort_kernel<<<segments, kSortThreads, 0, s>>>(quotas, offsets, w.run_keys, w.run_slots,
                                                        w.refined_keys, w.refined_local,
                                                        w.tmp_keys, w.tmp_values, nullptr, 0u,
                                                        nullptr, segments);
  if (int rc = check_launch("segment_sort")) return rc;
  size_t sort_bytes = w.sort_bytes;
  const hipError_t sorted = rocprim::radix_sort_pairs(
      w.sort_storage, sort_bytes, static_cast<const uint32_t*>(w.run_keys), w.tmp_keys,
      static_cast<const uint32_t*>(w.run_slots), w.tmp_values, static_cast<size_t>(count), 0u,
      32u, s);
  if (sorted != hipSuccess) {
    (void)hipGetLastError();
    set_error(std::string("queue order sort failed: ") + hipGetErrorString(sorted));
    return LR_ERR_HIP;
  }
  emit_kernel<<<ceil_div(count, 256), 256, 0, s>>>(w.tmp_keys, w.tmp_values, offsets, segments,
                                                   position_starts, w.refined_local, count,
                                                   out_values, out_segments, out_positions);
  return check_launch("select_emit");
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" size_t lr_select_workspace_bytes(int64_t total, int64_t segments, int64_t count) {
  if (total < 0 || segments < 0 || count < 0) return 0;
  return carve(nullptr, total, segments, count).bytes;
}

#define LR_SELECT_CHECK_SHAPE()                                                              \
  LR_REQUIRE(total > 0 && segments > 0, "Invalid segment bounds");                           \
  LR_REQUIRE(count > 0 && count <= total, "Selection count must lie in [1, total]");         \
  LR_REQUIRE(total < (int64_t{1} << 31), "Score table too large")

extern "C" int lr_select_refine_sets(const float* raw, const float* pooled, int64_t total,
                                     const int64_t* segment_ends, const int64_t* position_starts,
                                     int64_t segments, int64_t count, void* workspace,
                                     size_t workspace_bytes, int64_t* quotas, int64_t* offsets,
                                     int64_t* removed_positions, int64_t* changed,
                                     int64_t* host_info, const int32_t* nonfinite, void* stream) {
  clear_error();
  LR_SELECT_CHECK_SHAPE();
  LR_REQUIRE(raw && pooled && segment_ends && position_starts && workspace && quotas && offsets &&
                 removed_positions && changed,
             "Expected contiguous CUDA tensor");
  LR_REQUIRE((reinterpret_cast<uintptr_t>(raw) & 15) == 0, "Score table must be 16-byte aligned");
  const SelectWorkspace w = carve(workspace, total, segments, count);
  LR_REQUIRE(workspace_bytes >= w.bytes, "Workspace too small");
  return launch_sets(raw, pooled, total, segment_ends, position_starts, segments, count, w, quotas,
                     offsets, removed_positions, changed, host_info, nonfinite, false,
                     as_stream(stream));
}

extern "C" int lr_pool_select_refine_sets(const float* raw, int64_t total, const int64_t* bounds,
                                          int64_t max_count, int64_t width, float* pooled,
                                          const int64_t* segment_ends,
                                          const int64_t* position_starts, int64_t segments,
                                          int64_t count, void* workspace, size_t workspace_bytes,
                                          int64_t* quotas, int64_t* offsets,
                                          int64_t* removed_positions, int64_t* changed,
                                          int64_t* host_info, const int32_t* nonfinite,
                                          void* stream) {
  clear_error();
  LR_SELECT_CHECK_SHAPE();
  LR_REQUIRE(width > 0 && width % 2 == 1 && max_count > 0, "Invalid pool configuration");
  LR_REQUIRE(segments <= 65535, "Invalid pool layout");
  LR_REQUIRE(raw && bounds && pooled && segment_ends && position_starts && workspace && quotas &&
                 offsets && removed_positions && changed,
             "Expected contiguous CUDA tensor");
  LR_REQUIRE((reinterpret_cast<uintptr_t>(raw) & 15) == 0, "Score table must be 16-byte aligned");
  const SelectWorkspace w = carve(workspace, total, segments, count);
  LR_REQUIRE(workspace_bytes >= w.bytes, "Workspace too small");
  const hipStream_t s = as_stream(stream);
  if (int rc = launch_pool(raw, total, bounds, segments, max_count, width, pooled, w.hist,
                           kClearWords, s))
    return rc;
  return launch_sets(raw, pooled, total, segment_ends, position_starts, segments, count, w,
                     quotas, offsets, removed_positions, changed, host_info, nonfinite, true, s);
}

extern "C" int lr_select_refine_queue(const int64_t* position_starts, int64_t total,
                                      int64_t segments, int64_t count, void* workspace,
                                      size_t workspace_bytes, const int64_t* quotas,
                                      const int64_t* offsets, float* out_values,
                                      int64_t* out_segments, int64_t* out_positions,
                                      void* stream) {
  clear_error();
  LR_SELECT_CHECK_SHAPE();
  LR_REQUIRE(position_starts && workspace && quotas && offsets && out_values && out_segments &&
                 out_positions,
             "Expected contiguous CUDA tensor");
  const SelectWorkspace w = carve(workspace, total, segments, count);
  LR_REQUIRE(workspace_bytes >= w.bytes, "Workspace too small");
  return launch_queue(position_starts, segments, count, w, quotas, offsets, out_values,
                      out_segments, out_positions, as_stream(stream));
}

extern "C" int lr_select_refine(const float* raw, const float* pooled, int64_t total,
                                const int64_t* segment_ends, const int64_t* position_starts,
                                int64_t segments, int64_t count, void* workspace,
                                size_t workspace_bytes, float* out_values,
                                int64_t* out_segments, int64_t* out_positions, int64_t* quotas,
                                int64_t* offsets, int64_t* removed_positions, int64_t* changed,
                                void* stream) {
  if (int rc = lr_select_refine_sets(raw, pooled, total, segment_ends, position_starts, segments,
                                     count, workspace, workspace_bytes, quotas, offsets,
                                     removed_positions, changed, nullptr, nullptr, stream))
    return rc;
  return lr_select_refine_queue(position_starts, total, segments, count, workspace,
                                workspace_bytes, quotas, offsets, out_values, out_segments,
                                out_positions, stream);
}
