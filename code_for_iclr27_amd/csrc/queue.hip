// The lazy eviction queue on the device: what LazyController keeps between an audit and its
// evict_prefix batches (src/lazy_recall/controller.py:57-70,140-159).
//
// An audit selects `count` slots in queue order (ascending raw score, positions transplanted;
// lr_select_refine_queue) and removes only the first `immediate`; the rest stay queued and
// leave in batches (evict_prefix). A queued position was taken at audit time, so when it leaves
// it is shifted down by the number of earlier removals of the same head that lay below it:
// position - searchsorted(removed_at_audit, position), where removed_at_audit holds every
// position of that head already removed since the audit.
//
// Device state: each segment's picks sorted by position (removed_positions at offsets[s], the
// selection's removal sets) and, for each of those entries, its queue slot (`rank`, from
// lr_queue_index). The queue slots removed so far are exactly [0, begin) (a prefix), so for a
// batch of queue slots [begin, end) a segment's entries split into three kinds by rank: gone
// (< begin), leaving (in [begin, end)) and staying. One pass over the segment's entries in
// position order counts the gone ones below each leaving one (a block scan of ballots) and
// writes the leaving positions, already ascending, where lr_compact_heads reads a segment's
// removal list. No sort and no host round trip.
#include "lr_common.hpp"

namespace lr {
namespace {

constexpr int kQueueThreads = 256;
constexpr int kQueueWaves = kQueueThreads / 64;

// Queue slot j -> the slot of its position in its segment's position-sorted pick list.
__global__ __launch_bounds__(kQueueThreads) void queue_index_kernel(
    const int64_t* __restrict__ queue_segments, const int64_t* __restrict__ queue_positions,
    int64_t count, const int64_t* __restrict__ quotas, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ removed_positions, int64_t segments, int32_t* __restrict__ rank) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kQueueThreads + threadIdx.x;
  if (j >= count) return;
  const int64_t s = queue_segments[j];
  if (s < 0 || s >= segments) return;
  const int64_t position = queue_positions[j];
  const int64_t first = offsets[s], n = quotas[s];
  int64_t lo = 0, hi = n;
  while (lo < hi) {  // first entry >= position
    const int64_t mid = (lo + hi) >> 1;
    if (removed_positions[first + mid] < position) lo = mid + 1;
    else hi = mid;
  }
  if (lo < n && removed_positions[first + lo] == position) rank[first + lo] = static_cast<int32_t>(j);
}

// One workgroup per segment: its leaving entries (rank in [begin, end)), each remapped by the
// gone entries (rank < begin) below it, in position order at batch_positions[offsets[s]...].
__global__ __launch_bounds__(kQueueThreads) void queue_evict_plan_kernel(
    const int64_t* __restrict__ quotas, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ removed_positions, const int32_t* __restrict__ rank,
    int64_t begin, int64_t end, int64_t* __restrict__ batch_quotas,
    int64_t* __restrict__ batch_positions, int64_t* __restrict__ host_quotas) {
  __shared__ uint32_t wave_gone[kQueueWaves], wave_leaving[kQueueWaves];
  const int64_t s = blockIdx.x;
  const int64_t first = offsets[s], n = quotas[s];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint64_t below = (uint64_t{1} << lane) - 1;
  int64_t gone_carry = 0, leaving_carry = 0;
  for (int64_t base = 0; base < n; base += kQueueThreads) {  // uniform trip count
    const int64_t i = base + threadIdx.x;
    const bool valid = i < n;
    const int64_t r = valid ? rank[first + i] : -1;
    const int64_t position = valid ? removed_positions[first + i] : 0;
    const bool gone = valid && r < begin;
    const bool leaving = valid && r >= begin && r < end;
    const uint64_t gone_mask = __ballot(gone), leaving_mask = __ballot(leaving);
    if (lane == 0) {
      wave_gone[wave] = __popcll(gone_mask);
      wave_leaving[wave] = __popcll(leaving_mask);
    }
    __syncthreads();
    int64_t gone_before = gone_carry + __popcll(gone_mask & below);
    int64_t leaving_before = leaving_carry + __popcll(leaving_mask & below);
    for (int w = 0; w < kQueueWaves; ++w) {
      if (w < wave) {
        gone_before += wave_gone[w];
        leaving_before += wave_leaving[w];
      }
      gone_carry += wave_gone[w];
      leaving_carry += wave_leaving[w];
    }
    if (leaving) batch_positions[first + leaving_before] = position - gone_before;
    __syncthreads();  // wave_* are rewritten by the next round
  }
  if (threadIdx.x == 0) {
    batch_quotas[s] = leaving_carry;
    if (host_quotas != nullptr) host_quotas[s] = leaving_carry;
  }
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_queue_index(const int64_t* queue_segments, const int64_t* queue_positions,
                              int64_t count, const int64_t* quotas, const int64_t* offsets,
                              const int64_t* removed_positions, int64_t segments, int32_t* rank,
                              void* stream) {
  clear_error();
  LR_REQUIRE(count >= 0 && count < (int64_t{1} << 31) && segments > 0, "Invalid queue size");
  if (count == 0) return LR_OK;
  LR_REQUIRE(queue_segments && queue_positions && quotas && offsets && removed_positions && rank,
             "Expected contiguous CUDA tensor");
  const unsigned blocks = static_cast<unsigned>(ceil_div(count, kQueueThreads));
  queue_index_kernel<<<blocks, kQueueThreads, 0, as_stream(stream)>>>(
      queue_segments, queue_positions, count, quotas, offsets, removed_positions, segments, rank);
  return check_launch("queue_index");
}

extern "C" int lr_queue_evict_plan(const int64_t* quotas, const int64_t* offsets,
                                   const int64_t* removed_positions, const int32_t* rank,
                                   int64_t segments, int64_t begin, int64_t end,
                                   int64_t* batch_quotas, int64_t* batch_positions,
                                   int64_t* host_quotas, void* stream) {
  clear_error();
  LR_REQUIRE(segments > 0 && segments <= (int64_t{1} << 31) - 1, "Invalid queue size");
  LR_REQUIRE(begin >= 0 && begin <= end && end < (int64_t{1} << 31), "Invalid queue range");
  LR_REQUIRE(quotas && offsets && removed_positions && rank && batch_quotas && batch_positions,
             "Expected contiguous CUDA tensor");
  queue_evict_plan_kernel<<<static_cast<unsigned>(segments), kQueueThreads, 0, as_stream(stream)>>>(
      quotas, offsets, removed_positions, rank, begin, end, batch_quotas, batch_positions,
      host_quotas);
  return check_launch("queue_evict_plan");
}
