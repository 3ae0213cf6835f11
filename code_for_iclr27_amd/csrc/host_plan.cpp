// Host-side planning of an audit step (CPU code, built as the Python module
// code_for_iclr27_amd._plan). It validates every layer's tensors and fills the int64 metadata
// block that the HIP entry points read, in one pass over the layers:
//   [segment table: segments x LR_SEG_WORDS] [pool bounds: segments + 1] [segment ends]
//   [segment position starts] [head table: layers * heads x LR_HEAD_WORDS]
// This is the planning part of compute_score_table (src/lazy_recall/scoring.py:218-287: the
// per-(layer, KV head) candidate range [prompt_len, len - protect_recent), the head row
// offsets and the mapped query heads) and of remove_positions (src/lazy_recall/cache.py:
// 113-147: absolute rows of every head). Done from Python it costs ~27 tensor attribute
// reads per layer at ~0.2 us each; here the whole 32-layer plan takes a few microseconds.
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/extension.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <optional>
#include <stdexcept>
#include <vector>

#include "lazyrecall.h"

namespace {

void require(bool ok, const char* message) {
  if (!ok) throw std::runtime_error(message);
}

// The same checks, in the same order and with the same messages, as the Python layer checks.
void validate_layer(const torch::Tensor& k, const torch::Tensor& v, const torch::Tensor& p,
                    const torch::Tensor& q, const torch::Tensor& g, const torch::Device& device,
                    int64_t hq, int64_t window, int64_t dim, int64_t query_stride) {
  for (const torch::Tensor* t : {&k, &v, &p, &g})
    require(t->is_cuda() && t->is_contiguous() && t->device() == device,
            "Expected contiguous CUDA tensor");
  // Queries may be a window of a longer per-head history (a ring view): rows of one query head
  // are contiguous, and consecutive query heads sit query_stride rows apart.
  require(q.is_cuda() && q.device() == device, "Expected contiguous CUDA tensor");
  require(k.scalar_type() == torch::kBFloat16 && v.scalar_type() == torch::kBFloat16 &&
              q.scalar_type() == torch::kBFloat16,
          "The fused scorer takes bf16 keys, values and queries");
  require(k.dim() == 2 && k.sizes() == v.sizes() && k.size(1) == dim, "Invalid KV layout");
  require(p.scalar_type() == torch::kFloat32 && p.numel() == k.size(0), "Invalid positions");
  require(q.dim() == 3 && q.size(0) == hq && q.size(1) == window && q.size(2) == dim,
          "Historical query-head count changed");
  require(q.stride(2) == 1 && (window == 1 || q.stride(1) == dim) &&
              (hq == 1 || q.stride(0) == query_stride * dim),
          "Queries must be [Hq, W, d] with contiguous rows and one head stride for every layer");
  require(g.scalar_type() == torch::kFloat32 && g.dim() == 2 && g.size(0) == hq &&
              g.size(1) == dim,
          "Invalid margin gradient");
  for (const torch::Tensor* t : {&k, &v, &q})
    require(reinterpret_cast<uintptr_t>(t->data_ptr()) % 16 == 0,
            "bf16 operands must be 16-byte aligned");
}

inline int64_t ptr(const torch::Tensor& t) { return reinterpret_cast<int64_t>(t.data_ptr()); }

// Returns (block, meta, per-segment [layer, head, first candidate, count] int64 [4, S],
//          per-head [segment index or -1, length] int64 [2, L*H]).
// meta = (segments, groups, window, dim, max segment length, max candidates, total candidates,
//         projected floats, head slots, total rows, max head length, query stride in rows).
struct Plan {
  torch::Tensor block, segment_info, head_info;
  int64_t segments, groups, window, dim, max_seg_length, max_candidates, total, projected, slots,
      rows_total, max_head_length, layers, query_stride;
  // word offsets of the block's parts
  int64_t bounds_at() const { return segments * LR_SEG_WORDS; }
  int64_t ends_at() const { return bounds_at() + segments + 1; }
  int64_t starts_at() const { return ends_at() + segments; }
  int64_t heads_at() const { return starts_at() + segments; }
  py::tuple meta() const {
    return py::make_tuple(segments, groups, window, dim, max_seg_length, max_candidates, total,
                          projected, slots, rows_total, max_head_length, query_stride);
  }
};

Plan make_plan(const std::vector<torch::Tensor>& keys, const std::vector<torch::Tensor>& values,
               const std::vector<torch::Tensor>& positions, const std::vector<torch::Tensor>& queries,
               const std::vector<torch::Tensor>& gradients,
               const std::vector<std::vector<int64_t>>& head_lens,
               const std::vector<std::optional<std::vector<int64_t>>>& prompt_lens,
               bool protect_prompt, int64_t protect_recent, bool pinned) {
  const size_t layers = keys.size();
  require(layers > 0, "No layers to score");
  require(values.size() == layers && positions.size() == layers && queries.size() == layers &&
              gradients.size() == layers && head_lens.size() == layers &&
              prompt_lens.size() == layers,
          "Layer lists differ in length");
  require(queries[0].dim() == 3, "Historical query-head count changed");
  const int64_t hq = queries[0].size(0), window = queries[0].size(1), dim = queries[0].size(2);
  require(dim > 0 && (hq == 1 || queries[0].stride(0) % dim == 0),
          "Queries must be [Hq, W, d] with contiguous rows and one head stride for every layer");
  const int64_t query_stride = hq == 1 ? window : queries[0].stride(0) / dim;
  require(query_stride >= window,
          "Queries must be [Hq, W, d] with contiguous rows and one head stride for every layer");
  const torch::Device device = keys[0].device();
  const int64_t heads = static_cast<int64_t>(head_lens[0].size());
  require(heads > 0 && hq % heads == 0, "Query heads must be a multiple of KV heads");
  const int64_t groups = hq / heads;
  require(protect_recent >= 0, "protect_recent must be non-negative");

  // pass 1: validate, count segments
  int64_t segments = 0;
  for (size_t l = 0; l < layers; ++l) {
    validate_layer(keys[l], values[l], positions[l], queries[l], gradients[l], device, hq, window,
                   dim, query_stride);
    require(static_cast<int64_t>(head_lens[l].size()) == heads,
            "Every layer must have the same number of KV heads");
    int64_t rows = 0;
    for (int64_t n : head_lens[l]) {
      require(n >= 0, "Position/KV lengths differ");
      rows += n;
    }
    require(rows == keys[l].size(0), "Position/KV lengths differ");
    const bool has_prompt = protect_prompt && prompt_lens[l].has_value();
    if (has_prompt) require(static_cast<int64_t>(prompt_lens[l]->size()) == heads, "Invalid prompt lengths");
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t n = head_lens[l][h];
      const int64_t first = has_prompt ? (*prompt_lens[l])[h] : 0;
      require(first >= 0, "Invalid prompt lengths");
      const int64_t last = std::max(first, n - protect_recent);
      segments += last > first;
    }
  }
  require(segments > 0, "No eligible KV remains after prompt/recent protection");

  const int64_t slots = static_cast<int64_t>(layers) * heads;
  const int64_t seg_words = segments * LR_SEG_WORDS;
  const int64_t total_words = seg_words + (segments + 1) + segments + segments + slots * LR_HEAD_WORDS;
  auto options = torch::TensorOptions().dtype(torch::kInt64).pinned_memory(pinned);
  torch::Tensor block = torch::zeros({total_words}, options);
  torch::Tensor segment_info = torch::empty({4, segments}, torch::dtype(torch::kInt64));
  torch::Tensor head_info = torch::empty({2, slots}, torch::dtype(torch::kInt64));
  int64_t* table = block.data_ptr<int64_t>();
  int64_t* bounds = table + seg_words;
  int64_t* ends = bounds + segments + 1;
  int64_t* starts = ends + segments;
  int64_t* head_table = starts + segments;
  int64_t* seg_layer = segment_info.data_ptr<int64_t>();
  int64_t* seg_head = seg_layer + segments;
  int64_t* seg_first = seg_head + segments;
  int64_t* seg_count = seg_first + segments;
  int64_t* slot_segment = head_info.data_ptr<int64_t>();
  int64_t* slot_length = slot_segment + slots;

  // pass 2: fill
  int64_t s = 0, total = 0, projected = 0, max_seg_length = 0, max_candidates = 0;
  int64_t rows_total = 0, max_head_length = 0;
  bounds[0] = 0;
  for (size_t l = 0; l < layers; ++l) {
    const int64_t kp = ptr(keys[l]), vp = ptr(values[l]), pp = ptr(positions[l]);
    const int64_t qp = ptr(queries[l]), gp = ptr(gradients[l]);
    const bool has_prompt = protect_prompt && prompt_lens[l].has_value();
    int64_t base = 0;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t n = head_lens[l][h];
      const int64_t first = has_prompt ? (*prompt_lens[l])[h] : 0;
      const int64_t last = std::max(first, n - protect_recent);
      const int64_t slot = static_cast<int64_t>(l) * heads + h;
      int64_t* hrow = head_table + slot * LR_HEAD_WORDS;
      hrow[0] = kp + base * dim * 2;
      hrow[1] = vp + base * dim * 2;
      hrow[2] = pp + base * 4;
      hrow[3] = n;
      hrow[4] = -1;
      slot_segment[slot] = -1;
      slot_length[slot] = n;
      if (last > first) {
        const int64_t count = last - first;
        int64_t* row = table + s * LR_SEG_WORDS;
        row[0] = kp + base * dim * 2;
        row[1] = vp + base * dim * 2;
        row[2] = pp + base * 4;
        row[3] = qp + h * groups * query_stride * dim * 2;
        row[4] = gp + h * groups * dim * 4;
        row[5] = n;
        row[6] = first;
        row[7] = last;
        row[8] = total;
        row[9] = s * groups * window;
        row[10] = projected;
        row[11] = 0;
        total += count;
        projected += groups * n;
        bounds[s + 1] = total;
        ends[s] = total;
        starts[s] = first;
        seg_layer[s] = static_cast<int64_t>(l);
        seg_head[s] = h;
        seg_first[s] = first;
        seg_count[s] = count;
        hrow[4] = s;
        slot_segment[slot] = s;
        max_seg_length = std::max(max_seg_length, n);
        max_candidates = std::max(max_candidates, count);
        ++s;
      }
      base += n;
      max_head_length = std::max(max_head_length, n);
    }
    rows_total += base;
  }
  return Plan{block, segment_info, head_info, segments, groups, window, dim, max_seg_length,
              max_candidates, total, projected, slots, rows_total, max_head_length,
              static_cast<int64_t>(layers), query_stride};
}

py::tuple plan_audit(const std::vector<torch::Tensor>& keys, const std::vector<torch::Tensor>& values,
                     const std::vector<torch::Tensor>& positions,
                     const std::vector<torch::Tensor>& queries,
                     const std::vector<torch::Tensor>& gradients,
                     const std::vector<std::vector<int64_t>>& head_lens,
                     const std::vector<std::optional<std::vector<int64_t>>>& prompt_lens,
                     bool protect_prompt, int64_t protect_recent, bool pinned) {
  const Plan plan = make_plan(keys, values, positions, queries, gradients, head_lens, prompt_lens,
                              protect_prompt, protect_recent, pinned);
  return py::make_tuple(plan.block, plan.meta(), plan.segment_info, plan.head_info);
}

// Entry points of liblazyrecall_hip.so, bound once from Python (the addresses of the library
// that the ctypes layer loaded), so that this module needs no link-time dependency on it.
struct Library {
  decltype(&lr_score_workspace_bytes) score_workspace_bytes = nullptr;
  decltype(&lr_score_segments) score_segments = nullptr;
  decltype(&lr_pool) pool = nullptr;
  decltype(&lr_select_workspace_bytes) select_workspace_bytes = nullptr;
  decltype(&lr_pool_select_refine_sets) pool_select_refine_sets = nullptr;
  decltype(&lr_select_refine_queue) select_refine_queue = nullptr;
  decltype(&lr_queue_index) queue_index = nullptr;
  decltype(&lr_queue_evict_plan) queue_evict_plan = nullptr;
  decltype(&lr_compact_heads_layout) compact_heads = nullptr;
  decltype(&lr_append) append = nullptr;
  decltype(&lr_compact) compact = nullptr;
  decltype(&lr_append_layers) append_layers = nullptr;
  decltype(&lr_append_layers_host) append_layers_host = nullptr;
  decltype(&lr_batch_append) batch_append = nullptr;
  decltype(&lr_batch_append_host) batch_append_host = nullptr;
  decltype(&lr_packed_attention) packed_attention = nullptr;
  decltype(&lr_packed_attention_workspace_bytes) attention_workspace_bytes = nullptr;
  decltype(&lr_packed_attention_pending) packed_attention_pending = nullptr;
  decltype(&lr_packed_attention_pending_workspace_bytes) pending_workspace_bytes = nullptr;
  decltype(&lr_last_error) last_error = nullptr;
  decltype(&lr_staging_alloc) staging_alloc = nullptr;
  decltype(&lr_staging_free) staging_free = nullptr;
  decltype(&lr_copy_words) copy_words = nullptr;
  decltype(&lr_reinsert_group) reinsert_group = nullptr;
  decltype(&lr_reinsert_plan_layout) reinsert_plan_layout = nullptr;
  decltype(&lr_reinsert_resident) reinsert_resident = nullptr;
  decltype(&lr_reinsert_recalled) reinsert_recalled = nullptr;
};
Library library;

template <typename F>
void bind_one(F& slot, int64_t address) {
  require(address != 0, "null entry point");
  slot = reinterpret_cast<F>(static_cast<uintptr_t>(address));
}

void bind_library(int64_t score_workspace_bytes, int64_t score_segments, int64_t pool,
                  int64_t select_workspace_bytes, int64_t pool_select_refine_sets,
                  int64_t select_refine_queue, int64_t queue_index, int64_t queue_evict_plan,
                  int64_t compact_heads, int64_t last_error, int64_t staging_alloc,
                  int64_t staging_free, int64_t copy_words) {
  bind_one(library.score_workspace_bytes, score_workspace_bytes);
  bind_one(library.score_segments, score_segments);
  bind_one(library.pool, pool);
  bind_one(library.select_workspace_bytes, select_workspace_bytes);
  bind_one(library.pool_select_refine_sets, pool_select_refine_sets);
  bind_one(library.select_refine_queue, select_refine_queue);
  bind_one(library.queue_index, queue_index);
  bind_one(library.queue_evict_plan, queue_evict_plan);
  bind_one(library.compact_heads, compact_heads);
  bind_one(library.last_error, last_error);
  bind_one(library.staging_alloc, staging_alloc);
  bind_one(library.staging_free, staging_free);
  bind_one(library.copy_words, copy_words);
}

void bind_data_movement(int64_t append, int64_t compact, int64_t append_layers,
                        int64_t batch_append, int64_t batch_append_host,
                        int64_t append_layers_host) {
  bind_one(library.append, append);
  bind_one(library.compact, compact);
  bind_one(library.append_layers, append_layers);
  bind_one(library.batch_append, batch_append);
  bind_one(library.batch_append_host, batch_append_host);
  bind_one(library.append_layers_host, append_layers_host);
}

void bind_reinsert(int64_t group, int64_t plan_layout, int64_t resident, int64_t recalled) {
  bind_one(library.reinsert_group, group);
  bind_one(library.reinsert_plan_layout, plan_layout);
  bind_one(library.reinsert_resident, resident);
  bind_one(library.reinsert_recalled, recalled);
}

void bind_attention(int64_t packed_attention, int64_t workspace_bytes, int64_t pending,
                    int64_t pending_workspace_bytes) {
  bind_one(library.packed_attention, packed_attention);
  bind_one(library.attention_workspace_bytes, workspace_bytes);
  bind_one(library.packed_attention_pending, pending);
  bind_one(library.pending_workspace_bytes, pending_workspace_bytes);
}

void check_call(int status) {
  if (status != LR_OK) throw std::runtime_error(library.last_error());
}

inline void* dptr(const torch::Tensor& t) { return t.data_ptr(); }

// Small per-call metadata blocks (batch_append's descriptors) go to the device the way the
// audit's block does: written into a pinned, host-coherent staging buffer that a kernel reads in
// place, or that a copy kernel (lr_copy_words) copies on the caller's stream, not by a
// copy-engine transfer. A ring of buffers per device lets consecutive calls (one per layer in a
// decode step) proceed without waiting: a buffer is rewritten only after an event recorded
// behind the work that reads it, which for a ring this long has long completed. One event
// covers up to kGroup consecutive buffers used on one stream (recorded behind the last of them):
// an event per call put an extra barrier between every two dependent kernels (batch_append
// 34.4 against 30.2 us per call on a held stream). The buffers start as 64 KB shares of one
// allocation made at the ring's first use (a pinned allocation costs 75-85 us of host time, and a
// per-slot first allocation put one on the critical path of each of the first 64 calls); a
// larger block gets a buffer of its own, grown to at least twice the old size. The rings live
// until the process ends (their pinned memory is released with it), so no buffer is freed while
// the runtime shuts down.
struct StagingRing {
  static constexpr size_t kSlots = 64;
  static constexpr size_t kGroup = 8;
  static constexpr size_t kSlotBytes = size_t{64} << 10;
  struct Slot {
    void* host = nullptr;
    size_t bytes = 0;
    bool owned = false;    // a buffer of its own (else a share of `shared`)
    c10::Event done{c10::DeviceType::CUDA};
    bool pending = false;  // enqueued work may still read the buffer
    size_t cover = 0;      // the slot whose `done` event follows that work
  };
  void* shared = nullptr;  // kSlots * kSlotBytes
  std::vector<Slot> slots{kSlots};
  size_t next = 0;
  // Pending slots that no recorded event follows yet, in ring order, all used on `open_stream`.
  std::vector<size_t> open;
  c10::Stream open_stream{c10::Stream::DEFAULT, c10::Device(c10::DeviceType::CUDA, 0)};

  // Records the last open slot's event behind every open slot's work. A covering slot is the
  // last of its group in ring order, so the group's other slots are settled before it is reused
  // and its event recorded again.
  void cover() {
    if (open.empty()) return;
    const size_t last = open.back();
    slots[last].done.record(open_stream);
    for (size_t j : open) slots[j].cover = last;
    open.clear();
  }
  // Waits until no enqueued work reads slot i.
  void settle(size_t i) {
    Slot& slot = slots[i];
    if (!slot.pending) return;
    if (std::find(open.begin(), open.end(), i) != open.end()) cover();
    slots[slot.cover].done.synchronize();
    slot.pending = false;
  }
  // Slot i is read by work just enqueued on `stream`.
  void mark(size_t i, const c10::Stream& stream) {
    if (!open.empty() && stream != open_stream) cover();
    open.push_back(i);
    open_stream = stream;
    slots[i].pending = true;
    if (open.size() >= kGroup) cover();
  }
  void* fill(size_t i, const int64_t* words, int64_t count) {
    if (shared == nullptr) {
      check_call(library.staging_alloc(kSlots * kSlotBytes, &shared));
      for (size_t j = 0; j < kSlots; ++j) {
        slots[j].host = static_cast<char*>(shared) + j * kSlotBytes;
        slots[j].bytes = kSlotBytes;
      }
    }
    Slot& slot = slots[i];
    settle(i);
    const size_t bytes = static_cast<size_t>(count) * sizeof(int64_t);
    if (slot.bytes < bytes) {
      const size_t grown = std::max(bytes, 2 * slot.bytes);
      if (slot.owned) check_call(library.staging_free(slot.host));
      slot.host = nullptr;
      slot.bytes = 0;
      slot.owned = false;
      check_call(library.staging_alloc(grown, &slot.host));
      slot.bytes = grown;
      slot.owned = true;
    }
    std::memcpy(slot.host, words, bytes);
    return slot.host;
  }

  // The next buffer, holding `count` words, for a kernel that reads them in place (pinned,
  // host-coherent memory); release() must follow once that kernel is enqueued.
  int64_t* stage(const int64_t* words, int64_t count) {
    return static_cast<int64_t*>(fill(next, words, count));
  }
  // Marks the buffer stage() returned as read by the work enqueued so far on the device's
  // current stream, and moves to the next buffer.
  void release(const torch::Device& device) {
    mark(next, c10::impl::getDeviceGuardImpl(c10::DeviceType::CUDA)->getStream(device));
    next = (next + 1) % kSlots;
  }

  torch::Tensor upload(const int64_t* words, int64_t count, const torch::Device& device,
                       void* stream) {
    const size_t i = next;
    next = (next + 1) % kSlots;
    const void* host = fill(i, words, count);
    torch::Tensor block =
        torch::empty({count}, torch::TensorOptions().device(device).dtype(torch::kInt64));
    check_call(library.copy_words(static_cast<const int64_t*>(host), block.data_ptr<int64_t>(),
                                  count, stream));
    mark(i, c10::impl::getDeviceGuardImpl(c10::DeviceType::CUDA)->getStream(device));
    return block;
  }
};

StagingRing& staging_ring(const torch::Device& device) {
  static std::vector<StagingRing*> rings;
  const size_t index = static_cast<size_t>(device.index() < 0 ? 0 : device.index());
  if (rings.size() <= index) rings.resize(index + 1, nullptr);
  if (rings[index] == nullptr) rings[index] = new StagingRing();  // kept until exit, see above
  return *rings[index];
}

// The recall archive's hook of a fused layout change (None: no transport): called with the
// device addresses of the head table and of the removal sets the compaction is about to read,
// so that the removed rows are packed for the archive before the compaction is enqueued, as
// remove_positions calls record_evicted first (src/lazy_recall/cache.py:110-112). Arguments:
// (head table, slots, heads per layer, quotas, offsets, positions, rows removed, most rows
// removed from one slot).
void archive_removals(const py::object& archive, const int64_t* head_table, int64_t slots,
                      int64_t heads_per_layer, const int64_t* quotas, const int64_t* offsets,
                      const int64_t* positions, int64_t count, int64_t max_rows) {
  if (archive.is_none() || count <= 0) return;
  auto address = [](const void* p) { return static_cast<int64_t>(reinterpret_cast<uintptr_t>(p)); };
  archive(address(head_table), slots, heads_per_layer, address(quotas), address(offsets),
          address(positions), count, max_rows);
}

// Device block for the per-layer metadata a compaction or reinsertion writes: the new length
// of every (layer, head) slot (i32 [layers * heads]), then each layer's cumulative lengths
// (i32 [layers, heads + 1]). Views of it are what the reference keeps as metadata.head_lens and
// metadata.cu_seqlens_k (src/lazy_recall/cache.py:171-177).
torch::Tensor new_layout(int64_t layers, int64_t heads, const torch::Device& device) {
  return torch::empty({layers * heads + layers * (heads + 1)},
                      torch::TensorOptions().device(device).dtype(torch::kInt32));
}

// The host side of an audit step's two copies and its one wait.
//  - upload(): the metadata block goes through the device's staging ring (pinned, host-coherent
//    buffers, one event per group of buffers) and a copy kernel (lr_copy_words) on the step's
//    stream, so the upload costs one small kernel between the previous work and the step's
//    first kernel, not a copy-engine round trip (measured ~19 us of idle GPU between two
//    steps), and no event of its own between that kernel and the next.
//  - info_buffer() / post(): the per-segment quotas and the non-finite score count are final
//    once the selection kernels are done; the selection's plan workgroup writes them straight
//    into this object's host-coherent `info` buffer (no copy), and post() records `ready`
//    right after the selection, before the compaction is enqueued.
// wait() blocks on `ready` only and builds the new ragged layout while the compaction still
// runs. One object serves one step at a time (an AuditStep keeps one per device); each step's
// wait() must return before the next audit_launch with the same object.
struct StepSync {
  c10::Event ready{c10::DeviceType::CUDA};
  int64_t* info = nullptr;  // host-coherent int64 [segments + 1], written by the device
  size_t info_bytes = 0;
  std::vector<int64_t> slot_segment, slot_length;   // per (layer, head): segment or -1, length
  int64_t layers = 0, heads = 0, segments = 0;
  bool pending = false;
  bool subtract = true;  // heads lose info[segment] rows (false: the step removed nothing)

  StepSync() = default;
  StepSync(const StepSync&) = delete;
  StepSync& operator=(const StepSync&) = delete;
  ~StepSync() {
    if (pending) ready.synchronize();
    if (info != nullptr) library.staging_free(info);
  }

  // The buffer the step's selection writes into. A step's wait() (or the destructor) has seen
  // the previous writer finish before a new step gets it.
  int64_t* info_buffer(int64_t words) {
    require(!pending, "the previous audit step on this StepSync was not waited for");
    const size_t bytes = static_cast<size_t>(words) * sizeof(int64_t);
    if (info_bytes < bytes) {
      if (info != nullptr) check_call(library.staging_free(info));
      info = nullptr;
      info_bytes = 0;
      void* memory = nullptr;
      check_call(library.staging_alloc(bytes, &memory));
      info = static_cast<int64_t*>(memory);
      info_bytes = bytes;
    }
    return info;
  }

  torch::Tensor upload(const torch::Tensor& words, const torch::Device& device, void* stream) {
    return staging_ring(device).upload(words.data_ptr<int64_t>(), words.numel(), device, stream);
  }

  // Records `ready` and keeps what wait() needs: each head slot's segment (or -1) and length.
  // With removes = false the step removes nothing (every head keeps its length).
  void post_slots(const int64_t* segment_of_slot, const int64_t* length_of_slot, int64_t slots,
                  int64_t layer_count, int64_t segment_count, bool removes,
                  const torch::Device& device) {
    ready.record(c10::impl::getDeviceGuardImpl(c10::DeviceType::CUDA)->getStream(device));
    slot_segment.assign(segment_of_slot, segment_of_slot + slots);
    slot_length.assign(length_of_slot, length_of_slot + slots);
    layers = layer_count;
    heads = slots / layer_count;
    segments = segment_count;
    subtract = removes;
    pending = true;
  }

  // Drops a posted step whose launch sequence failed after post(): waits for its selection
  // (which writes `info`) so that the buffers may be reused.
  void abandon() {
    if (!pending) return;
    pending = false;
    py::gil_scoped_release release;
    ready.synchronize();
  }

  void post(const Plan& plan, const torch::Device& device, bool removes = true) {
    const int64_t* slot = plan.head_info.data_ptr<int64_t>();
    post_slots(slot, slot + plan.slots, plan.slots, plan.layers, plan.segments, removes, device);
  }

  // Waits for the selection, refuses non-finite scores (scoring.py:292-293's message), and
  // returns (rows kept per head as [L][H] lists, row offset of each layer in the packed
  // output [L + 1]).
  py::tuple wait(bool check_finite) {
    require(pending, "no audit step is pending on this StepSync");
    pending = false;
    {
      py::gil_scoped_release release;
      ready.synchronize();
    }
    int32_t bad = 0;
    std::memcpy(&bad, info + segments, sizeof(bad));
    if (check_finite && bad != 0)
      throw std::runtime_error(
          "LazyRecall produced non-finite scores; refusing to construct a deletion queue");
    py::list kept(layers);
    py::list offsets(layers + 1);
    int64_t row = 0;
    offsets[0] = py::int_(0);
    for (int64_t l = 0; l < layers; ++l) {
      py::list lengths(heads);
      for (int64_t h = 0; h < heads; ++h) {
        const int64_t slot = l * heads + h;
        const int64_t s = slot_segment[slot];
        const int64_t n = slot_length[slot] - (subtract && s >= 0 ? info[s] : 0);
        lengths[h] = py::int_(n);
        row += n;
      }
      kept[l] = lengths;
      offsets[l + 1] = py::int_(row);
    }
    return py::make_tuple(kept, offsets);
  }
};

// One whole audit step on the device (controller.py:140-159): plan, one metadata upload, fused
// scores, Pool7, the removal sets of the allocation-preserving selection and the compaction of
// every layer, all enqueued on `stream` from here (no Python between the launches). Returns
// (plan block, meta, segment_info, head_info, scores [2*total] (raw then pooled), info i64
// [S+1] (quotas, then the non-finite score count as i32), quotas, offsets, removed positions,
// changed, out keys, out values, out positions, the block on the device, the selection
// workspace (for the queue order, lr_select_refine_queue), queue). count is clamped to
// [0, total]; with count 0 nothing is selected and the layers are copied as they are.
// immediate < 0 or >= count removes every selected slot (queue None). 0 <= immediate < count is
// the lazy form: the queue order is computed on `stream`, only its first `immediate` slots are
// removed (none: the out tensors are undefined and the layers stay as they are), and queue =
// (values f32 [count], segments then positions i64 [2 * count], rank i32 [count]) is the device
// state lr_queue_evict_plan needs for the rest (with quotas, offsets and removed positions).
// `mark` (None or a callable) is called with a stage name after each stage's launches and with
// "start" before the first (then the scorer is launched stage by stage), for event timing.
// `sync` (or None) receives the quota copy and its event between the selection and the
// compaction (StepSync above). `stream_handle` must be torch's current stream on the layers'
// device: the kernels go to it, and the quota copy and the event go to torch's current stream.
py::tuple audit_launch(const std::vector<torch::Tensor>& keys,
                       const std::vector<torch::Tensor>& values,
                       const std::vector<torch::Tensor>& positions,
                       const std::vector<torch::Tensor>& queries,
                       const std::vector<torch::Tensor>& gradients,
                       const std::vector<std::vector<int64_t>>& head_lens,
                       const std::vector<std::optional<std::vector<int64_t>>>& prompt_lens,
                       int64_t protect_recent, const torch::Tensor& query_positions,
                       const torch::Tensor& margin, int64_t count, int64_t immediate,
                       int64_t pool_kernel, double epsilon, int64_t stream_handle,
                       const py::object& mark, StepSync* sync, const py::object& archive,
                       bool order_queue) {
  require(library.score_segments != nullptr, "library entry points are not bound");
  require(pool_kernel > 0 && pool_kernel % 2 == 1, "pool kernel must be a positive odd integer");
  // with a StepSync the block goes through its staging buffer, so it need not be pinned
  const Plan plan = make_plan(keys, values, positions, queries, gradients, head_lens, prompt_lens,
                              true, protect_recent, /*pinned=*/sync == nullptr);
  const torch::Device device = keys[0].device();
  require(query_positions.is_cuda() && query_positions.device() == device &&
              query_positions.scalar_type() == torch::kInt64 && query_positions.is_contiguous() &&
              query_positions.numel() == plan.window,
          "Query positions do not match the window");
  require(margin.is_cuda() && margin.device() == device && margin.scalar_type() == torch::kFloat32 &&
              margin.numel() == 1,
          "Invalid base margin");
  void* stream = reinterpret_cast<void*>(static_cast<uintptr_t>(stream_handle));
  const auto on_device = torch::TensorOptions().device(device);
  const int64_t S = plan.segments;
  count = std::min(std::max<int64_t>(count, 0), plan.total);
  // controller.py:151-153: the selection must cover the slots the budget removes now
  require(immediate <= count, "Not enough unprotected candidates to enforce the budget");

  // The step's first buffers are allocated before the upload, so that its copy kernel and the
  // first scorer kernel are launched back to back (the copy takes less time than the host
  // between the two launches otherwise).
  // quotas (written for every segment by the selection) and the non-finite count (cleared by
  // the first scorer kernel) come back in one small copy
  torch::Tensor info = count > 0 ? torch::empty({S + 1}, on_device.dtype(torch::kInt64))
                                 : torch::zeros({S + 1}, on_device.dtype(torch::kInt64));
  int32_t* nonfinite = reinterpret_cast<int32_t*>(info.data_ptr<int64_t>() + S);

  const size_t score_bytes =
      library.score_workspace_bytes(S, plan.groups, plan.window, S * plan.groups * plan.max_seg_length);
  torch::Tensor score_ws = torch::empty({static_cast<int64_t>(score_bytes)}, on_device.dtype(torch::kUInt8));
  torch::Tensor scores = torch::empty({2 * plan.total}, on_device.dtype(torch::kFloat32));
  float* raw = scores.data_ptr<float>();
  float* pooled = raw + plan.total;
  torch::Tensor block = sync != nullptr ? sync->upload(plan.block, device, stream)
                                        : plan.block.to(device, /*non_blocking=*/true);
  const int64_t* words = block.data_ptr<int64_t>();
  const bool timed = !mark.is_none();
  auto stage = [&](const char* name) {
    if (timed) mark(name);
  };
  static const char* kScoreStages[3] = {"projected_values", "row_stats", "column_scores"};
  stage("start");
  for (int i = 0; i < (timed ? 3 : 1); ++i) {
    check_call(library.score_segments(
        words, S, plan.groups, plan.window, plan.dim, plan.max_seg_length, plan.max_candidates,
        plan.query_stride, query_positions.data_ptr<int64_t>(), margin.data_ptr<float>(),
        static_cast<float>(1.0 / std::sqrt(static_cast<double>(plan.dim))), epsilon,
        dptr(score_ws), score_bytes, raw, nonfinite, timed ? 1 << i : 7, stream));
    stage(timed ? kScoreStages[i] : "score");
  }
  // With a selection to make, the pool runs inside lr_pool_select_refine_sets (its launch also
  // resets the selection's counters); the "select" stage then covers both.
  if (count <= 0) {
    check_call(library.pool(raw, plan.total, words + plan.bounds_at(), S, plan.max_candidates,
                            pool_kernel, pooled, stream));
    stage("pool");
  }

  // The lazy form: only the queue's first `immediate` slots leave now, the rest stay queued
  // (controller.py:148-158). It needs the queue order before the compaction.
  const bool lazy = count > 0 && immediate >= 0 && immediate < count;
  const int64_t out_rows = plan.rows_total - (lazy ? immediate : count);
  const auto kv = on_device.dtype(keys[0].scalar_type());
  torch::Tensor out_keys, out_values, out_positions;
  if (!lazy || immediate > 0) {
    out_keys = torch::empty({out_rows, plan.dim}, kv);
    out_values = torch::empty({out_rows, plan.dim}, kv);
    out_positions = torch::empty({out_rows}, on_device.dtype(torch::kFloat32));
  }
  torch::Tensor sets, quotas, offsets, removed, changed, select_ws;
  torch::Tensor queue_values, queue_order, queue_rank, batch;
  torch::Tensor queue_order_out;  // the eager step's queue order (order_queue)
  torch::Tensor layout;  // device i32: head lengths [slots], then cumulative [layers, H + 1]
  if (lazy) {
    const size_t select_bytes = library.select_workspace_bytes(plan.total, S, count);
    select_ws = torch::empty({static_cast<int64_t>(select_bytes)}, on_device.dtype(torch::kUInt8));
    sets = torch::empty({count + 2 * S + 1}, on_device.dtype(torch::kInt64));
    quotas = info.narrow(0, 0, S);
    removed = sets.narrow(0, 0, count);
    offsets = sets.narrow(0, count, S + 1);
    changed = sets.narrow(0, count + S + 1, S);
    queue_values = torch::empty({count}, on_device.dtype(torch::kFloat32));
    queue_order = torch::empty({2 * count}, on_device.dtype(torch::kInt64));
    queue_rank = torch::empty({count}, on_device.dtype(torch::kInt32));
    batch = torch::empty({count + S}, on_device.dtype(torch::kInt64));
    int64_t* host = sync != nullptr ? sync->info_buffer(S + 1) : nullptr;
    check_call(library.pool_select_refine_sets(
        raw, plan.total, words + plan.bounds_at(), plan.max_candidates, pool_kernel, pooled,
        words + plan.ends_at(), words + plan.starts_at(), S, count, dptr(select_ws), select_bytes,
        quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(), removed.data_ptr<int64_t>(),
        changed.data_ptr<int64_t>(), host, nonfinite, stream));
    int64_t* queue_segments = queue_order.data_ptr<int64_t>();
    int64_t* queue_positions = queue_segments + count;
    check_call(library.select_refine_queue(
        words + plan.starts_at(), plan.total, S, count, dptr(select_ws), select_bytes,
        quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(), queue_values.data_ptr<float>(),
        queue_segments, queue_positions, stream));
    check_call(library.queue_index(queue_segments, queue_positions, count,
                                   quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(),
                                   removed.data_ptr<int64_t>(), S, queue_rank.data_ptr<int32_t>(),
                                   stream));
    int64_t* batch_positions = batch.data_ptr<int64_t>();
    int64_t* batch_quotas = batch_positions + count;
    if (immediate > 0)
      check_call(library.queue_evict_plan(
          quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(), removed.data_ptr<int64_t>(),
          queue_rank.data_ptr<int32_t>(), S, 0, immediate, batch_quotas, batch_positions, host,
          stream));
    stage("select");
    if (sync != nullptr) sync->post(plan, device, /*removes=*/immediate > 0);
    if (immediate > 0) {  // with nothing to remove now the layers stay as they are
      try {
        archive_removals(archive, words + plan.heads_at(), plan.slots, plan.slots / plan.layers,
                         batch_quotas, offsets.data_ptr<int64_t>(), batch_positions, immediate,
                         std::min(immediate, plan.max_candidates));
      } catch (...) {
        if (sync != nullptr) sync->abandon();
        throw;
      }
      layout = new_layout(plan.layers, plan.slots / plan.layers, device);
      check_call(library.compact_heads(
          words + plan.heads_at(), plan.slots, batch_quotas, offsets.data_ptr<int64_t>(),
          batch_positions, plan.dim, static_cast<int>(keys[0].element_size()),
          plan.max_head_length, out_rows, dptr(out_keys), dptr(out_values),
          out_positions.data_ptr<float>(), plan.slots / plan.layers,
          layout.data_ptr<int32_t>(), layout.data_ptr<int32_t>() + plan.slots, stream));
      stage("compact");
    }
  } else if (count > 0) {
    const size_t select_bytes = library.select_workspace_bytes(plan.total, S, count);
    select_ws = torch::empty({static_cast<int64_t>(select_bytes)}, on_device.dtype(torch::kUInt8));
    sets = torch::empty({count + 2 * S + 1}, on_device.dtype(torch::kInt64));
    quotas = info.narrow(0, 0, S);
    removed = sets.narrow(0, 0, count);
    offsets = sets.narrow(0, count, S + 1);
    changed = sets.narrow(0, count + S + 1, S);
    check_call(library.pool_select_refine_sets(
        raw, plan.total, words + plan.bounds_at(), plan.max_candidates, pool_kernel, pooled,
        words + plan.ends_at(), words + plan.starts_at(), S, count, dptr(select_ws), select_bytes,
        quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(), removed.data_ptr<int64_t>(),
        changed.data_ptr<int64_t>(), sync != nullptr ? sync->info_buffer(S + 1) : nullptr,
        nonfinite, stream));
    stage("select");
    if (sync != nullptr) sync->post(plan, device);
    if (order_queue) {
      // the eviction queue's order too (every selected slot leaves now, so the removal sets do
      // not depend on it): on this stream, before the compaction
      queue_values = torch::empty({count}, on_device.dtype(torch::kFloat32));
      queue_order_out = torch::empty({2 * count}, on_device.dtype(torch::kInt64));
      int64_t* queue_segments = queue_order_out.data_ptr<int64_t>();
      check_call(library.select_refine_queue(
          words + plan.starts_at(), plan.total, S, count, dptr(select_ws), select_bytes,
          quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(), queue_values.data_ptr<float>(),
          queue_segments, queue_segments + count, stream));
      stage("queue");
    }
    try {
      archive_removals(archive, words + plan.heads_at(), plan.slots, plan.slots / plan.layers,
                       quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(),
                       removed.data_ptr<int64_t>(), count, std::min(count, plan.max_candidates));
    } catch (...) {
      if (sync != nullptr) sync->abandon();
      throw;
    }
    layout = new_layout(plan.layers, plan.slots / plan.layers, device);
    check_call(library.compact_heads(
        words + plan.heads_at(), plan.slots, quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(),
        removed.data_ptr<int64_t>(), plan.dim, static_cast<int>(keys[0].element_size()),
        plan.max_head_length, out_rows, dptr(out_keys), dptr(out_values),
        out_positions.data_ptr<float>(), plan.slots / plan.layers, layout.data_ptr<int32_t>(),
        layout.data_ptr<int32_t>() + plan.slots, stream));
    stage("compact");
  } else {
    if (sync != nullptr) {
      // no selection: the non-finite count (and zero quotas) go to the host buffer by a copy kernel
      check_call(library.copy_words(info.data_ptr<int64_t>(), sync->info_buffer(S + 1), S + 1,
                                    stream));
      sync->post(plan, device);
    }
    std::vector<torch::Tensor> flat_positions;
    for (const torch::Tensor& p : positions) flat_positions.push_back(p.reshape({-1}));
    out_keys.copy_(torch::cat(keys));
    out_values.copy_(torch::cat(values));
    out_positions.copy_(torch::cat(flat_positions));
  }
  py::object queue = py::none();
  if (lazy) queue = py::make_tuple(queue_values, queue_order, queue_rank);
  else if (queue_order_out.defined()) queue = py::make_tuple(queue_values, queue_order_out);
  py::object layout_out = py::none();
  if (layout.defined()) layout_out = py::cast(layout);
  return py::make_tuple(plan.block, plan.meta(), plan.segment_info, plan.head_info, scores, info,
                        quotas, offsets, removed, changed, out_keys, out_values, out_positions,
                        block, select_ws, queue, layout_out);
}

// One evict_prefix batch (controller.py:57-70) on the device: removes the queued slots
// [begin, end) of an audit's lazy queue from the layers as they are now (the audit's own
// removals done, tokens appended since at the end of each head). The queue state is the
// audit's (quotas, offsets, removed positions, rank; lr_queue_evict_plan) plus a host copy of
// the queue's segment ids (`segments_host`, CPU int64 [count], queue order), from which the
// batch's per-segment counts and so the new layout are known here without waiting for the
// device. slot_segment maps each (layer, head) slot to its score segment or -1, as at the audit.
// Enqueues on `stream`: the head-table upload (sync's staging buffer), the plan (remapped
// positions) and one compaction of every layer; nothing here waits for them. Returns (out keys,
// out values, out positions, rows kept per head [L][H], row offset of each layer [L + 1]).
py::tuple queue_evict_launch(const std::vector<torch::Tensor>& keys,
                             const std::vector<torch::Tensor>& values,
                             const std::vector<torch::Tensor>& positions,
                             const std::vector<std::vector<int64_t>>& head_lens,
                             const std::vector<int64_t>& slot_segment, const torch::Tensor& quotas,
                             const torch::Tensor& offsets, const torch::Tensor& removed,
                             const torch::Tensor& rank, const torch::Tensor& segments_host,
                             int64_t begin, int64_t end, int64_t stream_handle, StepSync* sync,
                             const std::vector<int64_t>& packed_offsets,
                             const py::object& archive) {
  require(library.queue_evict_plan != nullptr, "library entry points are not bound");
  require(sync != nullptr, "an evict_prefix batch needs a StepSync");
  // Packed form (an audit's or a batch's own output): one K, V and positions tensor holding
  // every layer, layer l at rows [packed_offsets[l], packed_offsets[l + 1]).
  const bool packed = !packed_offsets.empty();
  const size_t layers = packed ? packed_offsets.size() - 1 : keys.size();
  require(layers > 0 && head_lens.size() == layers &&
              (packed ? keys.size() == 1 && values.size() == 1 && positions.size() == 1
                      : values.size() == layers && positions.size() == layers),
          "Layer lists differ in length");
  const int64_t heads = static_cast<int64_t>(head_lens[0].size());
  const int64_t slots = static_cast<int64_t>(layers) * heads;
  require(heads > 0 && static_cast<int64_t>(slot_segment.size()) == slots,
          "The queue belongs to a cache of another shape");
  const int64_t S = quotas.numel();
  const torch::Device device = keys[0].device();
  for (const torch::Tensor* t : {&quotas, &offsets, &removed})
    require(t->is_cuda() && t->device() == device && t->is_contiguous() &&
                t->scalar_type() == torch::kInt64,
            "Invalid queue state");
  require(rank.is_cuda() && rank.device() == device && rank.is_contiguous() &&
              rank.scalar_type() == torch::kInt32 && rank.numel() == removed.numel() &&
              offsets.numel() == S + 1,
          "Invalid queue state");
  require(!segments_host.is_cuda() && segments_host.is_contiguous() &&
              segments_host.scalar_type() == torch::kInt64 &&
              segments_host.numel() == removed.numel(),
          "Invalid queue state");
  require(0 <= begin && begin <= end && end <= removed.numel(), "Discard queue underflow");
  // the batch's slots per segment, from the host copy of the queue order
  std::vector<int64_t> leaving(static_cast<size_t>(S), 0);
  const int64_t* queue_segments = segments_host.data_ptr<int64_t>();
  for (int64_t j = begin; j < end; ++j) {
    const int64_t segment = queue_segments[j];
    require(segment >= 0 && segment < S, "Invalid queue state");
    ++leaving[segment];
  }
  const int64_t dim = keys[0].dim() == 2 ? keys[0].size(1) : 0;
  const auto dtype = keys[0].scalar_type();
  torch::Tensor table = torch::empty({slots * LR_HEAD_WORDS}, torch::TensorOptions().dtype(torch::kInt64));
  int64_t* rows = table.data_ptr<int64_t>();
  py::list kept(layers), layer_offsets(layers + 1);
  layer_offsets[0] = py::int_(0);
  int64_t rows_total = 0, out_rows = 0, max_length = 0;
  for (size_t l = 0; l < layers; ++l) {
    const size_t t_index = packed ? 0 : l;
    const torch::Tensor &k = keys[t_index], &v = values[t_index], &p = positions[t_index];
    if (!packed || l == 0) {
      for (const torch::Tensor* t : {&k, &v, &p})
        require(t->is_cuda() && t->is_contiguous() && t->device() == device,
                "Expected contiguous CUDA tensor");
      require(k.dim() == 2 && k.sizes() == v.sizes() && k.size(1) == dim && dim > 0 &&
                  k.scalar_type() == dtype && v.scalar_type() == dtype,
              "Invalid KV layout");
      require(p.scalar_type() == torch::kFloat32 && p.numel() == k.size(0), "Invalid positions");
    }
    const int64_t first_row = packed ? packed_offsets[l] : 0;
    const int64_t layer_rows = packed ? packed_offsets[l + 1] - first_row : k.size(0);
    require(first_row >= 0 && layer_rows >= 0 && first_row + layer_rows <= k.size(0),
            "Position/KV lengths differ");
    require(static_cast<int64_t>(head_lens[l].size()) == heads,
            "Every layer must have the same number of KV heads");
    py::list lengths(heads);
    int64_t base = first_row;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t n = head_lens[l][h];
      require(n >= 0, "Position/KV lengths differ");
      const int64_t slot = static_cast<int64_t>(l) * heads + h;
      const int64_t segment = slot_segment[slot];
      require(segment >= -1 && segment < S, "The queue belongs to a cache of another shape");
      const int64_t gone = segment >= 0 ? leaving[segment] : 0;
      require(gone <= n, "The queue belongs to a cache of another shape");
      int64_t* row = rows + slot * LR_HEAD_WORDS;
      row[0] = ptr(k) + base * dim * static_cast<int64_t>(k.element_size());
      row[1] = ptr(v) + base * dim * static_cast<int64_t>(v.element_size());
      row[2] = ptr(p) + base * 4;
      row[3] = n;
      row[4] = segment;
      row[5] = 0;
      lengths[h] = py::int_(n - gone);
      out_rows += n - gone;
      base += n;
      max_length = std::max(max_length, n);
    }
    require(base == first_row + layer_rows, "Position/KV lengths differ");
    rows_total += layer_rows;
    kept[l] = lengths;
    layer_offsets[l + 1] = py::int_(out_rows);
  }
  void* stream = reinterpret_cast<void*>(static_cast<uintptr_t>(stream_handle));
  const auto on_device = torch::TensorOptions().device(device);
  torch::Tensor head_table = sync->upload(table, device, stream);
  const int64_t count = removed.numel();
  torch::Tensor batch = torch::empty({count + S}, on_device.dtype(torch::kInt64));
  int64_t* batch_positions = batch.data_ptr<int64_t>();
  int64_t* batch_quotas = batch_positions + count;
  check_call(library.queue_evict_plan(quotas.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(),
                                      removed.data_ptr<int64_t>(), rank.data_ptr<int32_t>(), S,
                                      begin, end, batch_quotas, batch_positions, nullptr, stream));
  const auto kv = on_device.dtype(dtype);
  torch::Tensor out_keys = torch::empty({out_rows, dim}, kv);
  torch::Tensor out_values = torch::empty({out_rows, dim}, kv);
  torch::Tensor out_positions = torch::empty({out_rows}, on_device.dtype(torch::kFloat32));
  archive_removals(archive, head_table.data_ptr<int64_t>(), slots, heads, batch_quotas,
                   offsets.data_ptr<int64_t>(), batch_positions, end - begin,
                   *std::max_element(leaving.begin(), leaving.end()));
  torch::Tensor layout = new_layout(static_cast<int64_t>(layers), heads, device);
  check_call(library.compact_heads(head_table.data_ptr<int64_t>(), slots, batch_quotas,
                                   offsets.data_ptr<int64_t>(), batch_positions, dim,
                                   static_cast<int>(keys[0].element_size()), max_length, out_rows,
                                   dptr(out_keys), dptr(out_values), out_positions.data_ptr<float>(),
                                   heads, layout.data_ptr<int32_t>(),
                                   layout.data_ptr<int32_t>() + slots, stream));
  return py::make_tuple(out_keys, out_values, out_positions, kept, layer_offsets, layout);
}

// Host planning of a reinsertion (insert_payload, cache.py:201-253, for every layer): checks the
// layers and the recalled identities, counts each (layer, head)'s recalled rows (which fixes
// the new layout without any device read), and writes one pinned int64 block: the reinsert table
// (LR_REINSERT_WORDS per slot, lr_reinsert_plan), then the recalled positions grouped by slot
// (each slot's run in input order) and the input index of each grouped entry. Layers
// come as per-layer tensors, or packed: one tensor each plus the first row of every layer
// (packed_offsets, layers + 1 entries). Returns (block, new head lengths [L][H], first row of
// each merged layer [L + 1], output rows, longest resident head).
py::tuple reinsert_prepare(const std::vector<torch::Tensor>& keys,
                           const std::vector<torch::Tensor>& values,
                           const std::vector<torch::Tensor>& positions,
                           const std::vector<std::vector<int64_t>>& head_lens,
                           const std::vector<int64_t>& packed_offsets,
                           const torch::Tensor& metadata) {
  const bool packed = !packed_offsets.empty();
  const size_t layers = head_lens.size();
  require(layers > 0 && (packed ? packed_offsets.size() == layers + 1 && keys.size() == 1 &&
                                      values.size() == 1 && positions.size() == 1
                                : keys.size() == layers && values.size() == layers &&
                                      positions.size() == layers),
          "Layer lists differ in length");
  const int64_t heads = static_cast<int64_t>(head_lens[0].size());
  require(heads > 0, "Invalid KV layout");
  require(!metadata.is_cuda() && metadata.is_contiguous() &&
              metadata.scalar_type() == torch::kInt64 && metadata.dim() == 2 &&
              metadata.size(1) == 3,
          "Recall metadata must be a contiguous int64 [count, 3] host array");
  const int64_t count = metadata.size(0);
  const int64_t slots = static_cast<int64_t>(layers) * heads;
  std::vector<int64_t> counts(static_cast<size_t>(slots), 0);
  const int64_t* meta = metadata.data_ptr<int64_t>();
  // One pass checks and counts the identities and notes whether they already come grouped by
  // slot in slot order (a transport batch does), which turns the grouping below into a copy.
  bool grouped = true;
  int64_t previous_slot = 0;
  bool valid = true;
  for (int64_t i = 0; i < count; ++i) {
    const int64_t layer = meta[3 * i], head = meta[3 * i + 1], position = meta[3 * i + 2];
    valid &= layer >= 0 && layer < static_cast<int64_t>(layers) && head >= 0 && head < heads &&
             position >= 0 && position < (int64_t{1} << 31);
    if (!valid) break;
    const int64_t slot = layer * heads + head;
    grouped &= slot >= previous_slot;
    previous_slot = slot;
    ++counts[slot];
  }
  require(valid, "Invalid recall identity");
  const torch::Tensor& k0 = keys[0];
  require(k0.dim() == 2 && k0.size(1) > 0, "Invalid KV layout");
  const int64_t dim = k0.size(1);
  const auto dtype = k0.scalar_type();
  const torch::Device device = k0.device();
  const int64_t row_bytes = dim * static_cast<int64_t>(k0.element_size());
  for (size_t t = 0; t < keys.size(); ++t) {
    const torch::Tensor &k = keys[t], &v = values[t], &p = positions[t];
    for (const torch::Tensor* x : {&k, &v, &p})
      require(x->is_cuda() && x->is_contiguous() && x->device() == device,
              "Expected contiguous CUDA tensor");
    require(k.dim() == 2 && k.sizes() == v.sizes() && k.size(1) == dim &&
                k.scalar_type() == dtype && v.scalar_type() == dtype,
            "Expected contiguous CUDA tensor");
    require(p.scalar_type() == torch::kFloat32 && p.numel() == k.size(0),
            "Position lengths do not match metadata");
  }
  torch::Tensor block = torch::empty({slots * LR_REINSERT_WORDS + 2 * count},
                                     torch::TensorOptions().dtype(torch::kInt64).pinned_memory(true));
  int64_t* table = block.data_ptr<int64_t>();
  py::list new_lens(layers), offsets(layers + 1);
  offsets[0] = py::int_(0);
  int64_t run = 0, out_row = 0, max_length = 0;
  for (size_t l = 0; l < layers; ++l) {
    require(static_cast<int64_t>(head_lens[l].size()) == heads,
            "Every layer must have the same number of KV heads");
    const size_t t = packed ? 0 : l;
    const int64_t first = packed ? packed_offsets[l] : 0;
    const int64_t layer_rows = packed ? packed_offsets[l + 1] - first : keys[t].size(0);
    require(first >= 0 && layer_rows >= 0 && first + layer_rows <= keys[t].size(0),
            "Position lengths do not match metadata");
    const int64_t kp = ptr(keys[t]), vp = ptr(values[t]), pp = ptr(positions[t]);
    py::list lengths(heads);
    int64_t base = first;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t n = head_lens[l][h];
      require(n >= 0, "Position lengths do not match metadata");
      const int64_t slot = static_cast<int64_t>(l) * heads + h;
      int64_t* row = table + slot * LR_REINSERT_WORDS;
      row[0] = kp + base * row_bytes;
      row[1] = vp + base * row_bytes;
      row[2] = pp + base * 4;
      row[3] = n;
      row[4] = run;
      row[5] = counts[slot];
      row[6] = out_row;
      row[7] = 0;
      require(counts[slot] <= LR_REINSERT_MAX_PER_HEAD, "Too many recalled rows for one head");
      run += counts[slot];
      out_row += n + counts[slot];
      lengths[h] = py::int_(n + counts[slot]);
      base += n;
      max_length = std::max(max_length, n);
    }
    require(base == first + layer_rows, "Position lengths do not match metadata");
    new_lens[l] = lengths;
    offsets[l + 1] = py::int_(out_row);
  }
  // group by slot: entry i goes to the next place of its slot's run
  int64_t* grouped_position = table + slots * LR_REINSERT_WORDS;
  int64_t* grouped_source = grouped_position + count;
  if (grouped) {  // already in slot order: entry i stays at i
    for (int64_t i = 0; i < count; ++i) {
      grouped_position[i] = meta[3 * i + 2];
      grouped_source[i] = i;
    }
  } else {
    std::vector<int64_t> cursor(static_cast<size_t>(slots));
    for (int64_t slot = 0; slot < slots; ++slot) cursor[slot] = table[slot * LR_REINSERT_WORDS + 4];
    for (int64_t i = 0; i < count; ++i) {
      const int64_t at = cursor[meta[3 * i] * heads + meta[3 * i + 1]]++;
      grouped_position[at] = meta[3 * i + 2];
      grouped_source[at] = i;
    }
  }
  return py::make_tuple(block, new_lens, offsets, out_row, max_length);
}

// The reinsert table for identities already in device memory (lr_reinsert_group fills the
// rest on the device): checks the layers, writes words [0..3] of every slot (the head's first
// resident row and its length; [4..7] zero) and uploads the table through the staging ring on
// `stream`. Nothing here depends on the identities. Returns (device table, resident rows of
// each layer [L], longest resident head).
struct ReinsertTable {
  std::vector<int64_t> words;     // LR_REINSERT_WORDS per slot, words [4..7] zero, then extras
  std::vector<int64_t> resident;  // resident rows of each layer
  int64_t max_length = 0, slots = 0, heads = 0, dim = 0;
  torch::Device device{torch::kCPU};
  torch::ScalarType dtype = torch::kBFloat16;
  int64_t elem = 2;
};

// Checks a reinsertion's layers and fills the table words [0..3] of every slot (the head's
// first resident row and its length); nothing here depends on the identities.
ReinsertTable reinsert_table_words(const std::vector<torch::Tensor>& keys,
                                   const std::vector<torch::Tensor>& values,
                                   const std::vector<torch::Tensor>& positions,
                                   const std::vector<std::vector<int64_t>>& head_lens,
                                   const std::vector<int64_t>& packed_offsets, int64_t extra) {
  ReinsertTable out;

  const bool packed = !packed_offsets.empty();
  const size_t layers = head_lens.size();
  require(layers > 0 && (packed ? packed_offsets.size() == layers + 1 && keys.size() == 1 &&
                                      values.size() == 1 && positions.size() == 1
                                : keys.size() == layers && values.size() == layers &&
                                      positions.size() == layers),
          "Layer lists differ in length");
  const int64_t heads = static_cast<int64_t>(head_lens[0].size());
  require(heads > 0, "Invalid KV layout");
  const torch::Tensor& k0 = keys[0];
  require(k0.dim() == 2 && k0.size(1) > 0, "Invalid KV layout");
  const int64_t dim = k0.size(1);
  const auto dtype = k0.scalar_type();
  const torch::Device device = k0.device();
  const int64_t row_bytes = dim * static_cast<int64_t>(k0.element_size());
  for (size_t t = 0; t < keys.size(); ++t) {
    const torch::Tensor &k = keys[t], &v = values[t], &p = positions[t];
    for (const torch::Tensor* x : {&k, &v, &p})
      require(x->is_cuda() && x->is_contiguous() && x->device() == device,
              "Expected contiguous CUDA tensor");
    require(k.dim() == 2 && k.sizes() == v.sizes() && k.size(1) == dim &&
                k.scalar_type() == dtype && v.scalar_type() == dtype,
            "Expected contiguous CUDA tensor");
    require(p.scalar_type() == torch::kFloat32 && p.numel() == k.size(0),
            "Position lengths do not match metadata");
  }
  const int64_t slots = static_cast<int64_t>(layers) * heads;
  // the table, then `extra` zero words (the launcher's flag word rides along with the upload)
  std::vector<int64_t>& table = out.words;
  table.assign(static_cast<size_t>(slots * LR_REINSERT_WORDS + extra), 0);
  out.resident.assign(layers, 0);
  int64_t& max_length = out.max_length;
  max_length = 0;
  for (size_t l = 0; l < layers; ++l) {
    require(static_cast<int64_t>(head_lens[l].size()) == heads,
            "Every layer must have the same number of KV heads");
    const size_t t = packed ? 0 : l;
    const int64_t first = packed ? packed_offsets[l] : 0;
    const int64_t layer_rows = packed ? packed_offsets[l + 1] - first : keys[t].size(0);
    require(first >= 0 && layer_rows >= 0 && first + layer_rows <= keys[t].size(0),
            "Position lengths do not match metadata");
    const int64_t kp = ptr(keys[t]), vp = ptr(values[t]), pp = ptr(positions[t]);
    int64_t base = first;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t n = head_lens[l][h];
      require(n >= 0, "Position lengths do not match metadata");
      int64_t* row = table.data() + (static_cast<int64_t>(l) * heads + h) * LR_REINSERT_WORDS;
      row[0] = kp + base * row_bytes;
      row[1] = vp + base * row_bytes;
      row[2] = pp + base * 4;
      row[3] = n;
      base += n;
      max_length = std::max(max_length, n);
    }
    require(base == first + layer_rows, "Position lengths do not match metadata");
    out.resident[l] = layer_rows;
  }
  out.slots = slots;
  out.heads = heads;
  out.dim = dim;
  out.device = device;
  out.dtype = dtype;
  out.elem = static_cast<int64_t>(k0.element_size());
  return out;
}

// The reinsert table for identities already in device memory, uploaded through the staging
// ring on `stream` (lr_reinsert_group fills the rest on the device). Returns (device table,
// resident rows of each layer [L], longest resident head).
py::tuple reinsert_table(const std::vector<torch::Tensor>& keys,
                         const std::vector<torch::Tensor>& values,
                         const std::vector<torch::Tensor>& positions,
                         const std::vector<std::vector<int64_t>>& head_lens,
                         const std::vector<int64_t>& packed_offsets, int64_t stream_handle) {
  require(library.copy_words != nullptr, "library entry points are not bound");
  const ReinsertTable t = reinsert_table_words(keys, values, positions, head_lens, packed_offsets, 0);
  void* stream = reinterpret_cast<void*>(static_cast<uintptr_t>(stream_handle));
  torch::Tensor block = staging_ring(t.device).upload(t.words.data(),
                                                      static_cast<int64_t>(t.words.size()),
                                                      t.device, stream);
  py::list resident;
  for (int64_t r : t.resident) resident.append(r);
  return py::make_tuple(block, resident, t.max_length);
}

// The whole device-grouped reinsertion (insert_payload for every layer, identities in device
// memory) from here, so that no Python runs between its launches: the table upload (with a
// zeroed flag word after it), a wait for `metadata_ready` (the identities' copy: a raw event
// handle, 0 for none), the grouping, the plan with the merged layers' metadata, the flag's copy
// to host-coherent memory, then the resident rows, a wait for `payload_ready` (likewise) and the
// recalled rows, all on `stream`. Waits (without the
// GIL) for the plan only, then reads the flag and each slot's count. Returns (out keys, out
// values, out positions, layout block i32, recalled rows i64 [count], new head lengths [L][H],
// first row of each merged layer [L + 1], flag word).
py::tuple reinsert_device_launch(const std::vector<torch::Tensor>& keys,
                                 const std::vector<torch::Tensor>& values,
                                 const std::vector<torch::Tensor>& positions,
                                 const std::vector<std::vector<int64_t>>& head_lens,
                                 const std::vector<int64_t>& packed_offsets,
                                 const torch::Tensor& payload, const torch::Tensor& metadata,
                                 int64_t metadata_ready, int64_t payload_ready, int64_t host_flag,
                                 int64_t host_counts, int64_t stream_handle) {
  require(library.reinsert_group != nullptr && library.copy_words != nullptr,
          "library entry points are not bound");
  const ReinsertTable t = reinsert_table_words(keys, values, positions, head_lens, packed_offsets, 1);
  const int64_t count = metadata.size(0);
  require(metadata.is_cuda() && metadata.device() == t.device && metadata.is_contiguous() &&
              metadata.scalar_type() == torch::kInt64 && metadata.dim() == 2 &&
              metadata.size(1) == 3,
          "Recall metadata must be an int64 [count, 3] array");
  require(payload.is_cuda() && payload.device() == t.device && payload.is_contiguous() &&
              payload.scalar_type() == t.dtype && payload.dim() == 3 && payload.size(0) == count &&
              payload.size(1) == 2 && payload.size(2) == t.dim,
          "Recalled payload must match the cache dtype and head dim");
  void* stream = reinterpret_cast<void*>(static_cast<uintptr_t>(stream_handle));
  const torch::Device device = t.device;
  const int64_t slots = t.slots, heads = t.heads, layers = slots / heads;
  int64_t resident_rows = 0;
  for (int64_t r : t.resident) resident_rows += r;
  const int64_t out_rows = resident_rows + count;
  const auto on_device = torch::TensorOptions().device(device);
  // table and flag word in one upload; the flag starts at zero. The upload does not read the
  // identities, so it goes ahead of the wait for their copy.
  torch::Tensor block = staging_ring(device).upload(t.words.data(),
                                                    static_cast<int64_t>(t.words.size()), device,
                                                    stream);
  if (metadata_ready != 0) {
    const hipError_t waited = hipStreamWaitEvent(
        static_cast<hipStream_t>(stream),
        reinterpret_cast<hipEvent_t>(static_cast<uintptr_t>(metadata_ready)), 0);
    require(waited == hipSuccess, "hipStreamWaitEvent failed on the identities' copy event");
  }
  int64_t* table = block.data_ptr<int64_t>();
  int32_t* flag = reinterpret_cast<int32_t*>(table + slots * LR_REINSERT_WORDS);
  // one int64 scratch block: the plan's workspace [3 * count], the grouped runs [2 * count],
  // the recalled rows [count], the layout (i32)
  const int64_t n = std::max<int64_t>(count, 1);
  const int64_t layout_ints = slots + layers * (heads + 1);
  const int64_t layout_words = (layout_ints + 1) / 2;
  torch::Tensor scratch = torch::empty({6 * n + layout_words}, on_device.dtype(torch::kInt64));
  int64_t* workspace = scratch.data_ptr<int64_t>();
  int64_t* grouped = workspace + 3 * n;
  torch::Tensor recalled_rows = scratch.narrow(0, 5 * n, count);
  torch::Tensor layout =
      scratch.narrow(0, 6 * n, layout_words).view(torch::kInt32).narrow(0, 0, layout_ints);
  int32_t* layout_ptr = layout.data_ptr<int32_t>();
  int64_t* counts = reinterpret_cast<int64_t*>(static_cast<uintptr_t>(host_counts));
  int64_t* flag_host = reinterpret_cast<int64_t*>(static_cast<uintptr_t>(host_flag));
  check_call(library.reinsert_group(table, slots, heads, count ? metadata.data_ptr<int64_t>() : nullptr,
                                    count, grouped, counts, flag, stream));
  check_call(library.reinsert_plan_layout(table, slots, count ? grouped : nullptr, count, workspace,
                                          count ? recalled_rows.data_ptr<int64_t>() : nullptr,
                                          flag, heads, layout_ptr, layout_ptr + slots, stream));
  check_call(library.copy_words(reinterpret_cast<const int64_t*>(flag), flag_host, 1, stream));
  c10::Event planned{c10::DeviceType::CUDA};
  planned.record(c10::impl::getDeviceGuardImpl(c10::DeviceType::CUDA)->getStream(device));
  // the merged buffers are allocated while the grouping and the plan run
  torch::Tensor out_keys = torch::empty({out_rows, t.dim}, on_device.dtype(t.dtype));
  torch::Tensor out_values = torch::empty({out_rows, t.dim}, on_device.dtype(t.dtype));
  torch::Tensor out_positions = torch::empty({out_rows}, on_device.dtype(torch::kFloat32));
  check_call(library.reinsert_resident(table, slots, workspace, count, t.max_length, t.dim,
                                       static_cast<int>(t.elem), out_rows, dptr(out_keys),
                                       dptr(out_values), out_positions.data_ptr<float>(), stream));
  if (payload_ready != 0) {
    const hipError_t waited = hipStreamWaitEvent(
        static_cast<hipStream_t>(stream),
        reinterpret_cast<hipEvent_t>(static_cast<uintptr_t>(payload_ready)), 0);
    require(waited == hipSuccess, "hipStreamWaitEvent failed on the payload's copy event");
  }
  check_call(library.reinsert_recalled(workspace, count, count ? payload.data_ptr() : nullptr,
                                       t.dim, static_cast<int>(t.elem), out_rows,
                                       dptr(out_keys), dptr(out_values),
                                       out_positions.data_ptr<float>(), stream));
  {
    py::gil_scoped_release release;
    planned.synchronize();  // the grouping and the plan only; the merges may still run
  }
  const int64_t word = *flag_host;
  py::list new_lens(layers), offsets(layers + 1);
  offsets[0] = py::int_(0);
  int64_t row = 0;
  for (int64_t l = 0; l < layers; ++l) {
    py::list lengths(heads);
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t slot = l * heads + h;
      const int64_t length = head_lens[l][h] + counts[slot];
      lengths[h] = py::int_(length);
      row += length;
    }
    new_lens[l] = lengths;
    offsets[l + 1] = py::int_(row);
  }
  return py::make_tuple(out_keys, out_values, out_positions, layout, recalled_rows, new_lens,
                        offsets, word);
}

void* current_stream(const torch::Device& device);

// ---------------------------------------------------------------------------------------
// packed_attention (src/lazy_recall/attention.py:15-35) with its checks, output and workspace
// allocation and launch in C++: a decode step makes one call per layer, and from Python the
// checks, the device context and two ctypes calls cost about 20 us of host time per call, more
// than the kernel. Same checks, order and messages as the Python layer. Returns the output
// [batch, length, query_heads * dim].
torch::Tensor attention_launch(const torch::Tensor& queries, const torch::Tensor& keys_in,
                               const torch::Tensor& values_in, const torch::Tensor& cumulative,
                               int64_t decoding_count, int64_t max_keys, int64_t length,
                               int64_t kv_heads, const py::object& pending_keys_in,
                               const py::object& pending_values_in) {
  require(library.packed_attention != nullptr, "library entry points are not bound");
  require(queries.dim() == 4, "Query length differs from the queries tensor");
  const int64_t batch = queries.size(0), query_heads = queries.size(1), dim = queries.size(3);
  require(queries.size(2) == length, "Query length differs from the queries tensor");
  require(kv_heads > 0 && query_heads % kv_heads == 0,
          "Number of heads in key/value must divide number of heads in query");
  const int64_t groups = query_heads / kv_heads;
  const auto dtype = queries.scalar_type();
  require(dtype == torch::kHalf || dtype == torch::kBFloat16,
          "FlashAttention only supports fp16 and bf16 data type");
  require(keys_in.scalar_type() == dtype && values_in.scalar_type() == dtype,
          "query and key must have the same dtype");
  for (const torch::Tensor* t : {&queries, &keys_in, &values_in}) {
    require(t->is_cuda(), "Expected contiguous CUDA tensor");
    require(t->device() == queries.device(), "CUDA devices differ");
  }
  require(dim == 64 || dim == 128 || dim == 256, "Head dimension must be 64, 128 or 256");
  require(queries.stride(3) == 1, "Input tensor must have contiguous last dimension");
  const torch::Tensor keys = keys_in.reshape({-1, dim}), values = values_in.reshape({-1, dim});
  require(keys.is_contiguous() && values.is_contiguous(), "Expected contiguous CUDA tensor");
  require(keys.sizes() == values.sizes(), "Keys and values differ in shape");
  const int64_t segments = batch * kv_heads;
  require(cumulative.is_cuda() && cumulative.scalar_type() == torch::kInt32 &&
              cumulative.is_contiguous() && cumulative.numel() == segments + 1,
          "cu_seqlens_k must have shape (batch_size + 1)");
  require(cumulative.device() == queries.device(), "CUDA devices differ");
  require(decoding_count == segments + 1, "cu_seqlens_q must have shape (batch_size + 1)");
  require(max_keys >= 0, "Invalid max_seqlen_k");
  const c10::DeviceGuard guard(queries.device());
  // The decode step's own tokens, attended to before they are appended ([batch, kv_heads, 1,
  // dim] each, one per segment)
  const bool pending = !pending_keys_in.is_none();
  require(pending == !pending_values_in.is_none(), "Pending keys and values go together");
  torch::Tensor pending_keys, pending_values;
  if (pending) {
    pending_keys = pending_keys_in.cast<torch::Tensor>();
    pending_values = pending_values_in.cast<torch::Tensor>();
    for (const torch::Tensor* t : {&pending_keys, &pending_values}) {
      require(t->is_cuda() && t->device() == queries.device(), "CUDA devices differ");
      require(t->is_contiguous() && t->scalar_type() == dtype &&
                  t->sizes() == torch::IntArrayRef({batch, kv_heads, 1, dim}),
              "Pending keys and values must be contiguous [batch, kv_heads, 1, head_dim]");
    }
    require(length == 1, "Pending rows need one query per segment");
  }
  torch::Tensor out = torch::empty({batch, length, query_heads, dim}, queries.options());
  const size_t size =
      pending ? library.pending_workspace_bytes(segments, groups, max_keys, dim)
              : library.attention_workspace_bytes(segments, groups, length, max_keys, dim);
  torch::Tensor workspace;
  if (size)
    workspace = torch::empty({static_cast<int64_t>(size)},
                             queries.options().dtype(torch::kUInt8));
  const float scale = static_cast<float>(std::pow(static_cast<double>(dim), -0.5));
  if (pending) {
    check_call(library.packed_attention_pending(
        queries.data_ptr(), queries.stride(0), queries.stride(1), queries.stride(2),
        keys.numel() ? keys.data_ptr() : nullptr, values.numel() ? values.data_ptr() : nullptr,
        keys.size(0), cumulative.data_ptr<int32_t>(), batch, kv_heads, groups, dim,
        dtype == torch::kBFloat16 ? LR_DTYPE_BF16 : LR_DTYPE_F16, max_keys, scale,
        pending_keys.data_ptr(), pending_values.data_ptr(), out.data_ptr(),
        size ? workspace.data_ptr() : nullptr, size, current_stream(queries.device())));
    return out.view({batch, length, query_heads * dim});
  }
  check_call(library.packed_attention(
      queries.data_ptr(), queries.stride(0), queries.stride(1), queries.stride(2),
      keys.numel() ? keys.data_ptr() : nullptr, values.numel() ? values.data_ptr() : nullptr,
      keys.size(0), cumulative.data_ptr<int32_t>(), batch, kv_heads, groups, length, dim,
      dtype == torch::kBFloat16 ? LR_DTYPE_BF16 : LR_DTYPE_F16, max_keys, scale, out.data_ptr(),
      size ? workspace.data_ptr() : nullptr, size, current_stream(queries.device())));
  return out.view({batch, length, query_heads * dim});
}

// ---------------------------------------------------------------------------------------
// The per-layer drop-ins _C.append and _C.compact with their checks, output allocation and
// launch in C++ (a decode step makes one append per layer; from Python each call cost ~20 us of
// host time in tensor checks, five allocations and the ctypes call). Same checks, order and
// messages as the Python mirror of csrc/scoring.cu:257-314.

void check_cuda(const torch::Tensor& t, const torch::Tensor& reference) {
  require(t.is_cuda() && t.is_contiguous(), "Expected contiguous CUDA tensor");
  require(t.device() == reference.device(), "CUDA devices differ");
}

void check_cache(const torch::Tensor& keys, const torch::Tensor& values,
                 const torch::Tensor& positions) {
  for (const torch::Tensor* t : {&keys, &values, &positions}) check_cuda(*t, keys);
  require(keys.dim() == 2 && keys.size(1) > 0 && keys.sizes() == values.sizes() &&
              keys.scalar_type() == values.scalar_type(),
          "Invalid KV layout");
  require(positions.scalar_type() == torch::kFloat32 && positions.numel() == keys.size(0),
          "Invalid positions");
}

int elem_bytes(const torch::Tensor& t, const char* op) {
  const auto type = t.scalar_type();
  if (type != torch::kFloat32 && type != torch::kFloat64 && type != torch::kFloat16 &&
      type != torch::kBFloat16)
    throw std::runtime_error(std::string("\"") + op + "\" not implemented for '" +
                             std::string(c10::toString(type)) + "'");
  return static_cast<int>(t.element_size());
}

void* current_stream(const torch::Device& device) {
  return c10::hip::getCurrentHIPStream(device.index()).stream();
}

std::vector<torch::Tensor> append_launch(const torch::Tensor& keys, const torch::Tensor& values,
                                         const torch::Tensor& positions,
                                         const torch::Tensor& new_keys,
                                         const torch::Tensor& new_values,
                                         const torch::Tensor& cumulative, int64_t logical_start,
                                         int64_t maximum_length) {
  require(library.append != nullptr, "library entry points are not bound");
  check_cache(keys, values, positions);
  for (const torch::Tensor* t : {&new_keys, &new_values, &cumulative}) check_cuda(*t, keys);
  require(new_keys.dim() == 4 && new_keys.size(0) == 1 && new_keys.sizes() == new_values.sizes() &&
              new_keys.scalar_type() == keys.scalar_type() &&
              new_values.scalar_type() == keys.scalar_type(),
          "Invalid appended KV");
  const int64_t heads = new_keys.size(1), added = new_keys.size(2), dim = keys.size(1);
  require(heads > 0 && added > 0 && new_keys.size(3) == dim && maximum_length >= 0,
          "Invalid appended shape");
  require(cumulative.scalar_type() == torch::kInt32 && cumulative.numel() == heads + 1,
          "Invalid cumulative lengths");
  const int elem = elem_bytes(keys, "lazy_recall_append");
  const c10::DeviceGuard guard(keys.device());
  const int64_t rows = keys.size(0) + heads * added;
  const auto options = keys.options();
  torch::Tensor out_keys = torch::empty({rows, dim}, options);
  torch::Tensor out_values = torch::empty({rows, dim}, options);
  torch::Tensor out_positions = torch::empty({rows, 1}, positions.options());
  torch::Tensor out_cumulative = torch::empty_like(cumulative);
  torch::Tensor out_lengths = torch::empty({heads}, cumulative.options());
  check_call(library.append(
      keys.numel() ? keys.data_ptr() : nullptr, values.numel() ? values.data_ptr() : nullptr,
      positions.numel() ? positions.data_ptr<float>() : nullptr, keys.size(0),
      new_keys.data_ptr(), new_values.data_ptr(), cumulative.data_ptr<int32_t>(), heads, added,
      dim, elem, logical_start, maximum_length, out_keys.data_ptr(), out_values.data_ptr(),
      out_positions.data_ptr<float>(), out_cumulative.data_ptr<int32_t>(),
      out_lengths.data_ptr<int32_t>(), current_stream(keys.device())));
  return {out_keys, out_values, out_positions, out_cumulative, out_lengths};
}

std::vector<torch::Tensor> compact_launch(const torch::Tensor& keys, const torch::Tensor& values,
                                          const torch::Tensor& positions,
                                          const torch::Tensor& removed) {
  require(library.compact != nullptr, "library entry points are not bound");
  check_cache(keys, values, positions);
  check_cuda(removed, keys);
  require(removed.scalar_type() == torch::kInt64 && removed.dim() == 1 &&
              removed.numel() <= keys.size(0),
          "Invalid removals");
  const int elem = elem_bytes(keys, "lazy_recall_compact");
  const c10::DeviceGuard guard(keys.device());
  const int64_t rows = keys.size(0) - removed.numel(), dim = keys.size(1);
  torch::Tensor out_keys = torch::empty({rows, dim}, keys.options());
  torch::Tensor out_values = torch::empty({rows, dim}, keys.options());
  torch::Tensor out_positions = torch::empty({rows, 1}, positions.options());
  if (rows > 0)
    check_call(library.compact(keys.data_ptr(), values.data_ptr(), positions.data_ptr<float>(),
                               keys.size(0), dim, elem,
                               removed.numel() ? removed.data_ptr<int64_t>() : nullptr,
                               removed.numel(), out_keys.data_ptr(), out_values.data_ptr(),
                               out_positions.data_ptr<float>(), current_stream(keys.device())));
  return {out_keys, out_values, out_positions};
}

// The most layers whose append table lr_append_layers_host takes in the launch.
constexpr int64_t kInlineAppendLayers = 48;

// One decode step's append into every layer (lr_append_layers): the per-layer checks of
// append_launch for each layer, the table (in the launch's kernel arguments for up to
// kInlineAppendLayers layers, else pinned and uploaded without blocking), packed outputs and
// one launch. Returns (keys, values, positions [rows, 1], cumulative [L, H + 1] i32, lengths
// [L, H] i32, first output row of each layer [L + 1]).
py::tuple append_layers_launch(const std::vector<torch::Tensor>& keys,
                               const std::vector<torch::Tensor>& values,
                               const std::vector<torch::Tensor>& positions,
                               const std::vector<torch::Tensor>& new_keys,
                               const std::vector<torch::Tensor>& new_values,
                               const std::vector<torch::Tensor>& cumulative,
                               const std::vector<int64_t>& logical_starts,
                               int64_t maximum_length) {
  require(library.append_layers != nullptr, "library entry points are not bound");
  const size_t layers = keys.size();
  require(layers > 0 && values.size() == layers && positions.size() == layers &&
              new_keys.size() == layers && new_values.size() == layers &&
              cumulative.size() == layers && logical_starts.size() == layers,
          "Layer lists differ in length");
  const torch::Tensor& k0 = keys[0];
  int64_t heads = 0, added = 0, dim = 0;
  const bool inline_table = static_cast<int64_t>(layers) <= kInlineAppendLayers;
  std::vector<int64_t> host_rows;
  torch::Tensor table;
  if (inline_table) {
    host_rows.resize(layers * LR_APPEND_WORDS);
  } else {
    table = torch::empty({static_cast<int64_t>(layers) * LR_APPEND_WORDS},
                         torch::TensorOptions().dtype(torch::kInt64).pinned_memory(true));
  }
  int64_t* rows = inline_table ? host_rows.data() : table.data_ptr<int64_t>();
  py::list firsts(layers + 1);
  int64_t total = 0;
  int elem = 0;
  for (size_t l = 0; l < layers; ++l) {
    const torch::Tensor &k = keys[l], &v = values[l], &p = positions[l];
    check_cache(k, v, p);
    check_cuda(k, k0);
    for (const torch::Tensor* t : {&new_keys[l], &new_values[l], &cumulative[l]}) check_cuda(*t, k0);
    const torch::Tensor &nk = new_keys[l], &nv = new_values[l];
    require(nk.dim() == 4 && nk.size(0) == 1 && nk.sizes() == nv.sizes() &&
                nk.scalar_type() == k0.scalar_type() && nv.scalar_type() == k0.scalar_type() &&
                k.scalar_type() == k0.scalar_type(),
            "Invalid appended KV");
    if (l == 0) {
      heads = nk.size(1);
      added = nk.size(2);
      dim = k0.size(1);
      elem = elem_bytes(k0, "lazy_recall_append");
    }
    require(heads > 0 && added > 0 && nk.size(1) == heads && nk.size(2) == added &&
                nk.size(3) == dim && k.size(1) == dim && maximum_length >= 0,
            "Invalid appended shape");
    require(cumulative[l].scalar_type() == torch::kInt32 && cumulative[l].numel() == heads + 1,
            "Invalid cumulative lengths");
    int64_t* row = rows + l * LR_APPEND_WORDS;
    row[0] = k.numel() ? ptr(k) : 0;
    row[1] = v.numel() ? ptr(v) : 0;
    row[2] = p.numel() ? ptr(p) : 0;
    row[3] = k.size(0);
    row[4] = ptr(cumulative[l]);
    row[5] = ptr(nk);
    row[6] = ptr(nv);
    row[7] = logical_starts[l];
    row[8] = total;
    row[9] = row[10] = row[11] = 0;
    firsts[l] = py::int_(total);
    total += k.size(0) + heads * added;
  }
  firsts[layers] = py::int_(total);
  const c10::DeviceGuard guard(k0.device());
  torch::Tensor device_table;
  if (!inline_table) device_table = table.to(k0.device(), /*non_blocking=*/true);
  torch::Tensor out_keys = torch::empty({total, dim}, k0.options());
  torch::Tensor out_values = torch::empty({total, dim}, k0.options());
  torch::Tensor out_positions = torch::empty({total, 1}, positions[0].options());
  const auto i32 = cumulative[0].options();
  torch::Tensor out_cumulative = torch::empty({static_cast<int64_t>(layers), heads + 1}, i32);
  torch::Tensor out_lengths = torch::empty({static_cast<int64_t>(layers), heads}, i32);
  const auto launch = inline_table ? library.append_layers_host : library.append_layers;
  check_call(launch(inline_table ? host_rows.data() : device_table.data_ptr<int64_t>(),
                    static_cast<int64_t>(layers), heads, added, dim, elem, maximum_length,
                    out_keys.data_ptr(), out_values.data_ptr(), out_positions.data_ptr<float>(),
                    out_cumulative.data_ptr<int32_t>(), out_lengths.data_ptr<int32_t>(),
                    current_stream(k0.device())));
  return py::make_tuple(out_keys, out_values, out_positions, out_cumulative, out_lengths, firsts);
}

// The most batch_append segments whose descriptors lr_batch_append_host takes in the launch.
constexpr int64_t kInlineDescriptorSegments = 64;

// The batch_append descriptors of csrc/batch_append.cu:49-80, one 7-word row per (request,
// head): [keys ptr, values ptr, positions ptr, first source row, old length, destination row,
// logical position]; same checks, order and messages as the reference's host loop. Returns
// (descriptors int64 [R*H, 7] already copied to `device` on the current stream (from pinned
// memory, without blocking the host), total output rows, rows of the longest head + 1).
// _C.batch_append (csrc/batch_append.cu:36-94): the reference's descriptor loop and checks
// (batch_append.cu:49-80), the output allocation and the launch, all here. Up to 64 (request,
// head) descriptors travel in the launch's kernel arguments; larger tables are written into a
// pinned, host-coherent staging buffer that the kernel reads in place. Either way the launch
// needs neither a copy (the reference's copy, batch_append.cu:81, blocks the host) nor a copy
// kernel. Returns [keys, values, positions [rows, 1]] packed.
std::vector<torch::Tensor> batch_append_launch(const std::vector<torch::Tensor>& keys,
                                               const std::vector<torch::Tensor>& values,
                                               const std::vector<torch::Tensor>& positions,
                                               const torch::Tensor& new_keys,
                                               const torch::Tensor& new_values,
                                               const std::vector<std::vector<int64_t>>& lengths,
                                               const std::vector<int64_t>& logical_positions,
                                               int64_t stream_handle) {
  require(library.batch_append != nullptr && library.staging_alloc != nullptr,
          "library entry points are not bound");
  const int64_t heads = new_keys.size(1), dim = new_keys.size(3);
  const auto dtype = new_keys.scalar_type();
  const torch::Device device = new_keys.device();
  const size_t requests = keys.size();
  const int64_t row_bytes = dim * c10::elementSize(dtype);
  int64_t granule = 16;
  while (granule > 1 && row_bytes % granule) granule /= 2;
  std::vector<int64_t> host(requests * static_cast<size_t>(heads) * 7);
  int64_t* out = host.data();
  int64_t destination = 0, maximum = 0;
  for (size_t r = 0; r < requests; ++r) {
    const torch::Tensor &k = keys[r], &v = values[r], &p = positions[r];
    require(k.is_cuda() && k.is_contiguous() && v.is_contiguous() && p.is_contiguous(),
            "Contiguous CUDA cache required");
    require(k.device() == device && v.device() == device && p.device() == device,
            "Cache devices differ");
    require(k.dim() == 2 && k.size(1) == dim && k.sizes() == v.sizes() && k.scalar_type() == dtype &&
                v.scalar_type() == dtype,
            "Cache K/V mismatch");
    const int64_t logical = logical_positions[r];
    require(p.scalar_type() == torch::kFloat32 && p.numel() == k.size(0) &&
                static_cast<int64_t>(lengths[r].size()) == heads && logical >= 0 &&
                logical < (int64_t{1} << 24),
            "Invalid positions or head metadata");
    require(reinterpret_cast<uintptr_t>(k.data_ptr()) % granule == 0 &&
                reinterpret_cast<uintptr_t>(v.data_ptr()) % granule == 0,
            "Cache rows must be aligned to the row granule");
    int64_t source = 0;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t n = lengths[r][h];
      require(n >= 0, "Invalid head length");
      require(source + n <= k.size(0), "Invalid head length");
      int64_t* row = out + (static_cast<int64_t>(r) * heads + h) * 7;
      row[0] = ptr(k);
      row[1] = ptr(v);
      row[2] = ptr(p);
      row[3] = source;
      row[4] = n;
      row[5] = destination;
      row[6] = logical;
      source += n;
      destination += n + 1;
      maximum = std::max(maximum, n + 1);
    }
    require(source == k.size(0), "Head lengths do not cover cache rows");
  }
  void* stream = reinterpret_cast<void*>(static_cast<uintptr_t>(stream_handle));
  const auto options = torch::TensorOptions().device(device);
  torch::Tensor out_keys = torch::empty({destination, dim}, options.dtype(dtype));
  torch::Tensor out_values = torch::empty({destination, dim}, options.dtype(dtype));
  torch::Tensor out_positions = torch::empty({destination, 1}, options.dtype(torch::kFloat32));
  const int64_t segments = static_cast<int64_t>(requests) * heads;
  const int elem_bytes = static_cast<int>(c10::elementSize(dtype));
  if (segments <= kInlineDescriptorSegments) {
    check_call(library.batch_append_host(host.data(), segments, new_keys.data_ptr(),
                                         new_values.data_ptr(), dim, elem_bytes, maximum,
                                         out_keys.data_ptr(), out_values.data_ptr(),
                                         out_positions.data_ptr<float>(), stream));
    return {out_keys, out_values, out_positions};
  }
  StagingRing& ring = staging_ring(device);
  const int64_t* descriptors = ring.stage(host.data(), static_cast<int64_t>(host.size()));
  check_call(library.batch_append(descriptors, segments, new_keys.data_ptr(),
                                  new_values.data_ptr(), dim, elem_bytes, maximum,
                                  out_keys.data_ptr(), out_values.data_ptr(),
                                  out_positions.data_ptr<float>(), stream));
  ring.release(device);
  return {out_keys, out_values, out_positions};
}

}  // namespace

PYBIND11_MODULE(_plan, module) {
  module.def("plan_audit", &plan_audit, "Validate layers and build the audit metadata block");
  module.def("bind_library", &bind_library, "Bind the entry points of liblazyrecall_hip.so");
  module.def("bind_data_movement", &bind_data_movement,
             "Bind lr_append and lr_compact of liblazyrecall_hip.so");
  module.def("append", &append_launch, "_C.append (csrc/scoring.cu:264-292)");
  module.def("compact", &compact_launch, "_C.compact (csrc/scoring.cu:294-314)");
  module.def("append_layers", &append_layers_launch, "One decode step's append into every layer");
  py::class_<StepSync>(module, "StepSync")
      .def(py::init<>())
      .def("wait", &StepSync::wait, py::arg("check_finite"),
           "Wait for the selection of the pending step; returns (kept [L][H], layer offsets)");
  module.def("audit_launch", &audit_launch, "Enqueue one whole audit step");
  module.def("queue_evict_launch", &queue_evict_launch,
             "Enqueue one evict_prefix batch of an audit's lazy queue");
  module.def("bind_attention", &bind_attention,
             "Bind lr_packed_attention and its workspace size (addresses from the ctypes handle)");
  module.def("packed_attention", &attention_launch,
             "packed_attention: checks, output and workspace allocation and launch from C++");
  module.def("reinsert_prepare", &reinsert_prepare,
             "Check a reinsertion and build its pinned table + metadata block");
  module.def("reinsert_table", &reinsert_table,
             "Check a reinsertion's layers and upload its table for lr_reinsert_group");
  module.def("bind_reinsert", &bind_reinsert,
             "Bind the reinsertion entry points of liblazyrecall_hip.so");
  module.def("reinsert_device", &reinsert_device_launch,
             "Enqueue a whole device-grouped reinsertion and wait for its plan");
  module.def("batch_append", &batch_append_launch,
             "_C.batch_append: checks, descriptors in host-coherent staging, outputs and launch");
  module.attr("LR_SEG_WORDS") = LR_SEG_WORDS;
  module.attr("LR_HEAD_WORDS") = LR_HEAD_WORDS;
}
