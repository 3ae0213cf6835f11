// CPU-owned bounded exact maximum-inner-product archive of evicted KV rows: the recall worker's
// ArchiveIndex / HeadArchive (src/lazy_recall/recall/cpu_worker.py:17-134) without faiss.
//
// Per (layer, KV head) segment the rows live in slot-indexed arrays: f32 keys [slots, dim] for
// the inner products, the bf16 payload [slots, 2, dim], the position (identity, -1 = empty) and
// an index sequence number. faiss's IndexIDMap2(IndexFlatIP) keeps its vectors in the order they
// were added (removal compacts without reordering), and a flat search visits them in that order;
// the sequence number reproduces that order for equal inner products, so a search is a scan of
// the live slots keeping the top-k by (product descending, sequence ascending).
#include "../../include/lazyrecall_archive.h"

#include <algorithm>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

thread_local std::string g_error;

int fail(const char* message) {
  g_error = message;
  return 1;
}

float bf16_to_f32(uint16_t bits) {
  const uint32_t word = static_cast<uint32_t>(bits) << 16;
  float value;
  std::memcpy(&value, &word, sizeof(value));
  return value;
}

// f32 inner product with eight independent partial sums (vectorised without reassociation),
// added pairwise at the end.
float inner_product(const float* a, const float* b, int64_t dim) {
  float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t e = 0;
  for (; e + 8 <= dim; e += 8)
    for (int j = 0; j < 8; ++j) part[j] += a[e + j] * b[e + j];
  for (; e < dim; ++e) part[e & 7] += a[e] * b[e];
  return ((part[0] + part[4]) + (part[2] + part[6])) + ((part[1] + part[5]) + (part[3] + part[7]));
}

struct Head {
  int64_t dim = 0, capacity = 0;
  std::vector<float> keys;          // [allocated, dim]
  std::vector<uint16_t> payload;    // [allocated, 2, dim]
  std::vector<int64_t> positions;   // [allocated], -1 = empty
  std::vector<uint64_t> sequence;   // [allocated], order in the index
  std::unordered_map<int64_t, int64_t> lookup;  // position -> slot
  std::vector<int64_t> free;
  int64_t used = 0, cursor = 0, dropped = 0;
  uint64_t next_sequence = 0;

  int64_t allocated() const { return static_cast<int64_t>(positions.size()); }

  void grow() {  // cpu_worker.py:29-35: double, at least 128, at most capacity
    const int64_t length = std::min(capacity, std::max<int64_t>(128, allocated() * 2));
    keys.resize(static_cast<size_t>(length * dim));
    payload.resize(static_cast<size_t>(length * 2 * dim));
    positions.resize(static_cast<size_t>(length), -1);
    sequence.resize(static_cast<size_t>(length), 0);
  }

  void remove(const int64_t* list, int64_t count) {  // cpu_worker.py:37-46
    for (int64_t i = 0; i < count; ++i) {
      const auto it = lookup.find(list[i]);
      if (it == lookup.end()) continue;
      const int64_t slot = it->second;
      lookup.erase(it);
      positions[slot] = -1;
      free.push_back(slot);
    }
  }

  // cpu_worker.py:48-82. rows: indices into the batch arrays of this segment's rows.
  void add(const std::vector<int64_t>& rows, const int64_t* metadata, const uint16_t* batch) {
    std::vector<int64_t> present;
    for (const int64_t row : rows) present.push_back(metadata[3 * row + 2]);
    remove(present.data(), static_cast<int64_t>(present.size()));
    std::vector<int64_t> slots, kept;
    for (const int64_t row : rows) {
      const int64_t position = metadata[3 * row + 2];
      int64_t slot;
      if (!free.empty()) {
        slot = free.back();
        free.pop_back();
      } else if (used < capacity) {
        if (used == allocated()) grow();
        slot = used++;
      } else {
        slot = cursor;
        cursor = (cursor + 1) % capacity;
        const int64_t previous = positions[slot];
        if (previous >= 0) {
          lookup.erase(previous);
          ++dropped;
        }
        const auto earlier = std::find(slots.begin(), slots.end(), slot);
        if (earlier != slots.end()) {  // overwritten within this batch: never indexed
          kept.erase(kept.begin() + (earlier - slots.begin()));
          slots.erase(earlier);
        }
      }
      std::memcpy(&payload[static_cast<size_t>(slot * 2 * dim)], batch + row * 2 * dim,
                  sizeof(uint16_t) * 2 * dim);
      positions[slot] = position;
      lookup[position] = slot;
      slots.push_back(slot);
      kept.push_back(row);
    }
    for (const int64_t slot : slots) {  // indexed in batch order, after every overwrite
      float* key = &keys[static_cast<size_t>(slot * dim)];
      const uint16_t* bits = &payload[static_cast<size_t>(slot * 2 * dim)];
      for (int64_t e = 0; e < dim; ++e) key[e] = bf16_to_f32(bits[e]);
      sequence[slot] = next_sequence++;
    }
  }

  // Top-k live slots by (inner product descending, sequence ascending).
  int64_t search(const float* query, int64_t topk, int64_t* out_positions,
                 uint16_t* out_payload) const {
    const int64_t k = std::min<int64_t>(topk, static_cast<int64_t>(lookup.size()));
    if (k <= 0) return 0;
    std::vector<float> best_score;
    std::vector<uint64_t> best_sequence;
    std::vector<int64_t> best_slot;
    best_score.reserve(k + 1);
    best_sequence.reserve(k + 1);
    best_slot.reserve(k + 1);
    const int64_t limit = allocated();
    for (int64_t slot = 0; slot < limit; ++slot) {
      if (positions[slot] < 0) continue;
      const float dot = inner_product(&keys[static_cast<size_t>(slot * dim)], query, dim);
      const uint64_t seq = sequence[slot];
      const int64_t have = static_cast<int64_t>(best_slot.size());
      if (have == k) {
        const float worst = best_score[k - 1];
        if (dot < worst || (dot == worst && seq > best_sequence[k - 1])) continue;
        if (dot != dot) continue;  // NaN never enters a full list
      }
      int64_t at = have;
      while (at > 0 && (dot > best_score[at - 1] ||
                        (dot == best_score[at - 1] && seq < best_sequence[at - 1])))
        --at;
      best_score.insert(best_score.begin() + at, dot);
      best_sequence.insert(best_sequence.begin() + at, seq);
      best_slot.insert(best_slot.begin() + at, slot);
      if (static_cast<int64_t>(best_slot.size()) > k) {
        best_score.pop_back();
        best_sequence.pop_back();
        best_slot.pop_back();
      }
    }
    for (int64_t i = 0; i < static_cast<int64_t>(best_slot.size()); ++i) {
      out_positions[i] = positions[best_slot[i]];
      std::memcpy(out_payload + i * 2 * dim, &payload[static_cast<size_t>(best_slot[i] * 2 * dim)],
                  sizeof(uint16_t) * 2 * dim);
    }
    return static_cast<int64_t>(best_slot.size());
  }
};

struct Archive {
  int64_t layers, heads, dim, capacity;
  int threads;
  std::vector<Head> segments;
};

}  // namespace

extern "C" const char* lra_last_error(void) { return g_error.c_str(); }

extern "C" void* lra_create(int64_t layers, int64_t heads, int64_t dim, int64_t capacity,
                            int threads) {
  g_error.clear();
  if (layers <= 0 || heads <= 0 || dim <= 0 || capacity <= 0 || threads <= 0) {
    fail("Invalid archive configuration");
    return nullptr;
  }
  auto* archive = new Archive{layers, heads, dim, capacity, threads, {}};
  archive->segments.resize(static_cast<size_t>(layers * heads));
  for (Head& head : archive->segments) {
    head.dim = dim;
    head.capacity = capacity;
  }
  return archive;
}

extern "C" void lra_destroy(void* handle) { delete static_cast<Archive*>(handle); }

extern "C" int lra_add(void* handle, const int64_t* metadata, const uint16_t* payload,
                       int64_t count) {
  g_error.clear();
  auto* archive = static_cast<Archive*>(handle);
  if (!archive || count < 0 || (count > 0 && (!metadata || !payload)))
    return fail("Archive payload shape mismatch");
  std::vector<std::vector<int64_t>> rows(archive->segments.size());
  std::vector<int64_t> order;  // segments in ascending order (np.unique)
  for (int64_t i = 0; i < count; ++i) {
    const int64_t layer = metadata[3 * i], head = metadata[3 * i + 1];
    if (layer < 0 || head < 0 || metadata[3 * i + 2] < 0 || layer >= archive->layers ||
        head >= archive->heads)
      return fail("Invalid archive identity");
    rows[static_cast<size_t>(layer * archive->heads + head)].push_back(i);
  }
  for (const auto& segment_rows : rows) {  // checked before any segment changes
    std::unordered_set<int64_t> seen;
    for (const int64_t row : segment_rows)
      if (!seen.insert(metadata[3 * row + 2]).second)
        return fail("Duplicate identities in one archive batch");
  }
  for (size_t s = 0; s < rows.size(); ++s)
    if (!rows[s].empty()) archive->segments[s].add(rows[s], metadata, payload);
  return 0;
}

extern "C" int lra_remove(void* handle, const int64_t* metadata, int64_t count) {
  g_error.clear();
  auto* archive = static_cast<Archive*>(handle);
  if (!archive || count < 0 || (count > 0 && !metadata)) return fail("Invalid archive identity");
  for (int64_t i = 0; i < count; ++i) {
    const int64_t layer = metadata[3 * i], head = metadata[3 * i + 1];
    if (layer < 0 || head < 0 || layer >= archive->layers || head >= archive->heads) continue;
    archive->segments[static_cast<size_t>(layer * archive->heads + head)].remove(
        &metadata[3 * i + 2], 1);
  }
  return 0;
}

extern "C" int lra_search(void* handle, const float* queries, int64_t topk,
                          int64_t* out_metadata, uint16_t* out_payload, int64_t* out_count) {
  g_error.clear();
  auto* archive = static_cast<Archive*>(handle);
  if (!archive || !queries || topk <= 0 || !out_metadata || !out_payload || !out_count)
    return fail("Invalid archive search");
  const int64_t segments = static_cast<int64_t>(archive->segments.size());
  const int64_t dim = archive->dim;
  std::vector<int64_t> found(static_cast<size_t>(segments), 0);
  std::vector<int64_t> positions(static_cast<size_t>(segments * topk));
  std::vector<uint16_t> rows(static_cast<size_t>(segments * topk * 2 * dim));
  auto work = [&](int64_t first, int64_t stride) {
    for (int64_t s = first; s < segments; s += stride)
      found[s] = archive->segments[s].search(queries + s * dim, topk, &positions[s * topk],
                                             &rows[static_cast<size_t>(s * topk * 2 * dim)]);
  };
  const int workers = static_cast<int>(std::min<int64_t>(archive->threads, segments));
  std::vector<std::thread> pool;
  for (int t = 1; t < workers; ++t) pool.emplace_back(work, t, workers);
  work(0, workers);
  for (auto& thread : pool) thread.join();
  int64_t n = 0;
  for (int64_t s = 0; s < segments; ++s) {
    for (int64_t i = 0; i < found[s]; ++i, ++n) {
      out_metadata[3 * n] = s / archive->heads;
      out_metadata[3 * n + 1] = s % archive->heads;
      out_metadata[3 * n + 2] = positions[s * topk + i];
      std::memcpy(out_payload + n * 2 * dim, &rows[static_cast<size_t>((s * topk + i) * 2 * dim)],
                  sizeof(uint16_t) * 2 * dim);
    }
  }
  *out_count = n;
  return 0;
}

extern "C" int64_t lra_size(void* handle) {
  auto* archive = static_cast<Archive*>(handle);
  int64_t total = 0;
  if (archive)
    for (const Head& head : archive->segments) total += static_cast<int64_t>(head.lookup.size());
  return total;
}

extern "C" int64_t lra_dropped(void* handle) {
  auto* archive = static_cast<Archive*>(handle);
  int64_t total = 0;
  if (archive)
    for (const Head& head : archive->segments) total += head.dropped;
  return total;
}
