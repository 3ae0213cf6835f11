// The recall transport's host side as one native object (liblazyrecall_recall.so): staging slot
// states, the two copy streams and their events, the archive and the worker thread that runs
// the CPU half. Declared in include/lazyrecall_recall.h.
//
// Behaviour follows src/lazy_recall/recall/transport.py:46-361 and its worker
// recall/cpu_worker.py:136-182 (slot state machine, copy ordering, counters), built differently:
// the reference's main thread polls copy events and forwards messages to a spawned process over
// queues and shared memory; here the caller only enqueues work and commits slots, and the worker
// thread of the same process waits for each job's copy event itself, calls the archive directly
// and enqueues the results' copy back into device staging.
#include <hip/hip_runtime_api.h>
#include <sys/resource.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "lazyrecall_archive.h"
#include "lazyrecall_recall.h"

namespace {

thread_local std::string g_error;

int fail(int status, const std::string& message) {
  g_error = message;
  return status;
}

#define LRR_CHECK(cond, message) \
  do {                           \
    if (!(cond)) return fail(LRR_ERR_INVALID, message); \
  } while (0)

#define LRR_HIP(expr)                                                               \
  do {                                                                              \
    const hipError_t status_ = (expr);                                              \
    if (status_ != hipSuccess) {                                                    \
      (void)hipGetLastError();                                                      \
      return fail(LRR_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(status_)); \
    }                                                                               \
  } while (0)

enum JobKind { kArchiveJob, kSearchJob, kRemoveJob };

struct Job {
  JobKind kind;
  int slot = -1;
  int64_t count = 0;
  std::vector<int64_t> metadata;  // removals
};

int64_t peak_rss_kib() {
  rusage usage{};
  getrusage(RUSAGE_SELF, &usage);
  return static_cast<int64_t>(usage.ru_maxrss);  // KiB on Linux
}

struct Ring {
  // configuration
  int64_t layers = 0, heads = 0, dim = 0, topk = 0, archive_slots = 0, capacity = 0,
          result_capacity = 0;
  int device = 0;
  // caller-owned buffers
  uint16_t* host_archive_payload = nullptr;
  int64_t* host_archive_metadata = nullptr;
  float* host_queries = nullptr;
  uint16_t* host_result_payload = nullptr;
  int64_t* host_result_metadata = nullptr;
  char* device_archive_payload = nullptr;
  char* device_archive_metadata = nullptr;
  char* device_queries = nullptr;
  char* device_result_payload = nullptr;
  char* device_result_metadata = nullptr;
  // copies and their events
  hipStream_t out_stream = nullptr, in_stream = nullptr;
  std::vector<hipEvent_t> archive_ready, archive_copied;  // per archive slot
  hipEvent_t query_ready[2] = {}, query_copied[2] = {}, result_copied[2] = {},
             result_released[2] = {};
  // slot states (written by both threads, hence atomic)
  std::unique_ptr<std::atomic<int>[]> archive_state;
  std::atomic<int> query_state[2];
  std::atomic<int64_t> query_step[2];
  std::atomic<int64_t> result_count[2];
  // the archive, touched only by the worker once the ring exists
  void* archive = nullptr;
  std::atomic<int64_t> counters[LRR_COUNTERS];
  // the job queue
  std::mutex mutex;
  std::condition_variable changed;
  std::deque<Job> jobs;
  bool busy = false, stop = false;
  std::string worker_error;
  std::thread worker;
  std::atomic<bool> alive{false};

  size_t archive_payload_bytes() const { return static_cast<size_t>(capacity * 2 * dim) * 2; }
  size_t archive_metadata_bytes() const { return static_cast<size_t>(capacity * 3) * 8; }
  size_t query_bytes() const { return static_cast<size_t>(layers * heads * dim) * 4; }
  size_t result_payload_bytes() const { return static_cast<size_t>(result_capacity * 2 * dim) * 2; }
  size_t result_metadata_bytes() const { return static_cast<size_t>(result_capacity * 3) * 8; }

  void push(Job job) {
    {
      std::lock_guard<std::mutex> lock(mutex);
      jobs.push_back(std::move(job));
    }
    changed.notify_all();
  }

  // A failure the worker recorded, reported once to the caller's next call.
  int take_worker_error() {
    std::lock_guard<std::mutex> lock(mutex);
    if (worker_error.empty()) return LRR_OK;
    const std::string message = std::move(worker_error);
    worker_error.clear();
    return fail(LRR_ERR_WORKER, "CPU recall worker failed: " + message);
  }

  void refresh_archive_counters() {
    counters[LRR_COUNTER_INDEXED] = lra_size(archive);
    counters[LRR_COUNTER_CAPACITY_DROPS] = lra_dropped(archive);
    counters[LRR_COUNTER_PEAK_RSS_KIB] = peak_rss_kib();
  }

  // One job on the worker thread; returns an error message or "".
  std::string execute(Job& job) {
    if (job.kind == kRemoveJob) {
      const int status = lra_remove(archive, job.metadata.data(),
                                    static_cast<int64_t>(job.metadata.size() / 3));
      refresh_archive_counters();
      return status ? std::string("remove: ") + lra_last_error() : std::string();
    }
    const int slot = job.slot;
    if (job.kind == kArchiveJob) {
      hipError_t status = hipEventSynchronize(archive_copied[slot]);
      if (status != hipSuccess) {
        archive_state[slot] = LRR_ARCHIVE_FREE;
        return std::string("archive copy: ") + hipGetErrorString(status);
      }
      archive_state[slot] = LRR_ARCHIVE_ARCHIVING;
      const int added = lra_add(archive, host_archive_metadata + slot * capacity * 3,
                                host_archive_payload + slot * capacity * 2 * dim, job.count);
      const std::string message = added ? std::string("archive: ") + lra_last_error() : "";
      refresh_archive_counters();
      archive_state[slot] = LRR_ARCHIVE_FREE;
      return message;
    }
    // search
    hipError_t status = hipEventSynchronize(query_copied[slot]);
    if (status != hipSuccess) {
      query_state[slot] = LRR_QUERY_FREE;
      return std::string("query copy: ") + hipGetErrorString(status);
    }
    query_state[slot] = LRR_QUERY_SEARCHING;
    int64_t found = 0;
    int64_t* metadata = host_result_metadata + slot * result_capacity * 3;
    uint16_t* payload = host_result_payload + slot * result_capacity * 2 * dim;
    const int searched = lra_search(archive, host_queries + slot * layers * heads * dim, topk,
                                    metadata, payload, &found);
    refresh_archive_counters();
    if (searched) {
      query_state[slot] = LRR_QUERY_FREE;
      return std::string("search: ") + lra_last_error();
    }
    counters[LRR_COUNTER_SEARCHES] += 1;
    counters[LRR_COUNTER_RETRIEVED] += found;
    result_count[slot] = found;
    if (found == 0) {
      query_state[slot] = LRR_QUERY_FREE;
      return "";
    }
    const size_t payload_bytes = static_cast<size_t>(found * 2 * dim) * 2;
    const size_t metadata_bytes = static_cast<size_t>(found * 3) * 8;
    status = hipMemcpyAsync(device_result_payload + slot * result_payload_bytes(), payload,
                            payload_bytes, hipMemcpyHostToDevice, in_stream);
    if (status == hipSuccess)
      status = hipMemcpyAsync(device_result_metadata + slot * result_metadata_bytes(), metadata,
                              metadata_bytes, hipMemcpyHostToDevice, in_stream);
    if (status == hipSuccess) status = hipEventRecord(result_copied[slot], in_stream);
    if (status != hipSuccess) {
      query_state[slot] = LRR_QUERY_FREE;
      return std::string("result copy: ") + hipGetErrorString(status);
    }
    counters[LRR_COUNTER_H2D_BYTES] += static_cast<int64_t>(payload_bytes + metadata_bytes);
    query_state[slot].store(LRR_QUERY_RESULT, std::memory_order_release);
    return "";
  }

  void run() {
    (void)hipSetDevice(device);
    for (;;) {
      Job job;
      {
        std::unique_lock<std::mutex> lock(mutex);
        changed.wait(lock, [&] { return stop || !jobs.empty(); });
        if (jobs.empty()) break;  // stop requested and nothing left to run
        job = std::move(jobs.front());
        jobs.pop_front();
        busy = true;
      }
      std::string message = execute(job);
      {
        std::lock_guard<std::mutex> lock(mutex);
        busy = false;
        if (!message.empty() && worker_error.empty()) worker_error = std::move(message);
      }
      changed.notify_all();
    }
    alive = false;
  }

  // Waits (with the mutex held by `lock`) until no job is queued or running.
  bool wait_idle(std::unique_lock<std::mutex>& lock, double timeout_seconds) {
    return changed.wait_for(lock, std::chrono::duration<double>(timeout_seconds),
                            [&] { return jobs.empty() && !busy; });
  }
};

Ring* as_ring(void* ring) { return static_cast<Ring*>(ring); }

bool valid_slot(const Ring* r, int slot, bool archive) {
  return slot >= 0 && slot < (archive ? r->archive_slots : 2);
}

void destroy(Ring* r) {
  if (r->worker.joinable()) {
    {
      std::lock_guard<std::mutex> lock(r->mutex);
      r->stop = true;
    }
    r->changed.notify_all();
    r->worker.join();
  }
  (void)hipSetDevice(r->device);
  if (r->out_stream) (void)hipStreamSynchronize(r->out_stream);
  if (r->in_stream) (void)hipStreamSynchronize(r->in_stream);
  for (hipEvent_t e : r->archive_ready) if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : r->archive_copied) if (e) (void)hipEventDestroy(e);
  for (int s = 0; s < 2; ++s)
    for (hipEvent_t e : {r->query_ready[s], r->query_copied[s], r->result_copied[s],
                         r->result_released[s]})
      if (e) (void)hipEventDestroy(e);
  if (r->out_stream) (void)hipStreamDestroy(r->out_stream);
  if (r->in_stream) (void)hipStreamDestroy(r->in_stream);
  if (r->archive) lra_destroy(r->archive);
  delete r;
}

int make_event(hipEvent_t* event) {
  LRR_HIP(hipEventCreateWithFlags(event, hipEventDisableTiming));
  return LRR_OK;
}

int setup(Ring* r, int64_t archive_capacity_per_head, int threads) {
  LRR_HIP(hipSetDevice(r->device));
  // default priority (hipStreamNonBlocking: no implicit order with the null stream)
  LRR_HIP(hipStreamCreateWithFlags(&r->out_stream, hipStreamNonBlocking));
  LRR_HIP(hipStreamCreateWithFlags(&r->in_stream, hipStreamNonBlocking));
  r->archive_ready.assign(static_cast<size_t>(r->archive_slots), nullptr);
  r->archive_copied.assign(static_cast<size_t>(r->archive_slots), nullptr);
  for (int64_t s = 0; s < r->archive_slots; ++s) {
    if (int status = make_event(&r->archive_ready[s])) return status;
    if (int status = make_event(&r->archive_copied[s])) return status;
  }
  for (int s = 0; s < 2; ++s)
    for (hipEvent_t* e : {&r->query_ready[s], &r->query_copied[s], &r->result_copied[s],
                          &r->result_released[s]})
      if (int status = make_event(e)) return status;
  r->archive = lra_create(r->layers, r->heads, r->dim, archive_capacity_per_head, threads);
  if (r->archive == nullptr) return fail(LRR_ERR_INVALID, lra_last_error());
  r->alive = true;
  r->worker = std::thread([r] { r->run(); });
  return LRR_OK;
}

}  // namespace

extern "C" const char* lrr_last_error(void) { return g_error.c_str(); }

extern "C" void* lrr_create(int64_t layers, int64_t heads, int64_t dim, int64_t topk,
                            int64_t archive_slots, int64_t capacity, int64_t result_capacity,
                            int64_t archive_capacity_per_head, int threads, int device,
                            uint16_t* host_archive_payload, int64_t* host_archive_metadata,
                            float* host_queries, uint16_t* host_result_payload,
                            int64_t* host_result_metadata, void* device_archive_payload,
                            void* device_archive_metadata, void* device_queries,
                            void* device_result_payload, void* device_result_metadata) {
  g_error.clear();
  if (layers <= 0 || heads <= 0 || dim <= 0 || topk <= 0 || archive_slots <= 0 || capacity <= 0 ||
      result_capacity < layers * heads * topk || threads <= 0 || device < 0) {
    fail(LRR_ERR_INVALID, "Invalid recall configuration");
    return nullptr;
  }
  if (!host_archive_payload || !host_archive_metadata || !host_queries || !host_result_payload ||
      !host_result_metadata || !device_archive_payload || !device_archive_metadata ||
      !device_queries || !device_result_payload || !device_result_metadata) {
    fail(LRR_ERR_INVALID, "Invalid recall staging buffers");
    return nullptr;
  }
  Ring* r = new Ring();
  r->layers = layers;
  r->heads = heads;
  r->dim = dim;
  r->topk = topk;
  r->archive_slots = archive_slots;
  r->capacity = capacity;
  r->result_capacity = result_capacity;
  r->device = device;
  r->host_archive_payload = host_archive_payload;
  r->host_archive_metadata = host_archive_metadata;
  r->host_queries = host_queries;
  r->host_result_payload = host_result_payload;
  r->host_result_metadata = host_result_metadata;
  r->device_archive_payload = static_cast<char*>(device_archive_payload);
  r->device_archive_metadata = static_cast<char*>(device_archive_metadata);
  r->device_queries = static_cast<char*>(device_queries);
  r->device_result_payload = static_cast<char*>(device_result_payload);
  r->device_result_metadata = static_cast<char*>(device_result_metadata);
  r->archive_state.reset(new std::atomic<int>[static_cast<size_t>(archive_slots)]);
  for (int64_t s = 0; s < archive_slots; ++s) r->archive_state[s] = LRR_ARCHIVE_FREE;
  for (int s = 0; s < 2; ++s) {
    r->query_state[s] = LRR_QUERY_FREE;
    r->query_step[s] = 0;
    r->result_count[s] = 0;
  }
  for (auto& counter : r->counters) counter = 0;
  if (setup(r, archive_capacity_per_head, threads) != LRR_OK) {
    const std::string message = g_error;
    destroy(r);
    g_error = message;
    return nullptr;
  }
  return r;
}

extern "C" void lrr_destroy(void* ring) {
  if (ring) destroy(as_ring(ring));
}

extern "C" int lrr_acquire_archive(void* ring, double timeout_seconds, int* slot, int* waited) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && slot && waited, "Invalid recall ring");
  *slot = -1;
  *waited = 0;
  if (int status = r->take_worker_error()) return status;
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::duration<double>(timeout_seconds);
  std::unique_lock<std::mutex> lock(r->mutex);
  for (;;) {
    for (int64_t s = 0; s < r->archive_slots; ++s) {
      int expected = LRR_ARCHIVE_FREE;
      if (r->archive_state[s].compare_exchange_strong(expected, LRR_ARCHIVE_FILLING)) {
        *slot = static_cast<int>(s);
        return LRR_OK;
      }
    }
    *waited = 1;
    if (!r->worker_error.empty()) {
      lock.unlock();
      return r->take_worker_error();
    }
    // the worker notifies after every job, which is when an archive slot comes free
    if (r->changed.wait_until(lock, deadline) == std::cv_status::timeout &&
        std::chrono::steady_clock::now() >= deadline)
      return fail(LRR_ERR_TIMEOUT, "CPU archive backpressure exceeded timeout");
  }
}

extern "C" int lrr_abandon_archive(void* ring, int slot) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && valid_slot(r, slot, true), "Invalid archive slot");
  int expected = LRR_ARCHIVE_FILLING;
  LRR_CHECK(r->archive_state[slot].compare_exchange_strong(expected, LRR_ARCHIVE_FREE),
            "Archive slot is not being filled");
  r->changed.notify_all();
  return LRR_OK;
}

extern "C" int lrr_commit_archive(void* ring, int slot, int64_t count, void* stream) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && valid_slot(r, slot, true), "Invalid archive slot");
  LRR_CHECK(r->archive_state[slot] == LRR_ARCHIVE_FILLING, "Archive slot is not being filled");
  LRR_CHECK(count > 0 && count <= r->capacity,
            "Eviction batch exceeds configured archive staging capacity");
  const size_t payload_bytes = static_cast<size_t>(count * 2 * r->dim) * 2;
  const size_t metadata_bytes = static_cast<size_t>(count * 3) * 8;
  LRR_HIP(hipEventRecord(r->archive_ready[slot], static_cast<hipStream_t>(stream)));
  LRR_HIP(hipStreamWaitEvent(r->out_stream, r->archive_ready[slot], 0));
  LRR_HIP(hipMemcpyAsync(r->host_archive_payload + slot * r->capacity * 2 * r->dim,
                         r->device_archive_payload + slot * r->archive_payload_bytes(),
                         payload_bytes, hipMemcpyDeviceToHost, r->out_stream));
  LRR_HIP(hipMemcpyAsync(r->host_archive_metadata + slot * r->capacity * 3,
                         r->device_archive_metadata + slot * r->archive_metadata_bytes(),
                         metadata_bytes, hipMemcpyDeviceToHost, r->out_stream));
  LRR_HIP(hipEventRecord(r->archive_copied[slot], r->out_stream));
  r->archive_state[slot] = LRR_ARCHIVE_COPYING;
  Job job;
  job.kind = kArchiveJob;
  job.slot = slot;
  job.count = count;
  r->push(std::move(job));
  return LRR_OK;
}

extern "C" int lrr_acquire_query(void* ring, int* slot) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && slot, "Invalid recall ring");
  *slot = -1;
  if (int status = r->take_worker_error()) return status;
  for (int s = 0; s < 2; ++s) {
    int expected = LRR_QUERY_FREE;
    if (r->query_state[s].compare_exchange_strong(expected, LRR_QUERY_FILLING)) {
      *slot = s;
      return LRR_OK;
    }
  }
  return LRR_OK;
}

extern "C" int lrr_abandon_query(void* ring, int slot) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && valid_slot(r, slot, false), "Invalid query slot");
  int expected = LRR_QUERY_FILLING;
  LRR_CHECK(r->query_state[slot].compare_exchange_strong(expected, LRR_QUERY_FREE),
            "Query slot is not being filled");
  return LRR_OK;
}

extern "C" int lrr_check(void* ring) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r, "Invalid recall ring");
  return r->take_worker_error();
}

extern "C" int lrr_commit_query(void* ring, int slot, int64_t step, void* stream) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && valid_slot(r, slot, false), "Invalid query slot");
  LRR_CHECK(r->query_state[slot] == LRR_QUERY_FILLING, "Query slot is not being filled");
  LRR_HIP(hipEventRecord(r->query_ready[slot], static_cast<hipStream_t>(stream)));
  LRR_HIP(hipStreamWaitEvent(r->out_stream, r->query_ready[slot], 0));
  LRR_HIP(hipMemcpyAsync(r->host_queries + slot * r->layers * r->heads * r->dim,
                         r->device_queries + slot * r->query_bytes(), r->query_bytes(),
                         hipMemcpyDeviceToHost, r->out_stream));
  LRR_HIP(hipEventRecord(r->query_copied[slot], r->out_stream));
  r->query_step[slot] = step;
  r->result_count[slot] = 0;
  r->query_state[slot] = LRR_QUERY_COPYING;
  Job job;
  job.kind = kSearchJob;
  job.slot = slot;
  r->push(std::move(job));
  return LRR_OK;
}

extern "C" int lrr_result_ready(void* ring, int slot) {
  Ring* r = as_ring(ring);
  if (!r || !valid_slot(r, slot, false)) return 0;
  if (r->query_state[slot].load(std::memory_order_acquire) != LRR_QUERY_RESULT) return 0;
  return hipEventQuery(r->result_copied[slot]) == hipSuccess ? 1 : 0;
}

extern "C" int lrr_release_result(void* ring, int slot, void* stream) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && valid_slot(r, slot, false), "Invalid query slot");
  LRR_CHECK(r->query_state[slot] == LRR_QUERY_RESULT, "Query slot holds no result");
  LRR_HIP(hipEventRecord(r->result_released[slot], static_cast<hipStream_t>(stream)));
  r->query_state[slot] = LRR_QUERY_RETIRING;
  return LRR_OK;
}

extern "C" int lrr_drop_result(void* ring, int slot) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && valid_slot(r, slot, false), "Invalid query slot");
  LRR_CHECK(lrr_result_ready(ring, slot), "Query slot holds no finished result");
  r->query_state[slot] = LRR_QUERY_FREE;
  return LRR_OK;
}

extern "C" int lrr_retire(void* ring) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r, "Invalid recall ring");
  for (int s = 0; s < 2; ++s)
    if (r->query_state[s] == LRR_QUERY_RETIRING && hipEventQuery(r->result_released[s]) == hipSuccess)
      r->query_state[s] = LRR_QUERY_FREE;
  return LRR_OK;
}

extern "C" int lrr_remove(void* ring, const int64_t* metadata, int64_t count) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && count >= 0 && (count == 0 || metadata), "Invalid removal");
  if (int status = r->take_worker_error()) return status;
  if (count == 0) return LRR_OK;
  Job job;
  job.kind = kRemoveJob;
  job.metadata.assign(metadata, metadata + 3 * count);
  r->push(std::move(job));
  return LRR_OK;
}

extern "C" int lrr_flush(void* ring, double timeout_seconds) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r, "Invalid recall ring");
  {
    std::unique_lock<std::mutex> lock(r->mutex);
    if (!r->wait_idle(lock, timeout_seconds))
      return fail(LRR_ERR_TIMEOUT, "CPU archive flush exceeded timeout");
  }
  return r->take_worker_error();
}

extern "C" int lrr_wait_pending(void* ring, double timeout_seconds) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r, "Invalid recall ring");
  const auto started = std::chrono::steady_clock::now();
  {
    std::unique_lock<std::mutex> lock(r->mutex);
    if (!r->wait_idle(lock, timeout_seconds))
      return fail(LRR_ERR_TIMEOUT, "Recall diagnostic wait exceeded timeout");
  }
  if (int status = r->take_worker_error()) return status;
  for (int s = 0; s < 2; ++s) {
    if (r->query_state[s].load(std::memory_order_acquire) != LRR_QUERY_RESULT) continue;
    while (hipEventQuery(r->result_copied[s]) == hipErrorNotReady) {
      if (std::chrono::duration<double>(std::chrono::steady_clock::now() - started).count() >
          timeout_seconds)
        return fail(LRR_ERR_TIMEOUT, "Recall diagnostic wait exceeded timeout");
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
  }
  return LRR_OK;
}

extern "C" int lrr_archive_state(void* ring, int slot) {
  Ring* r = as_ring(ring);
  return r && valid_slot(r, slot, true) ? r->archive_state[slot].load() : -1;
}

extern "C" int lrr_query_state(void* ring, int slot) {
  Ring* r = as_ring(ring);
  return r && valid_slot(r, slot, false) ? r->query_state[slot].load() : -1;
}

extern "C" int64_t lrr_query_step(void* ring, int slot) {
  Ring* r = as_ring(ring);
  return r && valid_slot(r, slot, false) ? r->query_step[slot].load() : -1;
}

extern "C" int64_t lrr_result_count(void* ring, int slot) {
  Ring* r = as_ring(ring);
  return r && valid_slot(r, slot, false) ? r->result_count[slot].load() : -1;
}

extern "C" int lrr_counters(void* ring, int64_t* out) {
  g_error.clear();
  Ring* r = as_ring(ring);
  LRR_CHECK(r && out, "Invalid recall ring");
  for (int i = 0; i < LRR_COUNTERS; ++i) out[i] = r->counters[i].load();
  return LRR_OK;
}

extern "C" int lrr_worker_alive(void* ring) {
  Ring* r = as_ring(ring);
  return r && r->alive.load() ? 1 : 0;
}
