/*
 * lazyrecall_recall.h — C ABI of liblazyrecall_recall.so: the host side of the recall transport
 * (src/lazy_recall/recall/transport.py:46-361, RecallTransport, with the CPU worker of
 * recall/cpu_worker.py:136-182), as one native object.
 *
 * A ring owns two copy streams of default priority (device->host and host->device), one event
 * per copy and per consumer release, the state of every staging slot, the recall archive
 * (liblazyrecall_archive.so) and one worker thread. The caller owns the buffers: pinned host
 * staging and device staging of the shapes given at creation, which must outlive the ring.
 *
 * Archive slots: free -> filling (lrr_acquire_archive: the caller packs the batch into the
 * slot's device staging on its own stream) -> copying (lrr_commit_archive: the copy out waits
 * for an event on the caller's stream) -> archiving (the worker has seen the copy finish) ->
 * free. Query slots: free -> filling -> copying_query (lrr_commit_query) -> searching ->
 * copying_result (the results' copy into device staging is enqueued) -> retiring
 * (lrr_release_result: an event on the consumer's stream) -> free (lrr_retire once that event
 * has passed); a search with no result goes straight back to free. The worker takes jobs in
 * submission order (archive batches, searches, removals), waits for each job's copy event
 * itself and advances the states; the caller never forwards messages.
 *
 * Status: 0 = ok, 1 = invalid argument or state, 2 = HIP error, 3 = timed out, 4 = the worker
 * failed (its message is returned, once). lrr_last_error() gives the calling thread's message.
 */
#ifndef LAZYRECALL_RECALL_H
#define LAZYRECALL_RECALL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LRR_OK 0
#define LRR_ERR_INVALID 1
#define LRR_ERR_HIP 2
#define LRR_ERR_TIMEOUT 3
#define LRR_ERR_WORKER 4

/* Archive slot states */
#define LRR_ARCHIVE_FREE 0
#define LRR_ARCHIVE_FILLING 1
#define LRR_ARCHIVE_COPYING 2
#define LRR_ARCHIVE_ARCHIVING 3
/* Query slot states */
#define LRR_QUERY_FREE 0
#define LRR_QUERY_FILLING 1
#define LRR_QUERY_COPYING 2
#define LRR_QUERY_SEARCHING 3
#define LRR_QUERY_RESULT 4
#define LRR_QUERY_RETIRING 5

/* Worker-side counters (lrr_counters): the keys of transport.py:61-66 the worker updates. */
#define LRR_COUNTER_INDEXED 0
#define LRR_COUNTER_CAPACITY_DROPS 1
#define LRR_COUNTER_SEARCHES 2
#define LRR_COUNTER_RETRIEVED 3
#define LRR_COUNTER_H2D_BYTES 4
#define LRR_COUNTER_PEAK_RSS_KIB 5
#define LRR_COUNTERS 6

const char* lrr_last_error(void);

/* One ring on `device`. Shapes (elements): host/device archive payload [archive_slots, capacity,
 * 2, dim] uint16 and metadata [archive_slots, capacity, 3] i64; queries [2, layers, heads, dim]
 * f32; result payload [2, result_capacity, 2, dim] uint16 and metadata [2, result_capacity, 3]
 * i64 (result_capacity >= layers * heads * topk). NULL on failure. */
void* lrr_create(int64_t layers, int64_t heads, int64_t dim, int64_t topk, int64_t archive_slots,
                 int64_t capacity, int64_t result_capacity, int64_t archive_capacity_per_head,
                 int threads, int device, uint16_t* host_archive_payload,
                 int64_t* host_archive_metadata, float* host_queries,
                 uint16_t* host_result_payload, int64_t* host_result_metadata,
                 void* device_archive_payload, void* device_archive_metadata,
                 void* device_queries, void* device_result_payload,
                 void* device_result_metadata);
/* Drains the queued jobs, stops and joins the worker, releases streams, events and the
 * archive. */
void lrr_destroy(void* ring);

/* A free archive slot, marked filling; waits up to timeout_seconds for one (*waited = 1 if it
 * had to). */
int lrr_acquire_archive(void* ring, double timeout_seconds, int* slot, int* waited);
/* Gives a filling slot back unused. */
int lrr_abandon_archive(void* ring, int slot);
/* The slot's first `count` rows are packed (or will be, by work already on `stream`): copy them
 * out after that work and archive them. */
int lrr_commit_archive(void* ring, int slot, int64_t count, void* stream);

/* A free query slot, marked filling, or *slot = -1 if none is free. */
int lrr_acquire_query(void* ring, int* slot);
/* Gives a filling query slot back unused. */
int lrr_abandon_query(void* ring, int slot);
/* The slot's device queries are written (or will be, by work already on `stream`): copy them
 * out after that work and search; `step` is the decode step they belong to. */
int lrr_commit_query(void* ring, int slot, int64_t step, void* stream);
/* 1 if the slot holds results whose copy into device staging has finished, else 0. */
int lrr_result_ready(void* ring, int slot);
/* Hands a ready slot's results to a consumer running on `stream`: the slot is reused only after
 * the consumer's work enqueued so far. */
int lrr_release_result(void* ring, int slot, void* stream);
/* Drops a ready slot's results that no consumer took (superseded by a newer search). */
int lrr_drop_result(void* ring, int slot);
/* Frees every retiring slot whose consumer work has finished. */
int lrr_retire(void* ring);

/* Queues the removal of `count` identities [count, 3] = (layer, head, position) (copied). */
int lrr_remove(void* ring, const int64_t* metadata, int64_t count);
/* Waits until every queued job has run, then until every result copy has finished. */
int lrr_wait_pending(void* ring, double timeout_seconds);
/* Waits until every queued job has run. */
int lrr_flush(void* ring, double timeout_seconds);

int lrr_archive_state(void* ring, int slot);
int lrr_query_state(void* ring, int slot);
int64_t lrr_query_step(void* ring, int slot);
int64_t lrr_result_count(void* ring, int slot);
/* out [LRR_COUNTERS] */
int lrr_counters(void* ring, int64_t* out);
int lrr_worker_alive(void* ring);
/* LRR_ERR_WORKER with the worker's message if it failed since the last report, else LRR_OK. */
int lrr_check(void* ring);

#ifdef __cplusplus
}
#endif

#endif /* LAZYRECALL_RECALL_H */
