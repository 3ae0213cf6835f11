/*
 * lazyrecall_archive.h — C ABI of liblazyrecall_archive.so, the CPU-owned bounded exact
 * maximum-inner-product archive of evicted KV rows (the recall worker's ArchiveIndex,
 * src/lazy_recall/recall/cpu_worker.py:17-134, which wraps faiss IndexIDMap2(IndexFlatIP)).
 *
 * One archive per (layer, KV head) segment. Each holds at most `capacity` rows: a bf16 key and
 * value ([2, dim] uint16 payload), its position (the identity) and the key as f32 for the inner
 * products. Adding a position already present replaces it; past capacity, rows are overwritten
 * in ring order (counted as drops); removed rows' slots are reused last-freed first. A search
 * returns, per segment, the min(topk, live rows) rows with the largest f32 inner product with
 * that segment's query, largest first, equal products in the order the rows were indexed.
 *
 * All pointers are host memory. Calls on one handle must not overlap; a search runs its
 * segments on up to `threads` threads. Status: 0 = ok, 1 = invalid argument (nothing changed),
 * with a message from lra_last_error() for the calling thread.
 */
#ifndef LAZYRECALL_ARCHIVE_H
#define LAZYRECALL_ARCHIVE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message describing the last failure on the calling thread ("" if none). */
const char* lra_last_error(void);

/* ArchiveIndex.__init__ (cpu_worker.py:95-99): layers * heads empty archives. NULL on bad
 * arguments. */
void* lra_create(int64_t layers, int64_t heads, int64_t dim, int64_t capacity, int threads);
void lra_destroy(void* archive);

/* ArchiveIndex.add (cpu_worker.py:109-117) / HeadArchive.add (:48-82). metadata [count, 3] i64
 * = (layer, head, position), payload [count, 2, dim] uint16 (bf16 bits: key, value). */
int lra_add(void* archive, const int64_t* metadata, const uint16_t* payload, int64_t count);

/* ArchiveIndex.remove (cpu_worker.py:119-123) / HeadArchive.remove (:37-46). Identities that are
 * not present are ignored. */
int lra_remove(void* archive, const int64_t* metadata, int64_t count);

/* ArchiveIndex.search (cpu_worker.py:125-134). queries [layers * heads, dim] f32 (segment
 * layer * heads + head). Writes up to layers * heads * topk results in segment order:
 * out_metadata [n, 3] = (layer, head, position), out_payload [n, 2, dim]; *out_count = n. */
int lra_search(void* archive, const float* queries, int64_t topk, int64_t* out_metadata,
               uint16_t* out_payload, int64_t* out_count);

/* ArchiveIndex.size / .dropped (cpu_worker.py:101-107). */
int64_t lra_size(void* archive);
int64_t lra_dropped(void* archive);

#ifdef __cplusplus
}
#endif

#endif /* LAZYRECALL_ARCHIVE_H */
