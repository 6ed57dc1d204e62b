/* urb_residency.h -- HBM expert-residency policy: the reference's deterministic per-layer LRU.
 *
 * The mechanics of LayerLruCache (src/runtime/cache.rs:66-519) for callers that keep more
 * experts than HBM holds: each layer keeps at most `capacity` resident experts, a miss evicts
 * the entry with the smallest (last use, key), and the grouped / ordered-batch schedules of the
 * reference (loads of distinct experts collapsed without adding misses or changing the final
 * hot set) are available as plans.  Host code only: a value is an opaque 64-bit handle the
 * caller chooses (an HBM slot index, a device pointer), so the policy owns no memory.  The
 * reference drops a displaced value; here it is handed back to the caller (`evicted`) to be
 * recycled or released.
 *
 * Loads go through a callback that returns 0 on success and any other value on failure; a
 * failing load's code is returned unchanged by the access call.
 *
 * Layer indices are checked (the reference indexes a Vec and panics): with a layer outside
 * [0, layers), or a required pointer NULL, the access calls return URB_ERR_ARGUMENT before
 * changing anything, queries return their empty answer (not resident, capacity 0, no entries,
 * every key a projected miss, no plan), and the other calls change nothing.
 */
#ifndef URB_RESIDENCY_H
#define URB_RESIDENCY_H

#include <stddef.h>
#include <stdint.h>

#include "urb_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ExpertTelemetry (src/runtime/cache.rs:5-28).  Counters saturate. */
typedef struct {
  uint64_t hits, misses, evictions, bytes_read;
  uint64_t resident_experts, resident_bytes;
} urb_lru_telemetry;

/* Loads `key`: sets *value (the handle to keep), *bytes (resident bytes) and *read_bytes;
 * returns 0, or a non-zero error code that the access call returns. */
typedef int (*urb_lru_load_fn)(void *user, uint32_t layer, uint64_t key, uint64_t *value,
                               uint64_t *bytes, uint64_t *read_bytes);

typedef struct urb_lru urb_lru;
typedef struct urb_lru_plan urb_lru_plan;

/* LayerLruCache::with_layer_capacities (cache.rs:95-103): `layers` layers with the given
 * slot counts (the capacity budget is their sum). */
urb_status urb_lru_create(uint32_t layers, const uint32_t *capacities, urb_lru **out);
void urb_lru_destroy(urb_lru *lru);

/* LayerLruCache::access_with_evicted (cache.rs:118-170).  On a hit *value is the resident
 * handle.  On a miss the least recently used entry is evicted first when the layer is full,
 * then `load` runs; *value is the loaded handle, which stays resident (capacity 0: it is also
 * returned through *evicted, being transient).  *has_evicted = 1 when *evicted holds a handle
 * the cache no longer owns -- also when the load failed after an eviction.  Returns 0 or the
 * load's error. */
int urb_lru_access(urb_lru *lru, urb_lru_telemetry *t, uint32_t layer, uint64_t key,
                   urb_lru_load_fn load, void *user, uint64_t *value, uint64_t *evicted,
                   int *has_evicted);

/* contains / peek / layer_is_empty / layer_capacity (cache.rs:172-193, 204-211): peek leaves
 * recency and telemetry alone and returns 1 with *value when resident. */
int urb_lru_contains(const urb_lru *lru, uint32_t layer, uint64_t key);
int urb_lru_peek(const urb_lru *lru, uint32_t layer, uint64_t key, uint64_t *value);
int urb_lru_layer_is_empty(const urb_lru *lru, uint32_t layer);
uint32_t urb_lru_layer_capacity(const urb_lru *lru, uint32_t layer);

/* residency (cache.rs:75-89): resident experts and bytes of one layer. */
void urb_lru_residency(const urb_lru *lru, uint32_t layer, uint64_t *experts, uint64_t *bytes);

/* Resident entries of one layer in storage order: keys, last uses and handles (any output
 * pointer may be NULL; each array holds at least the layer's capacity).  Returns the count. */
size_t urb_lru_entries(const urb_lru *lru, uint32_t layer, uint64_t *keys, uint64_t *last_used,
                       uint64_t *values);

/* The logical clock (each access advances it by one, saturating). */
uint64_t urb_lru_clock(const urb_lru *lru);
void urb_lru_set_clock(urb_lru *lru, uint64_t clock);

/* drain_layer (cache.rs:194-202): evicts every entry of a layer, capacity unchanged; the
 * handles go to values_out (storage order).  Returns their count. */
size_t urb_lru_drain_layer(urb_lru *lru, urb_lru_telemetry *t, uint32_t layer,
                           uint64_t *values_out);

/* can_insert_without_eviction (cache.rs:213-228). */
int urb_lru_can_insert_without_eviction(const urb_lru *lru, uint32_t layer, const uint64_t *keys,
                                        size_t n);

/* projected_misses (cache.rs:369-401): misses of replaying `keys` serially, state unchanged. */
size_t urb_lru_projected_misses(const urb_lru *lru, uint32_t layer, const uint64_t *keys,
                                size_t n);

/* grouped_access_order (cache.rs:230-249): the distinct keys in last-use order when replaying
 * them adds no projected miss; returns 1 and writes *order_n keys to order_out (room for n),
 * or 0 (None). */
int urb_lru_grouped_access_order(const urb_lru *lru, uint32_t layer, const uint64_t *keys,
                                 size_t n, uint64_t *order_out, size_t *order_n);
/* finish_grouped_accesses (cache.rs:251-261), after the grouped keys were accessed: the clock
 * then stands `groups` accesses after the schedule began.  A clock below `groups` (the
 * reference's subtraction would underflow) leaves everything unchanged. */
void urb_lru_finish_grouped_accesses(urb_lru *lru, uint32_t layer, const uint64_t *keys, size_t n,
                                     size_t groups);

/* grouped_access_plan (cache.rs:263-300): NULL when the plan would not save a load (None). */
urb_lru_plan *urb_lru_grouped_access_plan(const urb_lru *lru, uint32_t layer,
                                          const uint64_t *keys, size_t n);
void urb_lru_plan_destroy(urb_lru_plan *plan);
/* The plan's schedule (resident selected keys first, then the loads): writes to order_out
 * (room for the plan's key count), returns the count. */
size_t urb_lru_plan_order(const urb_lru_plan *plan, uint64_t *order_out);
/* access_grouped_with_evicted (cache.rs:302-352): a resident key is a plain access; a missing
 * key is loaded first (a failed load changes nothing), then kept only if it belongs to the
 * plan's final hot set (evicting only an entry outside it), else returned as transient through
 * *evicted.  Same outputs as urb_lru_access. */
int urb_lru_access_grouped(urb_lru *lru, urb_lru_telemetry *t, const urb_lru_plan *plan,
                           uint64_t key, urb_lru_load_fn load, void *user, uint64_t *value,
                           uint64_t *evicted, int *has_evicted);
/* finish_grouped_plan (cache.rs:354-366): publishes the serial schedule's clock and recency. */
void urb_lru_finish_grouped_plan(urb_lru *lru, const urb_lru_plan *plan);

/* prepare_ordered_batch (cache.rs:403-475): for a duplicate-free batch no larger than the
 * layer, evicts now exactly the entries a serial replay would, so the batch's misses can be
 * loaded concurrently and replayed without eviction.  Returns 1 and the evicted handles
 * (eviction order) in evicted_out (room for n), or 0 (None: nothing changed). */
int urb_lru_prepare_ordered_batch(urb_lru *lru, urb_lru_telemetry *t, uint32_t layer,
                                  const uint64_t *keys, size_t n, uint64_t *evicted_out,
                                  size_t *n_evicted);

/* lend_unused_capacity / restore_layer_capacity (cache.rs:477-518): lend a layer every
 * budgeted slot other layers do not occupy (at most `maximum`), returning its steady capacity;
 * restoring trims back to it oldest-first, the handles going to evicted_out (room for the
 * layer's resident count); returns their count. */
uint32_t urb_lru_lend_unused_capacity(urb_lru *lru, uint32_t layer, uint32_t maximum);
size_t urb_lru_restore_layer_capacity(urb_lru *lru, urb_lru_telemetry *t, uint32_t layer,
                                      uint32_t capacity, uint64_t *evicted_out);

#ifdef __cplusplus
}
#endif
#endif
