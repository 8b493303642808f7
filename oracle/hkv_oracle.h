/*
 * hkv_oracle.h -- host C++ restatement of the HierarchicalKV-ascend table
 * semantics.  TEST INFRASTRUCTURE ONLY: this is the checker that the HIP
 * library is compared against (tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py).  The product path never links or calls it.
 *
 * Semantics: every API applies its batch as if keys were processed one at a
 * time in increasing batch index, each key running the reference kernel's
 * per-key algorithm (probe, claim, eviction tournament, score functor) with
 * no other key in flight.  One LRU clock value is used per API call.
 * Reference citations are given per function in hkv_oracle.cpp.
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hkvo_table hkvo_table;

/* Status codes, identical to the product C-ABI (include/hkv_amd.h). */
enum {
  HKVO_OK = 0,
  HKVO_ERR_INVALID = 1,     /* HkvException-class argument check failed   */
  HKVO_ERR_RUNTIME = 2,     /* std::runtime_error-class failure           */
  HKVO_ERR_UNSUPPORTED = 3, /* feature outside what this build supports   */
};

/* Value element types (same codes as the product C-ABI). */
enum {
  HKVO_F32 = 0, HKVO_F64 = 1, HKVO_F16 = 2, HKVO_BF16 = 3,
  HKVO_I8 = 4, HKVO_U8 = 5, HKVO_I16 = 6, HKVO_U16 = 7,
  HKVO_I32 = 8, HKVO_U32 = 9, HKVO_I64 = 10, HKVO_U64 = 11,
};

hkvo_table* hkvo_create(uint64_t init_capacity, uint64_t max_capacity,
                        uint64_t max_bucket_size, uint64_t dim,
                        int value_type, int strategy, float max_load_factor,
                        int* status);
void hkvo_destroy(hkvo_table* t);
/* Number of host threads used by the bucket-partitioned parallel mode. */
void hkvo_set_threads(hkvo_table* t, int threads);
void hkvo_set_global_epoch(hkvo_table* t, uint64_t epoch);

int hkvo_insert_or_assign(hkvo_table* t, uint64_t n, const uint64_t* keys,
                          const void* values, const uint64_t* scores,
                          int unique_key, int ignore_evict_strategy,
                          uint64_t clock);
int hkvo_find(hkvo_table* t, uint64_t n, const uint64_t* keys, void* values,
              uint8_t* founds, uint64_t* scores);
int hkvo_find_missed(hkvo_table* t, uint64_t n, const uint64_t* keys,
                     void* values, uint64_t* missed_keys,
                     int32_t* missed_indices, int32_t* missed_size,
                     uint64_t* scores);
int hkvo_find_or_insert(hkvo_table* t, uint64_t n, const uint64_t* keys,
                        void* values, const uint64_t* scores, int unique_key,
                        int ignore_evict_strategy, uint64_t clock);
int hkvo_insert_and_evict(hkvo_table* t, uint64_t n, const uint64_t* keys,
                          const void* values, const uint64_t* scores,
                          uint64_t* evicted_keys, void* evicted_values,
                          uint64_t* evicted_scores, uint64_t* evicted_count,
                          int unique_key, int ignore_evict_strategy,
                          uint64_t clock);
int hkvo_accum_or_assign(hkvo_table* t, uint64_t n, const uint64_t* keys,
                         const void* value_or_deltas, const uint8_t* accum,
                         const uint64_t* scores, int ignore_evict_strategy,
                         uint64_t clock);
int hkvo_assign_scores(hkvo_table* t, uint64_t n, const uint64_t* keys,
                       const uint64_t* scores, uint64_t clock);
int hkvo_contains(hkvo_table* t, uint64_t n, const uint64_t* keys,
                  uint8_t* founds);
/* assign (with_scores = 1) and assign_values (with_scores = 0). */
int hkvo_assign(hkvo_table* t, uint64_t n, const uint64_t* keys,
                const void* values, const uint64_t* scores, int with_scores,
                uint64_t clock);
/* Pointer APIs: slot indices (bucket * B + slot) stand for the addresses the
 * product returns; HKVO_NO_SLOT for none. */
#define HKVO_NO_SLOT 0xFFFFFFFFFFFFFFFFull
int hkvo_find_ptr(hkvo_table* t, uint64_t n, const uint64_t* keys,
                  uint64_t* slots, uint8_t* founds, uint64_t* scores);
int hkvo_find_and_update(hkvo_table* t, uint64_t n, const uint64_t* keys,
                         uint64_t* slots, uint8_t* founds, uint64_t* scores,
                         int unique_key, uint64_t clock);
int hkvo_find_or_insert_ptr(hkvo_table* t, uint64_t n, const uint64_t* keys,
                            uint64_t* slots, uint8_t* founds,
                            const uint64_t* scores, int unique_key, int ignore,
                            int keep_locked, uint64_t clock);
int hkvo_lock_keys(hkvo_table* t, uint64_t n, const uint64_t* keys,
                   uint64_t* slots, uint8_t* success, const uint64_t* scores,
                   uint64_t clock);
int hkvo_unlock_keys(hkvo_table* t, uint64_t n, const uint64_t* slots,
                     const uint64_t* keys, uint8_t* success);
int hkvo_erase(hkvo_table* t, uint64_t n, const uint64_t* keys);
/* Predicate APIs with the product's built-in predicate kinds (HKV_PRED_*);
 * key_signed selects int64 keys.  export lists in slot order. */
int hkvo_erase_if(hkvo_table* t, int pred, uint64_t pattern, uint64_t threshold,
                  int key_signed, uint64_t* count);
int hkvo_size_if(hkvo_table* t, int pred, uint64_t pattern, uint64_t threshold,
                 int key_signed, uint64_t* count);
uint64_t hkvo_export_batch_if(hkvo_table* t, int pred, uint64_t pattern,
                              uint64_t threshold, int key_signed, uint64_t n,
                              uint64_t offset, uint64_t* keys, void* values,
                              uint64_t* scores);
int hkvo_set_max_capacity(hkvo_table* t, uint64_t new_max_capacity);
void hkvo_clear(hkvo_table* t);
uint64_t hkvo_export_batch(hkvo_table* t, uint64_t n, uint64_t offset,
                           uint64_t* keys, void* values, uint64_t* scores);
int hkvo_reserve(hkvo_table* t, uint64_t new_capacity);

uint64_t hkvo_size(hkvo_table* t);
uint64_t hkvo_capacity(hkvo_table* t);
uint64_t hkvo_bucket_count(hkvo_table* t);
/* Raw bucket state (slot-major arrays of capacity() entries). */
void hkvo_raw(hkvo_table* t, const uint8_t** digests, const uint64_t** keys,
              const uint64_t** scores, const int32_t** bucket_sizes,
              const uint8_t** values);

/* Building blocks exposed for known-answer tests. */
uint64_t hkvo_murmur3(uint64_t key);
uint64_t hkvo_global_idx(uint64_t hashed, uint64_t capacity);
uint8_t hkvo_empty_digest(void);
uint8_t hkvo_reclaim_digest(void);
/* Score functor building blocks; `has_in` selects the input-scores pointer
 * being non-null.  Return value is the score written (or `old` if none). */
uint64_t hkvo_score_desired(int strategy, int has_in, uint64_t in,
                            uint64_t epoch, uint64_t clock);
uint64_t hkvo_score_new(int strategy, int has_in, uint64_t in,
                        uint64_t desired, uint64_t old);
uint64_t hkvo_score_hit(int strategy, int has_in, uint64_t in,
                        uint64_t desired, uint64_t old);
uint64_t hkvo_score_without_missed(int strategy, int has_in, uint64_t in,
                                   uint64_t epoch, uint64_t clock,
                                   uint64_t old);

#ifdef __cplusplus
}
#endif
