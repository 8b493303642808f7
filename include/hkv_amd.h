/*
 * hkv_amd.h -- C ABI of the MI355X (gfx950) HierarchicalKV table.
 *
 * Every entry point takes plain pointers and sizes.  Batch buffers (keys,
 * values, scores, founds, outputs) are device-accessible pointers: HBM, or
 * host memory from hipHostMalloc.  All calls are asynchronous on `stream`
 * unless noted, exactly like the reference's HashTable methods they replace.
 *
 * Return value: HKV_OK (0) or an error code; hkv_last_error() gives the
 * message of the last failure on the calling thread.  The C++ facade
 * (hkv_hashtable.hpp) rethrows these as HkvException / NpuException /
 * std::runtime_error, matching the reference's error convention
 * (include/debug.h:30-74).
 *
 * Reference interfaces replaced (paths relative to the reference root):
 *   HashTableOptions            include/hashtable_options.h:33-65
 *   HashTable::init             include/hkv_hashtable.h:962-1042
 *   HashTable::insert_or_assign include/hkv_hashtable.h:1077-1215
 *   HashTable::insert_and_evict include/hkv_hashtable.h:1260-1324, :1368-1396
 *   HashTable::accum_or_assign  include/hkv_hashtable.h:1438-1507
 *   HashTable::find_or_insert   include/hkv_hashtable.h:1526-1632
 *   HashTable::find_or_insert (value and key pointers)
 *                               include/hkv_hashtable.h:1658-1728
 *   HashTable::lock_keys        include/hkv_hashtable.h:1744-1771
 *   HashTable::unlock_keys      include/hkv_hashtable.h:1788-1804
 *   HashTable::assign           include/hkv_hashtable.h:1830-1921
 *   HashTable::assign_scores    include/hkv_hashtable.h:1943-1977
 *   HashTable::assign_values    include/hkv_hashtable.h:2003-2093
 *   HashTable::contains         include/hkv_hashtable.h:2330-2347
 *   HashTable::find             include/hkv_hashtable.h:2113-2152
 *   HashTable::find (missed)    include/hkv_hashtable.h:2175-2220
 *   HashTable::erase_if / erase_if_v2
 *                               include/hkv_hashtable.h:2409-2470
 *   HashTable::export_batch_if / export_batch_if_v2
 *                               include/hkv_hashtable.h:2623-2735
 *   HashTable::for_each         include/hkv_hashtable.h:2755-2772
 *   HashTable::size_if          include/hkv_hashtable.h:2829-2845
 *   HashTable::find (pointers)  include/hkv_hashtable.h:2244-2262
 *   HashTable::find_and_update  include/hkv_hashtable.h:2288-2317
 *   HashTable::erase            include/hkv_hashtable.h:2358-2376
 *   HashTable::clear            include/hkv_hashtable.h:2482-2493
 *   HashTable::export_batch     include/hkv_hashtable.h:2519-2577
 *   HashTable::size             include/hkv_hashtable.h:2792-2819
 *   HashTable::reserve          include/hkv_hashtable.h:2873-2935
 *   HashTable::load_factor      include/hkv_hashtable.h:2945-2947
 *   HashTable::set_max_capacity include/hkv_hashtable.h:2955-2977
 *   HashTable::set_global_epoch include/hkv_hashtable.h:3197
 *   HashTable::save / load      include/hkv_hashtable.h:3021-3195
 *   BaseKVFile / LocalKVFile    include/types.h:291-464
 *   capacity/dim/max_bucket_size/bucket_count/is_pure_hbm_mode accessors
 *                               include/hkv_hashtable.h:2849, :171-871
 * The launch glue it also replaces: include/aclnn_helper.h (reductions),
 * include/simt_vf_dispatcher.h (template dispatch), include/tiling_helper.h.
 */
#ifndef HKV_AMD_H_
#define HKV_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hkv_table hkv_table;
/* A hipStream_t; 0 is the null stream. */
typedef void* hkv_stream;

enum hkv_status {
  HKV_OK = 0,
  HKV_ERR_INVALID = 1,     /* argument/option check (HkvException)        */
  HKV_ERR_RUNTIME = 2,     /* unsupported mode for this call (runtime_error) */
  HKV_ERR_UNSUPPORTED = 3, /* option or argument combination not accepted
                              (std::invalid_argument)                    */
  HKV_ERR_DEVICE = 4,      /* HIP runtime failure (NpuException)          */
};

/* Eviction strategies, include/hkv_hashtable.h:111-119. */
enum hkv_strategy {
  HKV_LRU = 0,
  HKV_LFU = 1,
  HKV_EPOCH_LRU = 2,
  HKV_EPOCH_LFU = 3,
  HKV_CUSTOMIZED = 4,
};

/* Key types (template parameter K). */
enum hkv_key_type { HKV_KEY_U64 = 0, HKV_KEY_I64 = 1 };

/* Value element types (template parameter V). */
enum hkv_value_type {
  HKV_F32 = 0, HKV_F64 = 1, HKV_F16 = 2, HKV_BF16 = 3,
  HKV_I8 = 4, HKV_U8 = 5, HKV_I16 = 6, HKV_U16 = 7,
  HKV_I32 = 8, HKV_U32 = 9, HKV_I64 = 10, HKV_U64 = 11,
};

/* Field-for-field HashTableOptions (include/hashtable_options.h:33-65);
 * the memory-pool sub-options are not carried (the library allocates its
 * scratch itself). */
typedef struct hkv_options {
  uint64_t init_capacity;
  uint64_t max_capacity;
  uint64_t max_hbm_for_vectors; /* bytes; values beyond it go to pinned host */
  uint64_t max_bucket_size;     /* 128 */
  uint64_t dim;                 /* 64 */
  float max_load_factor;        /* 0.5 */
  int32_t block_size;           /* accepted, not used */
  int32_t io_block_size;        /* accepted, not used */
  int32_t device_id;            /* -1: current device */
  int32_t io_by_cpu;            /* must be 0 */
  int32_t use_constant_memory;  /* reserved */
  int32_t reserved_key_start_bit;
  uint64_t num_of_buckets_per_alloc;
  int32_t api_lock;             /* must be 0 */
} hkv_options;

/* Fills the reference's defaults. */
void hkv_options_default(hkv_options* opt);

/* HashTable<K,V,S=uint64_t,Strategy>::init.  Synchronous. */
int hkv_create(const hkv_options* opt, int key_type, int value_type,
               int strategy, hkv_table** out);
int hkv_destroy(hkv_table* t);

int hkv_insert_or_assign(hkv_table* t, uint64_t n, const void* keys,
                         const void* values, const uint64_t* scores,
                         hkv_stream stream, int unique_key,
                         int ignore_evict_strategy);

/* insert_or_assign without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops).  Same arguments and results as
 * hkv_insert_or_assign; its partition scratch lives in a 64 MiB static
 * device array (one per GPU, kept until the process ends) instead of
 * handle-owned buffers.  Fails with HKV_ERR_INVALID, changing nothing, when
 * the batch needs more than 64 MiB of scratch (batches up to about 6.5e5 keys
 * fit on a 2^26-slot table) or the table is below its maximum capacity (growth allocates).
 * All calls on one GPU share the array: calls that overlap on a GPU race. */
int hkv_insert_or_assign_noalloc(hkv_table* t, uint64_t n, const void* keys,
                                 const void* values, const uint64_t* scores,
                                 hkv_stream stream, int unique_key,
                                 int ignore_evict_strategy);

/* As in the reference, the evicted_* buffers hold n records and
 * `d_evicted_counter` must be 0 at the call: the record count is added to it,
 * and records are written at positions below n before being compacted into
 * [0, count).  insert_and_evict fails (runtime_error) in hybrid mode. */
int hkv_insert_and_evict(hkv_table* t, uint64_t n, const void* keys,
                         const void* values, const uint64_t* scores,
                         void* evicted_keys, void* evicted_values,
                         uint64_t* evicted_scores, uint64_t* d_evicted_counter,
                         hkv_stream stream, int unique_key,
                         int ignore_evict_strategy);

int hkv_accum_or_assign(hkv_table* t, uint64_t n, const void* keys,
                        const void* value_or_deltas,
                        const uint8_t* accum_or_assigns,
                        const uint64_t* scores, hkv_stream stream,
                        int ignore_evict_strategy);

int hkv_find_or_insert(hkv_table* t, uint64_t n, const void* keys,
                       void* values, const uint64_t* scores, hkv_stream stream,
                       int unique_key, int ignore_evict_strategy);

int hkv_assign_scores(hkv_table* t, uint64_t n, const void* keys,
                      const uint64_t* scores, hkv_stream stream,
                      int unique_key);

/* assign: present keys take the input row and update_without_missed on
 * their score (the assign_scores functor); absent keys are no-ops.  With
 * unique_key=0 the scores apply in batch order and, for a repeated key, the
 * row of one of its occurrences lands (unspecified which, as in the
 * reference). */
int hkv_assign(hkv_table* t, uint64_t n, const void* keys, const void* values,
               const uint64_t* scores, hkv_stream stream, int unique_key);

/* assign_values: present keys take the input row; scores are untouched. */
int hkv_assign_values(hkv_table* t, uint64_t n, const void* keys,
                      const void* values, hkv_stream stream, int unique_key);

/* contains: founds only. */
int hkv_contains(hkv_table* t, uint64_t n, const void* keys, uint8_t* founds,
                 hkv_stream stream);

/* Missed rows of `values` are left untouched; `scores` may be NULL. */
int hkv_find(hkv_table* t, uint64_t n, const void* keys, void* values,
             uint8_t* founds, uint64_t* scores, hkv_stream stream);

/* `missed_size` (device int) is cleared by the call. */
int hkv_find_missed(hkv_table* t, uint64_t n, const void* keys, void* values,
                    void* missed_keys, int32_t* missed_indices,
                    int32_t* missed_size, uint64_t* scores, hkv_stream stream);

/* Pointer APIs.  `value_ptrs[i]` receives the address of key i's value row
 * (device-accessible: HBM, or pinned host memory in hybrid mode) or NULL;
 * `key_ptrs` entries are addresses of the table's key words.  Addresses stay
 * valid until the table grows (reserve or automatic growth) or is cleared.
 *
 * find: rows of present keys; `founds` and `scores` may be NULL, scores are
 * written for found keys only.  unique_key is accepted as in the reference. */
int hkv_find_ptr(hkv_table* t, uint64_t n, const void* keys, void** value_ptrs,
                 uint8_t* founds, uint64_t* scores, hkv_stream stream,
                 int unique_key);

/* find_and_update: find, then the hit score functor on each found key
 * (scores are input and output, as in the reference).  unique_key must be
 * 1 (runtime_error otherwise); scores follow the strategy checks. */
int hkv_find_and_update(hkv_table* t, uint64_t n, const void* keys,
                        void** value_ptrs, uint8_t* founds, uint64_t* scores,
                        hkv_stream stream, int unique_key);

/* find_or_insert, pointer overload: places keys exactly like
 * hkv_find_or_insert but moves no rows; a new key's row keeps whatever the
 * slot held, for the caller to write.  `founds` is required.  With
 * unique_key, every slot the batch claims or finds stays LOCKED until the
 * batch ends, so later keys of the batch cannot evict it; with
 * `locked_key_ptrs` non-NULL (unique_key required, invalid_argument
 * otherwise) the keys stay LOCKED after the call and their key addresses
 * are returned for hkv_unlock_keys.  Refused and reserved keys get NULL
 * addresses and founds 0. */
int hkv_find_or_insert_ptr(hkv_table* t, uint64_t n, const void* keys,
                           void** value_ptrs, uint8_t* founds,
                           const uint64_t* scores, hkv_stream stream,
                           int unique_key, int ignore_evict_strategy,
                           void** locked_key_ptrs);

/* lock_keys: a present key's slot key becomes LOCKED (found by find* no
 * more, never evicted) and the hit score functor runs with `scores` (may be
 * NULL except for EpochLfu and Customized).  `success` may be NULL. */
int hkv_lock_keys(hkv_table* t, uint64_t n, const void* keys,
                  void** locked_key_ptrs, uint8_t* success, hkv_stream stream,
                  const uint64_t* scores);

/* unlock_keys: LOCKED -> keys[i] at each address.  An address that is not
 * one of this table's key words, or whose word is not LOCKED, reports 0 in
 * `success` (may be NULL) and is not written. */
int hkv_unlock_keys(hkv_table* t, uint64_t n, void* const* locked_key_ptrs,
                    const void* keys, uint8_t* success, hkv_stream stream);

int hkv_erase(hkv_table* t, uint64_t n, const void* keys, hkv_stream stream);

/* Predicate APIs.  The reference takes the caller's device functor; the C++
 * facade does too (hkv_device_ops.hpp instantiates its kernels with it).  An
 * FFI caller picks one of these built-in predicates on (key, score), with
 * the table's key type:                                                    */
enum {
  HKV_PRED_SCORE_LT = 0,      /* score <  threshold                          */
  HKV_PRED_SCORE_GE = 1,      /* score >= threshold                          */
  HKV_PRED_SCORE_GT = 2,      /* score >  threshold                          */
  HKV_PRED_KEY_MASK_EQ = 3,   /* (key & pattern) == pattern                  */
  HKV_PRED_KEY_LOW7_GT_SCORE_GT = 4, /* (key & 0x7f) > pattern && score > threshold */
};

/* erase_if: matching live slots become RECLAIM.  Synchronous; `count` (host)
 * receives the number erased. */
int hkv_erase_if(hkv_table* t, int pred, uint64_t pattern, uint64_t threshold,
                 hkv_stream stream, uint64_t* count);

/* size_if: `d_counter` (device uint64) receives the number of matches. */
int hkv_size_if(hkv_table* t, int pred, uint64_t pattern, uint64_t threshold,
                uint64_t* d_counter, hkv_stream stream);

/* export_batch_if: matching live slots of [offset, offset + n), appended in
 * an unspecified order; `d_counter` (device uint64) receives the count. */
int hkv_export_batch_if(hkv_table* t, int pred, uint64_t pattern,
                        uint64_t threshold, uint64_t n, uint64_t offset,
                        uint64_t* d_counter, void* keys, void* values,
                        uint64_t* scores, hkv_stream stream);

/* Raw device view of a table, for the predicate and traversal kernels that
 * callers instantiate with their own functors (hkv_device_ops.hpp).  It
 * stands for the reference's Table<K, V, S> members those kernels read
 * (include/types.h:173-248).  Slot g = bucket * max_bucket_size + slot;
 * its key is slots[2g], its score slots[2g + 1]; its row is in
 * slices[bucket >> slice_shift] at ((bucket & ((1 << slice_shift) - 1)) *
 * max_bucket_size + slot) * row_bytes.  Valid until the table grows or is
 * destroyed. */
typedef struct hkv_device_view {
  uint8_t* digests;
  uint64_t* slots;
  int32_t* bucket_sizes;
  uint64_t* live;           /* live-key counter kept by every kernel */
  uint8_t* const* slices;   /* device array of value-slice base addresses */
  uint64_t capacity;
  uint64_t buckets;
  uint32_t max_bucket_size;
  uint32_t bucket_shift;
  uint32_t slice_shift;
  uint32_t row_bytes;
  uint8_t reclaim_digest;
} hkv_device_view;
int hkv_device_view_get(const hkv_table* t, hkv_device_view* out);
int hkv_clear(hkv_table* t, hkv_stream stream);

/* Exports live slots [offset, offset + n) in slot order; `d_counter`
 * (device uint64) receives the count. */
int hkv_export_batch(hkv_table* t, uint64_t n, uint64_t offset,
                     uint64_t* d_counter, void* keys, void* values,
                     uint64_t* scores, hkv_stream stream);

/* Synchronous. */
int hkv_reserve(hkv_table* t, uint64_t new_capacity, hkv_stream stream);

/* set_max_capacity: a power of 2 (invalid_argument otherwise); below the
 * current capacity it does nothing. */
int hkv_set_max_capacity(hkv_table* t, uint64_t new_max_capacity);
/* Key-value files (include/types.h:291-464, BaseKVFile / LocalKVFile): a
 * file is a pair of callbacks over `ctx`.  `row_bytes` = dim * sizeof(V);
 * each returns the number of records read or written. */
typedef uint64_t (*hkv_kv_write_fn)(void* ctx, uint64_t n, uint64_t row_bytes,
                                    const void* keys, const void* values,
                                    const uint64_t* scores);
typedef uint64_t (*hkv_kv_read_fn)(void* ctx, uint64_t n, uint64_t row_bytes,
                                   void* keys, void* values, uint64_t* scores);

/* HashTable::save (include/hkv_hashtable.h:3021-3118): the live records in
 * slot order, exported in chunks of max_workspace_size / (key + score + row)
 * slots and handed to `write`; *count = records written.  Synchronizes
 * `stream`.  Fails if max_workspace_size is below one record. */
int hkv_save(hkv_table* t, hkv_kv_write_fn write, void* ctx,
             uint64_t max_workspace_size, hkv_stream stream, uint64_t* count);

/* HashTable::load (include/hkv_hashtable.h:3134-3195): chunks of
 * max_workspace_size / (key + score + row) records read with `read`, each
 * applied as insert_or_assign(unique_key = true, ignore_evict_strategy =
 * true) after the global epoch is set to IGNORED (which it stays, as in the
 * reference); *count = records read.  Synchronizes `stream`. */
int hkv_load(hkv_table* t, hkv_kv_read_fn read, void* ctx,
             uint64_t max_workspace_size, hkv_stream stream, uint64_t* count);

/* LocalKVFile (include/types.h:350-464): three raw files (keys, rows,
 * scores) opened with fopen `mode`; null if any fails to open.  Its read and
 * write functions are the callbacks above, with the file as `ctx`; a read
 * returns 0 when the three files do not yield the same count. */
typedef struct hkv_local_kv_file hkv_local_kv_file;
hkv_local_kv_file* hkv_local_kv_file_open(const char* keys_path,
                                          const char* values_path,
                                          const char* scores_path,
                                          const char* mode);
void hkv_local_kv_file_close(hkv_local_kv_file* f);
uint64_t hkv_local_kv_file_write(void* f, uint64_t n, uint64_t row_bytes,
                                 const void* keys, const void* values,
                                 const uint64_t* scores);
uint64_t hkv_local_kv_file_read(void* f, uint64_t n, uint64_t row_bytes,
                                void* keys, void* values, uint64_t* scores);

int hkv_set_global_epoch(hkv_table* t, uint64_t epoch);

/* Synchronous (stream is synchronized). */
int hkv_size(hkv_table* t, hkv_stream stream, uint64_t* out);
int hkv_load_factor(hkv_table* t, hkv_stream stream, float* out);

uint64_t hkv_capacity(const hkv_table* t);
uint64_t hkv_dim(const hkv_table* t);
uint64_t hkv_max_bucket_size(const hkv_table* t);
uint64_t hkv_bucket_count(const hkv_table* t);
int hkv_is_pure_hbm_mode(const hkv_table* t);

const char* hkv_last_error(void);

/* Test hook with no reference counterpart: fixes the LRU clock used by
 * Lru/EpochLru (the reference reads a device cycle counter per launch).
 * enable=0 returns to the host monotonic clock read once per call. */
int hkv_set_lru_clock(hkv_table* t, uint64_t clock, int enable);

/* Test hook with no reference counterpart: the live-key count the kernels
 * maintain on the device (it selects the find probe order).  Synchronizes
 * `stream`; equals hkv_size() after every completed call. */
int hkv_live_count(hkv_table* t, hkv_stream stream, uint64_t* out);

/* Test hook with no reference counterpart: host-side addresses of the key
 * word and value row of global slots (bucket * max_bucket_size + slot), for
 * checking returned pointers against a slot layout.  No device work. */
int hkv_slot_addresses(const hkv_table* t, uint64_t n, const uint64_t* slots,
                       void** key_ptrs, void** value_ptrs);

#ifdef __cplusplus
}
#endif
#endif /* HKV_AMD_H_ */
