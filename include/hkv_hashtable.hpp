// hkv_hashtable.hpp -- header-only C++ facade of the gfx950 table with the
// reference's API: npu::hkv::HashTable<K, V, S, Strategy> (reference
// include/hkv_hashtable.h:895-3485), HashTableOptions
// (include/hashtable_options.h:33-65), EvictStrategy (:111-119) and the
// exception types of include/debug.h:30-74.  Every method forwards to the C
// ABI in hkv_amd.h; link with libhkv_amd.so.  `aclrtStream` is a HIP stream.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "hkv_amd.h"

#if defined(__HIPCC__)
// Predicate and traversal APIs take device functors: with hipcc their
// kernels are instantiated here from hkv_device_ops.hpp.  The reference's
// functors compile unchanged: its device-function and global-memory
// qualifiers map to HIP's.
#include "hkv_device_ops.hpp"
#ifndef __simt_callee__
#define __simt_callee__ __device__
#endif
#ifndef __gm__
#define __gm__
#endif
#endif

namespace npu {
namespace hkv {

#if defined(__HIPCC__)
// include/types.h:67,153-156: the four reserved key values.
template <class K>
__host__ __device__ inline bool IS_RESERVED_KEY(K key) {
  return hkv_ops::is_reserved_word(static_cast<uint64_t>(key));
}
#endif

using aclrtStream = hipStream_t;

struct EvictStrategy {
  enum EvictStrategyEnum {
    kLru = HKV_LRU,
    kLfu = HKV_LFU,
    kEpochLru = HKV_EPOCH_LRU,
    kEpochLfu = HKV_EPOCH_LFU,
    kCustomized = HKV_CUSTOMIZED,
  };
};

struct HashTableOptions {
  size_t init_capacity = 0;
  size_t max_capacity = 0;
  size_t max_hbm_for_vectors = 0;
  size_t max_bucket_size = 128;
  size_t dim = 64;
  float max_load_factor = 0.5f;
  int block_size = 128;
  int io_block_size = 1024;
  int device_id = -1;
  bool io_by_cpu = false;
  bool use_constant_memory = false;
  int reserved_key_start_bit = 0;
  size_t num_of_buckets_per_alloc = 1;
  bool api_lock = false;
};

class NpuException : public std::runtime_error {
 public:
  explicit NpuException(const std::string& what) : std::runtime_error(what) {}
};

class HkvException : public std::runtime_error {
 public:
  explicit HkvException(const std::string& what) : std::runtime_error(what) {}
};

namespace detail {

inline void hip(hipError_t e) {
  if (e != hipSuccess) throw NpuException(hipGetErrorString(e));
}

inline void check(int rc) {
  if (rc == HKV_OK) return;
  const std::string msg = hkv_last_error();
  switch (rc) {
    case HKV_ERR_INVALID: throw HkvException(msg);
    case HKV_ERR_RUNTIME: throw std::runtime_error(msg);
    case HKV_ERR_UNSUPPORTED: throw std::invalid_argument(msg);
    default: throw NpuException(msg);
  }
}

template <class V> struct value_code;
template <> struct value_code<float> { static constexpr int v = HKV_F32; };
template <> struct value_code<double> { static constexpr int v = HKV_F64; };
template <> struct value_code<int8_t> { static constexpr int v = HKV_I8; };
template <> struct value_code<uint8_t> { static constexpr int v = HKV_U8; };
template <> struct value_code<int16_t> { static constexpr int v = HKV_I16; };
template <> struct value_code<uint16_t> { static constexpr int v = HKV_U16; };
template <> struct value_code<int32_t> { static constexpr int v = HKV_I32; };
template <> struct value_code<uint32_t> { static constexpr int v = HKV_U32; };
template <> struct value_code<int64_t> { static constexpr int v = HKV_I64; };
template <> struct value_code<uint64_t> { static constexpr int v = HKV_U64; };

}  // namespace detail

// Key-value files for save/load (include/types.h:291-464): the same
// interface as the reference's BaseKVFile and LocalKVFile.
template <class K, class V, class S>
class BaseKVFile {
 public:
  virtual ~BaseKVFile() {}
  // Reads up to n records into the buffers; returns the number read.
  virtual size_t read(const size_t n, const size_t dim, K* keys, V* vectors, S* scores) = 0;
  // Writes n records; returns the number written.
  virtual size_t write(const size_t n, const size_t dim, const K* keys, const V* vectors,
                       const S* scores) = 0;
};

// Three raw files (keys, vectors, scores) opened with fopen modes.
template <class K, class V, class S>
class LocalKVFile : public BaseKVFile<K, V, S> {
 public:
  LocalKVFile() {}
  ~LocalKVFile() { close(); }
  bool open(const std::string& keys_path, const std::string& values_path,
            const std::string& scores_path, const char* mode) {
    close();
    f_ = hkv_local_kv_file_open(keys_path.c_str(), values_path.c_str(), scores_path.c_str(),
                                mode);
    return f_ != nullptr;
  }
  void close() noexcept {
    hkv_local_kv_file_close(f_);
    f_ = nullptr;
  }
  size_t read(const size_t n, const size_t dim, K* keys, V* vectors, S* scores) override {
    return hkv_local_kv_file_read(f_, n, dim * sizeof(V), keys, vectors,
                                  reinterpret_cast<uint64_t*>(scores));
  }
  size_t write(const size_t n, const size_t dim, const K* keys, const V* vectors,
               const S* scores) override {
    return hkv_local_kv_file_write(f_, n, dim * sizeof(V), keys, vectors,
                                   reinterpret_cast<const uint64_t*>(scores));
  }

 private:
  hkv_local_kv_file* f_ = nullptr;
};

template <typename K, typename V, typename S = uint64_t,
          int Strategy = EvictStrategy::kLru>
class HashTable {
 public:
  using size_type = size_t;
  using key_type = K;
  using value_type = V;
  using score_type = S;
  static constexpr int evict_strategy = Strategy;

  HashTable() {
    static_assert(std::is_same<K, int64_t>::value || std::is_same<K, uint64_t>::value,
                  "The key_type must be int64_t or uint64_t.");
    static_assert(std::is_same<S, uint64_t>::value, "The score_type must be uint64_t.");
  }
  ~HashTable() {
    if (t_) hkv_destroy(t_);
    if (d_count_) (void)hipFree(d_count_);
  }
  HashTable(const HashTable&) = delete;
  HashTable& operator=(const HashTable&) = delete;

  void init(const HashTableOptions& o) {
    if (t_) return;
    hkv_options c;
    hkv_options_default(&c);
    c.init_capacity = o.init_capacity;
    c.max_capacity = o.max_capacity;
    c.max_hbm_for_vectors = o.max_hbm_for_vectors;
    c.max_bucket_size = o.max_bucket_size;
    c.dim = o.dim;
    c.max_load_factor = o.max_load_factor;
    c.block_size = o.block_size;
    c.io_block_size = o.io_block_size;
    c.device_id = o.device_id;
    c.io_by_cpu = o.io_by_cpu;
    c.use_constant_memory = o.use_constant_memory;
    c.reserved_key_start_bit = o.reserved_key_start_bit;
    c.num_of_buckets_per_alloc = o.num_of_buckets_per_alloc;
    c.api_lock = o.api_lock;
    detail::check(hkv_create(&c, std::is_same<K, int64_t>::value ? HKV_KEY_I64 : HKV_KEY_U64,
                             detail::value_code<V>::v, Strategy, &t_));
  }

  void insert_or_assign(size_type n, const key_type* keys, const value_type* values,
                        const score_type* scores = nullptr, aclrtStream stream = 0,
                        bool unique_key = true, bool ignore_evict_strategy = false) {
    detail::check(hkv_insert_or_assign(t_, n, keys, values, scores, stream, unique_key,
                                       ignore_evict_strategy));
  }

  void insert_and_evict(size_type n, const key_type* keys, const value_type* values,
                        const score_type* scores, key_type* evicted_keys,
                        value_type* evicted_values, score_type* evicted_scores,
                        size_type* d_evicted_counter, aclrtStream stream = 0,
                        bool unique_key = true, bool ignore_evict_strategy = false) {
    detail::check(hkv_insert_and_evict(t_, n, keys, values, scores, evicted_keys,
                                       evicted_values, evicted_scores,
                                       reinterpret_cast<uint64_t*>(d_evicted_counter), stream,
                                       unique_key, ignore_evict_strategy));
  }

  size_type insert_and_evict(size_type n, const key_type* keys, const value_type* values,
                             const score_type* scores, key_type* evicted_keys,
                             value_type* evicted_values, score_type* evicted_scores,
                             aclrtStream stream = 0, bool unique_key = true,
                             bool ignore_evict_strategy = false) {
    if (n == 0) return 0;
    size_type* d = counter();
    zero_counter(d, stream);
    insert_and_evict(n, keys, values, scores, evicted_keys, evicted_values, evicted_scores, d,
                     stream, unique_key, ignore_evict_strategy);
    return read_counter(d, stream);
  }

  void accum_or_assign(size_type n, const key_type* keys, const value_type* value_or_deltas,
                       const bool* accum_or_assigns, const score_type* scores = nullptr,
                       aclrtStream stream = 0, bool ignore_evict_strategy = false) {
    detail::check(hkv_accum_or_assign(t_, n, keys, value_or_deltas,
                                      reinterpret_cast<const uint8_t*>(accum_or_assigns),
                                      scores, stream, ignore_evict_strategy));
  }

  void find_or_insert(size_type n, const key_type* keys, value_type* values,
                      score_type* scores = nullptr, aclrtStream stream = 0,
                      bool unique_key = true, bool ignore_evict_strategy = false) {
    detail::check(hkv_find_or_insert(t_, n, keys, values, scores, stream, unique_key,
                                     ignore_evict_strategy));
  }

  // Pointer overload: value-row addresses instead of row copies; with
  // locked_key_ptrs the keys stay LOCKED for unlock_keys.
  void find_or_insert(size_type n, const key_type* keys, value_type** values, bool* founds,
                      score_type* scores = nullptr, aclrtStream stream = 0,
                      bool unique_key = true, bool ignore_evict_strategy = false,
                      key_type** locked_key_ptrs = nullptr) {
    detail::check(hkv_find_or_insert_ptr(
        t_, n, keys, reinterpret_cast<void**>(values), reinterpret_cast<uint8_t*>(founds),
        scores, stream, unique_key, ignore_evict_strategy,
        reinterpret_cast<void**>(locked_key_ptrs)));
  }

  void lock_keys(size_type n, const key_type* keys, key_type** locked_key_ptrs,
                 bool* success = nullptr, aclrtStream stream = 0,
                 const score_type* scores = nullptr) {
    detail::check(hkv_lock_keys(t_, n, keys, reinterpret_cast<void**>(locked_key_ptrs),
                                reinterpret_cast<uint8_t*>(success), stream, scores));
  }

  void unlock_keys(size_type n, key_type** locked_key_ptrs, const key_type* keys,
                   bool* success = nullptr, aclrtStream stream = 0) {
    detail::check(hkv_unlock_keys(t_, n, reinterpret_cast<void* const*>(locked_key_ptrs), keys,
                                  reinterpret_cast<uint8_t*>(success), stream));
  }

  void assign(size_type n, const key_type* keys, const value_type* values,
              const score_type* scores = nullptr, aclrtStream stream = 0,
              bool unique_key = true) {
    detail::check(hkv_assign(t_, n, keys, values, scores, stream, unique_key));
  }

  // Alias of assign_scores, as in the reference.
  void assign(size_type n, const key_type* keys, const score_type* scores = nullptr,
              aclrtStream stream = 0, bool unique_key = true) {
    assign_scores(n, keys, scores, stream, unique_key);
  }

  void assign_values(size_type n, const key_type* keys, const value_type* values,
                     aclrtStream stream = 0, bool unique_key = true) {
    detail::check(hkv_assign_values(t_, n, keys, values, stream, unique_key));
  }

  void contains(size_type n, const key_type* keys, bool* founds, aclrtStream stream = 0) const {
    detail::check(hkv_contains(t_, n, keys, reinterpret_cast<uint8_t*>(founds), stream));
  }

  void assign_scores(size_type n, const key_type* keys, const score_type* scores = nullptr,
                     aclrtStream stream = 0, bool unique_key = true) {
    detail::check(hkv_assign_scores(t_, n, keys, scores, stream, unique_key));
  }

  void find(size_type n, const key_type* keys, value_type* values, bool* founds,
            score_type* scores = nullptr, aclrtStream stream = 0) const {
    detail::check(hkv_find(t_, n, keys, values, reinterpret_cast<uint8_t*>(founds), scores,
                           stream));
  }

  void find(size_type n, const key_type* keys, value_type* values, key_type* missed_keys,
            int* missed_indices, int* missed_size, score_type* scores = nullptr,
            aclrtStream stream = 0) const {
    detail::check(hkv_find_missed(t_, n, keys, values, missed_keys, missed_indices,
                                  missed_size, scores, stream));
  }

  // Pointer overload of find: value-row addresses (null when missing).
  void find(size_type n, const key_type* keys, value_type** values, bool* founds,
            score_type* scores = nullptr, aclrtStream stream = 0, bool unique_key = true) const {
    detail::check(hkv_find_ptr(t_, n, keys, reinterpret_cast<void**>(values),
                               reinterpret_cast<uint8_t*>(founds), scores, stream, unique_key));
  }

  void find_and_update(size_type n, const key_type* keys, value_type** values, bool* founds,
                       score_type* scores = nullptr, aclrtStream stream = 0,
                       bool unique_key = true) {
    detail::check(hkv_find_and_update(t_, n, keys, reinterpret_cast<void**>(values),
                                      reinterpret_cast<uint8_t*>(founds), scores, stream,
                                      unique_key));
  }

#if defined(__HIPCC__)
  // include/hkv_hashtable.h:2409-2441: PredFunctor<K, S>{}(key, score,
  // pattern, threshold) selects the live slots to erase.
  template <template <typename, typename> class PredFunctor>
  size_type erase_if(const key_type& pattern, const score_type& threshold,
                     aclrtStream stream = 0) {
    hkv_device_view v;
    detail::check(hkv_device_view_get(t_, &v));
    size_type* d = counter();
    zero_counter(d, stream);
    hkv_ops::PatternPred<K, V, S, PredFunctor> a{pattern, threshold};
    detail::hip(hkv_ops::erase_if<K, V, S>(v, a, reinterpret_cast<unsigned long long*>(d),
                                           stream));
    return read_counter(d, stream);
  }

  // include/hkv_hashtable.h:2447-2470: pred(key, row, score, group_size).
  template <typename PredFunctor>
  size_type erase_if_v2(PredFunctor& pred, aclrtStream stream = 0) {
    hkv_device_view v;
    detail::check(hkv_device_view_get(t_, &v));
    size_type* d = counter();
    zero_counter(d, stream);
    hkv_ops::RowPred<K, V, S, PredFunctor> a{pred};
    detail::hip(hkv_ops::erase_if<K, V, S>(v, a, reinterpret_cast<unsigned long long*>(d),
                                           stream));
    return read_counter(d, stream);
  }

  // include/hkv_hashtable.h:2623-2672 (order of the exported tuples is
  // unspecified, as in the reference).
  template <template <typename, typename> class PredFunctor>
  void export_batch_if(const key_type& pattern, const score_type& threshold, size_type n,
                       const size_type offset, size_type* d_counter, key_type* keys,
                       value_type* values, score_type* scores = nullptr,
                       aclrtStream stream = 0) const {
    hkv_device_view v;
    detail::check(hkv_device_view_get(t_, &v));
    hkv_ops::PatternPred<K, V, S, PredFunctor> a{pattern, threshold};
    detail::hip(hkv_ops::export_if<K, V, S>(v, a, n, offset,
                                            reinterpret_cast<unsigned long long*>(d_counter),
                                            keys, values, scores, stream));
  }

  // include/hkv_hashtable.h:2693-2735: pred.operator()<group_size>(key, row,
  // score).
  template <typename PredFunctor>
  void export_batch_if_v2(PredFunctor& pred, size_type n, const size_type offset,
                          size_type* d_counter, key_type* keys, value_type* values,
                          score_type* scores = nullptr, aclrtStream stream = 0) const {
    hkv_device_view v;
    detail::check(hkv_device_view_get(t_, &v));
    hkv_ops::RowPredT<K, V, S, PredFunctor> a{pred};
    detail::hip(hkv_ops::export_if<K, V, S>(v, a, n, offset,
                                            reinterpret_cast<unsigned long long*>(d_counter),
                                            keys, values, scores, stream));
  }

  // include/hkv_hashtable.h:2755-2772: f(key, row, &score, group_size) on
  // every slot of [first, last).
  template <typename ExecutionFunc>
  void for_each(const size_type first, const size_type last, ExecutionFunc& f,
                aclrtStream stream = 0) {
    hkv_device_view v;
    detail::check(hkv_device_view_get(t_, &v));
    detail::hip(hkv_ops::for_each<K, V, S>(v, f, first, last, stream));
  }

  // include/hkv_hashtable.h:2829-2845.
  template <template <typename, typename> class PredFunctor>
  void size_if(const key_type& pattern, const score_type& threshold, size_type* d_counter,
               aclrtStream stream = 0) const {
    hkv_device_view v;
    detail::check(hkv_device_view_get(t_, &v));
    hkv_ops::PatternPred<K, V, S, PredFunctor> a{pattern, threshold};
    detail::hip(hkv_ops::size_if<K, V, S>(v, a, reinterpret_cast<unsigned long long*>(d_counter),
                                          stream));
  }
#endif

  void erase(size_type n, const key_type* keys, aclrtStream stream = 0) {
    detail::check(hkv_erase(t_, n, keys, stream));
  }

  void clear(aclrtStream stream = 0) { detail::check(hkv_clear(t_, stream)); }

  void export_batch(size_type n, size_type offset, size_type* d_counter, key_type* keys,
                    value_type* values, score_type* scores = nullptr,
                    aclrtStream stream = 0) const {
    detail::check(hkv_export_batch(t_, n, offset, reinterpret_cast<uint64_t*>(d_counter),
                                   keys, values, scores, stream));
  }

  size_type export_batch(size_type n, size_type offset, key_type* keys, value_type* values,
                         score_type* scores = nullptr, aclrtStream stream = 0) const {
    size_type* d = const_cast<HashTable*>(this)->counter();
    export_batch(n, offset, d, keys, values, scores, stream);
    return read_counter(d, stream);
  }

  void reserve(size_type new_capacity, aclrtStream stream = 0) {
    detail::check(hkv_reserve(t_, new_capacity, stream));
  }

  void set_global_epoch(uint64_t epoch) { detail::check(hkv_set_global_epoch(t_, epoch)); }

  // include/hkv_hashtable.h:3021-3118: the live records in slot order,
  // written to `file` in chunks of max_workspace_size / (key + score + row).
  size_type save(BaseKVFile<K, V, S>* file, const size_t max_workspace_size = 1L * 1024 * 1024,
                 aclrtStream stream = 0) const {
    uint64_t n = 0;
    detail::check(hkv_save(t_, &kv_write, file, max_workspace_size, stream, &n));
    return n;
  }

  // include/hkv_hashtable.h:3134-3195: chunks read from `file`, each applied
  // as insert_or_assign(unique_key = true, ignore_evict_strategy = true)
  // with the global epoch set to IGNORED (as it stays afterwards).
  size_type load(BaseKVFile<K, V, S>* file, const size_t max_workspace_size = 1L * 1024 * 1024,
                 aclrtStream stream = 0) {
    uint64_t n = 0;
    detail::check(hkv_load(t_, &kv_read, file, max_workspace_size, stream, &n));
    return n;
  }

  size_type size(aclrtStream stream = 0) const {
    uint64_t s = 0;
    detail::check(hkv_size(t_, stream, &s));
    return s;
  }
  float load_factor(aclrtStream stream = 0) const {
    float f = 0;
    detail::check(hkv_load_factor(t_, stream, &f));
    return f;
  }
  // include/hkv_hashtable.h:2784
  bool empty(aclrtStream stream = 0) const { return size(stream) == 0; }

  // include/hkv_hashtable.h:2955-2977
  void set_max_capacity(size_type new_max_capacity) {
    detail::check(hkv_set_max_capacity(t_, new_max_capacity));
  }

  size_type capacity() const { return hkv_capacity(t_); }
  size_type dim() const noexcept { return hkv_dim(t_); }
  size_type max_bucket_size() const noexcept { return hkv_max_bucket_size(t_); }
  size_type bucket_count() const noexcept { return hkv_bucket_count(t_); }
  bool is_pure_hbm_mode() const { return hkv_is_pure_hbm_mode(t_) != 0; }

 private:
  size_type* counter() {
    if (!d_count_) {
      if (hipMalloc(&d_count_, sizeof(size_type)) != hipSuccess)
        throw NpuException("hipMalloc of the counter failed");
    }
    return d_count_;
  }
  static void zero_counter(size_type* d, aclrtStream stream) {
    if (hipMemsetAsync(d, 0, sizeof(size_type), stream) != hipSuccess)
      throw NpuException("hipMemsetAsync failed");
  }
  static size_type read_counter(size_type* d, aclrtStream stream) {
    size_type h = 0;
    if (hipMemcpyAsync(&h, d, sizeof(size_type), hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
      throw NpuException("counter read failed");
    return h;
  }

  static uint64_t kv_write(void* ctx, uint64_t n, uint64_t row_bytes, const void* keys,
                           const void* values, const uint64_t* scores) {
    return static_cast<BaseKVFile<K, V, S>*>(ctx)->write(
        n, row_bytes / sizeof(V), static_cast<const K*>(keys), static_cast<const V*>(values),
        reinterpret_cast<const S*>(scores));
  }
  static uint64_t kv_read(void* ctx, uint64_t n, uint64_t row_bytes, void* keys, void* values,
                          uint64_t* scores) {
    return static_cast<BaseKVFile<K, V, S>*>(ctx)->read(
        n, row_bytes / sizeof(V), static_cast<K*>(keys), static_cast<V*>(values),
        reinterpret_cast<S*>(scores));
  }

  hkv_table* t_ = nullptr;
  size_type* d_count_ = nullptr;
};

}  // namespace hkv
}  // namespace npu
