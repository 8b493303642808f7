// hkv_device_ops.hpp -- device-side predicate and traversal kernels over a
// table's raw view, for callers compiled with hipcc.
//
// The reference instantiates these operations with the caller's device
// functor (include/hkv_hashtable.h:2409-2447 erase_if / erase_if_v2,
// :2623-2719 export_batch_if / export_batch_if_v2, :2755-2772 for_each,
// :2829-2845 size_if; kernels in include/kernels/remove_kernel/remove_kernel.h:116-215,
// dump_kernel/dump_kernel_if.h, dump_kernel_if_v2.h,
// traverse_kernel/traverse_kernel.h:31-49, size_if_kernel/size_if_kernel.h).
// A functor is device code of the caller, so the kernels are templates in
// this header: the C++ facade (hkv_hashtable.hpp) launches them on the view
// that hkv_device_view_get() returns, and libhkv_amd instantiates the same
// templates with its built-in predicates for the C ABI (hkv_erase_if,
// hkv_size_if, hkv_export_batch_if).
//
// One lane per slot.  Functors receive lvalues: `key`, `score` (v1 and
// size_if: also `pattern`, `threshold`), a `V*` to the slot's row, and the
// reference's cooperative-group size as 1 (each lane evaluates its own slot).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hkv_amd.h"

namespace hkv_ops {

constexpr uint64_t kReclaimKey = 0xFFFFFFFFFFFFFFFEull;
constexpr int kBlock = 256;

__host__ __device__ inline bool is_reserved_word(uint64_t k) {
  return (k & 0xFFFFFFFFFFFFFFFCull) == 0xFFFFFFFFFFFFFFFCull;
}

__device__ inline uint8_t* row_of(const hkv_device_view& v, uint64_t g) {
  const uint64_t b = g >> v.bucket_shift, s = g & (v.max_bucket_size - 1);
  const uint64_t mask = (1ull << v.slice_shift) - 1;
  return v.slices[b >> v.slice_shift] + ((b & mask) * v.max_bucket_size + s) * v.row_bytes;
}

// Wave-aggregated count: one atomic per wave; `live` (optional) takes the
// negated count.
__device__ inline void wave_count(bool m, unsigned long long* counter, unsigned long long* live) {
  const unsigned long long bal = __ballot(m);
  if ((threadIdx.x & 63) == 0 && bal) {
    const unsigned long long c = (unsigned long long)__popcll(bal);
    atomicAdd(counter, c);
    if (live) atomicAdd(live, 0ull - c);
  }
}

// remove_if_kernel (remove_kernel.h:116-160): a matching live slot becomes
// RECLAIM with score 0 and the reclaim digest, and its bucket loses a key.
template <class K, class V, class S, class A>
__global__ __launch_bounds__(kBlock) void k_erase_if(hkv_device_view v, A a,
                                                     unsigned long long* count) {
  const uint64_t g = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  bool m = false;
  if (g < v.capacity) {
    const uint64_t raw = v.slots[2 * g];
    if (!is_reserved_word(raw)) {
      K key = (K)raw;
      S score = (S)v.slots[2 * g + 1];
      V* value = reinterpret_cast<V*>(row_of(v, g));
      if (a(key, value, score)) {
        unsigned long long* kp = reinterpret_cast<unsigned long long*>(v.slots + 2 * g);
        if (atomicCAS(kp, (unsigned long long)raw, (unsigned long long)kReclaimKey) == raw) {
          v.slots[2 * g + 1] = 0;
          v.digests[g] = v.reclaim_digest;
          atomicSub(v.bucket_sizes + (g >> v.bucket_shift), 1);
          m = true;
        }
      }
    }
  }
  wave_count(m, count, reinterpret_cast<unsigned long long*>(v.live));
}

// size_if_kernel: live slots that match.
template <class K, class V, class S, class A>
__global__ __launch_bounds__(kBlock) void k_size_if(hkv_device_view v, A a,
                                                    unsigned long long* count) {
  const uint64_t g = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  bool m = false;
  if (g < v.capacity) {
    const uint64_t raw = v.slots[2 * g];
    if (!is_reserved_word(raw)) {
      K key = (K)raw;
      S score = (S)v.slots[2 * g + 1];
      m = a(key, reinterpret_cast<V*>(row_of(v, g)), score);
    }
  }
  wave_count(m, count, nullptr);
}

// dump_kernel_if / dump_kernel_if_v2: matching live slots of
// [offset, offset + n) appended at the device counter (order unspecified).
template <class K, class V, class S, class A>
__global__ __launch_bounds__(kBlock) void k_export_if(hkv_device_view v, A a, uint64_t offset,
                                                      uint64_t n, unsigned long long* counter,
                                                      K* keys, V* values, S* scores) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const uint64_t g = offset + i;
  bool m = false;
  K key{};
  S score{};
  V* row = nullptr;
  if (i < n) {
    const uint64_t raw = v.slots[2 * g];
    if (!is_reserved_word(raw)) {
      key = (K)raw;
      score = (S)v.slots[2 * g + 1];
      row = reinterpret_cast<V*>(row_of(v, g));
      m = a(key, row, score);
    }
  }
  const unsigned long long bal = __ballot(m);
  const uint32_t lane = threadIdx.x & 63;
  unsigned long long base = 0;
  if (lane == 0 && bal) base = atomicAdd(counter, (unsigned long long)__popcll(bal));
  base = __shfl(base, 0, 64);
  if (m) {
    const uint64_t pos = base + (uint64_t)__popcll(bal & ((1ull << lane) - 1));
    keys[pos] = key;
    if (scores) scores[pos] = score;
    const uint32_t dim = v.row_bytes / (uint32_t)sizeof(V);
    V* dst = values + pos * dim;
    for (uint32_t j = 0; j < dim; j++) dst[j] = row[j];
  }
}

// traverse_kernel (traverse_kernel.h:31-49): f(key, row, &score, 1) on every
// slot of [first, first + n), live or not, as in the reference.
template <class K, class V, class S, class F>
__global__ __launch_bounds__(kBlock) void k_for_each(hkv_device_view v, F f, uint64_t first,
                                                     uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const uint64_t g = first + i;
  const K key = (K)v.slots[2 * g];
  S* score = reinterpret_cast<S*>(v.slots + 2 * g + 1);
  V* value = reinterpret_cast<V*>(row_of(v, g));
  f(key, value, score, 1);
}

// A template, so that every translation unit including this header may
// instantiate it.
template <class T>
__global__ void k_zero(T* p) {
  *p = 0;
}

/* ---- functor adapters: every kernel calls a(key, row, score) ------------ */

// v1 predicates: PredFunctor<K, S>{}(key, score, pattern, threshold),
// constructed in the kernel as the reference does.
template <class K, class V, class S, template <typename, typename> class P>
struct PatternPred {
  K pattern;
  S threshold;
  __device__ bool operator()(K& key, V*, S& score) const {
    P<K, S> p;
    K pt = pattern;
    S th = threshold;
    return p(key, score, pt, th);
  }
};

// erase_if_v2: pred(key, row, score, group_size).
template <class K, class V, class S, class P>
struct RowPred {
  P p;
  __device__ bool operator()(K& key, V* row, S& score) { return p(key, row, score, 1); }
};

// export_batch_if_v2: pred.operator()<group_size>(key, row, score).
template <class K, class V, class S, class P>
struct RowPredT {
  P p;
  __device__ bool operator()(K& key, V* row, S& score) {
    return p.template operator()<1>(key, row, score);
  }
};

/* ---- launchers ---------------------------------------------------------- */

inline unsigned blocks_for(uint64_t n) {
  const uint64_t b = (n + kBlock - 1) / kBlock;
  return (unsigned)(b ? b : 1);
}

// Adds the number of erased slots to *count (device); the caller zeroes it.
template <class K, class V, class S, class A>
hipError_t erase_if(const hkv_device_view& v, const A& a, unsigned long long* count,
                    hipStream_t s) {
  if (v.capacity == 0) return hipSuccess;
  hipLaunchKernelGGL((k_erase_if<K, V, S, A>), dim3(blocks_for(v.capacity)), dim3(kBlock), 0,
                     s, v, a, count);
  return hipGetLastError();
}

// Zeroes *count, then counts.
template <class K, class V, class S, class A>
hipError_t size_if(const hkv_device_view& v, const A& a, unsigned long long* count,
                   hipStream_t s) {
  hipLaunchKernelGGL(k_zero<unsigned long long>, dim3(1), dim3(1), 0, s, count);
  if (v.capacity)
    hipLaunchKernelGGL((k_size_if<K, V, S, A>), dim3(blocks_for(v.capacity)), dim3(kBlock), 0,
                       s, v, a, count);
  return hipGetLastError();
}

// Zeroes *counter, then exports matches among slots [offset, offset + n)
// (n clipped to the capacity).
template <class K, class V, class S, class A>
hipError_t export_if(const hkv_device_view& v, const A& a, uint64_t n, uint64_t offset,
                     unsigned long long* counter, K* keys, V* values, S* scores,
                     hipStream_t s) {
  hipLaunchKernelGGL(k_zero<unsigned long long>, dim3(1), dim3(1), 0, s, counter);
  if (offset >= v.capacity) return hipGetLastError();
  if (n > v.capacity - offset) n = v.capacity - offset;
  if (n == 0) return hipGetLastError();
  hipLaunchKernelGGL((k_export_if<K, V, S, A>), dim3(blocks_for(n)), dim3(kBlock), 0, s, v, a,
                     offset, n, counter, keys, values, scores);
  return hipGetLastError();
}

template <class K, class V, class S, class F>
hipError_t for_each(const hkv_device_view& v, const F& f, uint64_t first, uint64_t last,
                    hipStream_t s) {
  if (first >= v.capacity || last > v.capacity || first >= last) return hipSuccess;
  hipLaunchKernelGGL((k_for_each<K, V, S, F>), dim3(blocks_for(last - first)), dim3(kBlock), 0,
                     s, v, f, first, last - first);
  return hipGetLastError();
}

}  // namespace hkv_ops
