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
// One lane per slot at a time.  Functors receive lvalues: `key`, `score` (v1 and
// size_if: also `pattern`, `threshold`), a `V*` to the slot's row, and the
// reference's cooperative-group size as 1 (each lane evaluates its own slot).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hkv_amd.h"

namespace hkv_ops {

constexpr uint64_t kReclaimKey = 0xFFFFFFFFFFFFFFFEull;
constexpr int kBlock = 256;
constexpr int kScanUnroll = 4;  // slots per thread per pass of the scanning kernels

__host__ __device__ inline bool is_reserved_word(uint64_t k) {
  return (k & 0xFFFFFFFFFFFFFFFCull) == 0xFFFFFFFFFFFFFFFCull;
}

// Key (.x) and score (.y) of slot g in one 16-byte load through the global
// address space: the view holds plain pointers, which the compiler would
// otherwise access with slower generic (flat) instructions.
typedef uint64_t slot_pair __attribute__((ext_vector_type(2)));
__device__ inline slot_pair load_slot(const hkv_device_view& v, uint64_t g) {
  return ((const __attribute__((address_space(1))) slot_pair*)v.slots)[g];
}

__device__ inline uint8_t* row_of(const hkv_device_view& v, uint64_t g) {
  const uint64_t b = g >> v.bucket_shift, s = g & (v.max_bucket_size - 1);
  const uint64_t mask = (1ull << v.slice_shift) - 1;
  return v.slices[b >> v.slice_shift] + ((b & mask) * v.max_bucket_size + s) * v.row_bytes;
}

// Block-wide sum of per-thread counts, added to *dst by one atomic per
// block (negated when `negate`).  Every thread of the block calls it.
__device__ inline void block_add(uint32_t c, uint32_t* s_w, unsigned long long* dst,
                                 bool negate) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) c += __shfl_xor(c, m, 64);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long t = 0;
    for (int w = 0; w < kBlock / 64; w++) t += s_w[w];
    if (t) atomicAdd(dst, negate ? 0ull - t : t);
  }
}

// remove_if_kernel (remove_kernel.h:116-160): a matching live slot becomes
// RECLAIM with score 0 and the reclaim digest, and its bucket loses a key.
template <class K, class V, class S, class A>
__global__ __launch_bounds__(kBlock) void k_erase_if(hkv_device_view v, A a,
                                                     unsigned long long* count) {
  __shared__ uint32_t s_w[kBlock / 64];
  uint32_t c = 0;
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t g0 = (uint64_t)blockIdx.x * kBlock + threadIdx.x; g0 < v.capacity;
       g0 += kScanUnroll * stride) {
    uint64_t raw[kScanUnroll], sc[kScanUnroll];
#pragma unroll
    for (int q = 0; q < kScanUnroll; q++) {  // independent loads in flight
      const uint64_t g = g0 + q * stride;
      slot_pair r;
      r.x = ~0ull;
      r.y = 0;
      if (g < v.capacity) r = load_slot(v, g);
      raw[q] = r.x;
      sc[q] = r.y;
    }
#pragma unroll
    for (int q = 0; q < kScanUnroll; q++) {
      if (is_reserved_word(raw[q])) continue;
      const uint64_t g = g0 + q * stride;
      K key = (K)raw[q];
      S score = (S)sc[q];
      V* value = reinterpret_cast<V*>(row_of(v, g));
      if (!a(key, value, score)) continue;
      unsigned long long* kp = reinterpret_cast<unsigned long long*>(v.slots + 2 * g);
      if (atomicCAS(kp, (unsigned long long)raw[q], (unsigned long long)kReclaimKey) ==
          raw[q]) {
        v.slots[2 * g + 1] = 0;
        v.digests[g] = v.reclaim_digest;
        atomicSub(v.bucket_sizes + (g >> v.bucket_shift), 1);
        c++;
      }
    }
  }
  block_add(c, s_w, count, false);
  __syncthreads();
  block_add(c, s_w, reinterpret_cast<unsigned long long*>(v.live), true);
}

// size_if_kernel: live slots that match.
template <class K, class V, class S, class A>
__global__ __launch_bounds__(kBlock) void k_size_if(hkv_device_view v, A a,
                                                    unsigned long long* count) {
  __shared__ uint32_t s_w[kBlock / 64];
  uint32_t c = 0;
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t g0 = (uint64_t)blockIdx.x * kBlock + threadIdx.x; g0 < v.capacity;
       g0 += kScanUnroll * stride) {
    uint64_t raw[kScanUnroll], sc[kScanUnroll];
#pragma unroll
    for (int q = 0; q < kScanUnroll; q++) {  // independent loads in flight
      const uint64_t g = g0 + q * stride;
      slot_pair r;
      r.x = ~0ull;
      r.y = 0;
      if (g < v.capacity) r = load_slot(v, g);
      raw[q] = r.x;
      sc[q] = r.y;
    }
#pragma unroll
    for (int q = 0; q < kScanUnroll; q++) {
      if (is_reserved_word(raw[q])) continue;
      K key = (K)raw[q];
      S score = (S)sc[q];
      if (a(key, reinterpret_cast<V*>(row_of(v, g0 + q * stride)), score)) c++;
    }
  }
  block_add(c, s_w, count, false);
}

// dump_kernel_if / dump_kernel_if_v2: matching live slots of
// [offset, offset + n).  A block owns kExportPer * kBlock consecutive slots:
// it evaluates the predicate once per slot, reserves its output range with
// one atomic, and each wave copies its matched rows cooperatively (one row
// at a time, lanes across the row).  Order across blocks is unspecified.
constexpr int kExportPer = 16;

template <class K, class V, class S, class A>
__global__ __launch_bounds__(kBlock) void k_export_if(hkv_device_view v, A a, uint64_t offset,
                                                      uint64_t n, unsigned long long* counter,
                                                      K* keys, V* values, S* scores) {
  __shared__ uint32_t s_w[kBlock / 64];
  __shared__ unsigned long long s_base;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t c0 = (uint64_t)blockIdx.x * kBlock * kExportPer;
  uint32_t mask = 0;
#pragma unroll
  for (int j = 0; j < kExportPer; j++) {
    const uint64_t i = c0 + (uint64_t)j * kBlock + tid;
    if (i >= n) continue;
    const uint64_t g = offset + i;
    const slot_pair r = load_slot(v, g);
    if (is_reserved_word(r.x)) continue;
    K key = (K)r.x;
    S score = (S)r.y;
    if (a(key, reinterpret_cast<V*>(row_of(v, g)), score)) mask |= 1u << j;
  }
  // Exclusive prefix of the per-thread counts over the block.
  const uint32_t cnt = (uint32_t)__popc(mask);
  uint32_t x = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(x, d, 64);
    if (lane >= (uint32_t)d) x += y;
  }
  if (lane == 63) s_w[wv] = x;
  __syncthreads();
  uint32_t pre = x - cnt, tot = 0;
  for (uint32_t q = 0; q < kBlock / 64; q++) {
    pre += q < wv ? s_w[q] : 0u;
    tot += s_w[q];
  }
  if (tid == 0) s_base = tot ? atomicAdd(counter, (unsigned long long)tot) : 0ull;
  __syncthreads();
  uint64_t pos = s_base + pre;
  const uint32_t dim = v.row_bytes / (uint32_t)sizeof(V);
#pragma unroll 1
  for (int j = 0; j < kExportPer; j++) {
    const bool m = (mask >> j) & 1u;
    const uint64_t g = offset + c0 + (uint64_t)j * kBlock + tid;
    uint64_t src = 0;
    if (m) {
      const slot_pair r = load_slot(v, g);
      keys[pos] = (K)r.x;
      if (scores) scores[pos] = (S)r.y;
      src = (uint64_t)(uintptr_t)row_of(v, g);
    }
    const uint64_t my_pos = pos;
    pos += m ? 1 : 0;
    unsigned long long bal = __ballot(m);
    while (bal) {  // up to four rows per pass: all loads, then all stores
      int l[4] = {0, 0, 0, 0};
      int k = 0;
      for (; k < 4 && bal; k++) {
        l[k] = __ffsll((long long)bal) - 1;
        bal &= bal - 1;
      }
      const V* sr[4];
      V* dr[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        sr[q] = reinterpret_cast<const V*>((uintptr_t)__shfl(src, l[q], 64));
        dr[q] = values + (uint64_t)__shfl(my_pos, l[q], 64) * dim;
      }
      for (uint32_t e = lane; e < dim; e += 64) {
        V t[4];
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (q < k) t[q] = sr[q][e];
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (q < k) dr[q][e] = t[q];
      }
    }
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
inline unsigned stride_blocks(uint64_t n) {
  const unsigned b = blocks_for(n);
  return b < 4096u ? b : 4096u;
}

template <class K, class V, class S, class A>
hipError_t erase_if(const hkv_device_view& v, const A& a, unsigned long long* count,
                    hipStream_t s) {
  if (v.capacity == 0) return hipSuccess;
  hipLaunchKernelGGL((k_erase_if<K, V, S, A>), dim3(stride_blocks(v.capacity)), dim3(kBlock), 0,
                     s, v, a, count);
  return hipGetLastError();
}

// Zeroes *count, then counts.
template <class K, class V, class S, class A>
hipError_t size_if(const hkv_device_view& v, const A& a, unsigned long long* count,
                   hipStream_t s) {
  hipLaunchKernelGGL(k_zero<unsigned long long>, dim3(1), dim3(1), 0, s, count);
  if (v.capacity)
    hipLaunchKernelGGL((k_size_if<K, V, S, A>), dim3(stride_blocks(v.capacity)), dim3(kBlock),
                       0, s, v, a, count);
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
  const uint64_t per = (uint64_t)kBlock * kExportPer;
  hipLaunchKernelGGL((k_export_if<K, V, S, A>), dim3((unsigned)((n + per - 1) / per)),
                     dim3(kBlock), 0, s, v, a, offset, n, counter, keys, values, scores);
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
