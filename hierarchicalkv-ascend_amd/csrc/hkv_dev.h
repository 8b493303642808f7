// hkv_dev.h -- device-side building blocks of the gfx950 HierarchicalKV table.
//
// Table layout in HBM (one table):
//   digests  uint8 [buckets][B]     1-byte fingerprints, B = 128 slots/bucket
//   slots    uint64[buckets][B][2]  16-byte slot records {key, score}: a slot's
//                                   key and score share one 32-byte sector
//   bsize    int32 [buckets]        live keys per bucket
//   live     uint64                 live keys in the table (sum of bsize)
//   values   rows of dim*sizeof(V) bytes, one per slot, in value slices:
//            slice = slices[b >> slice_shift], row offset inside the slice =
//            ((b & slice_mask) * B + slot) * row_bytes.  Slices live in HBM
//            or, past max_hbm_for_vectors, in pinned host memory that the
//            kernels dereference directly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hkv {

constexpr uint64_t kEmptyKey = 0xFFFFFFFFFFFFFFFFull;    // types.h:63
constexpr uint64_t kReclaimKey = 0xFFFFFFFFFFFFFFFEull;  // types.h:64
constexpr uint64_t kLockedKey = 0xFFFFFFFFFFFFFFFDull;   // types.h:65
constexpr uint64_t kReservedMask = 0xFFFFFFFFFFFFFFFCull;  // types.h:67
constexpr uint64_t kMaxScore = 0xFFFFFFFFFFFFFFFFull;
constexpr uint64_t kIgnoredEpoch = 0xFFFFFFFFFFFFFFFFull;
constexpr uint64_t kScoreMask = 0xFFFFFFFFull;
constexpr uint64_t kEpochMask = 0xFFFFFFFF00000000ull;
// Digest of the EMPTY and RECLAIM sentinels: (fmix64(key) >> 32) & 0xff.
constexpr uint8_t kEmptyDigest = 0x0b;
constexpr uint8_t kReclaimDigest = 0x88;

enum Strategy { kLru = 0, kLfu = 1, kEpochLru = 2, kEpochLfu = 3, kCustomized = 4 };

__host__ __device__ __forceinline__ bool is_reserved(uint64_t k) {
  return (k & kReservedMask) == kReservedMask;
}

// MurmurHash3 fmix64 (reference include/utils.h:52-71).
__host__ __device__ __forceinline__ uint64_t murmur3(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

// Stored digest of a live key: byte 4 of its hash, except that the value of
// the empty digest moves to the next value.  A slot whose digest equals
// kEmptyDigest therefore holds EMPTY, and probes end or claim a slot on the
// digest alone.  Lookups use the same mapping, so results are unchanged.
__host__ __device__ __forceinline__ uint32_t key_digest(uint64_t h) {
  const uint32_t d = (uint32_t)(h >> 32) & 0xFFu;
  return d == kEmptyDigest ? kEmptyDigest + 1u : d;
}

// Pointers of the global address space.  Kernels reach table and batch
// memory through pointers held in structs or passed between lanes, which the
// compiler would otherwise treat as generic (flat) addresses: flat accesses
// also count against the LDS wait counter and are slower to issue.  Casting
// a generic pointer to global costs nothing on this target.
template <class T>
using gptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> G(T* p) {
  return (gptr<T>)p;
}
template <class T>
__device__ __forceinline__ gptr<T> G(uintptr_t p) {
  return (gptr<T>)p;
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
using g64 = __attribute__((address_space(1))) uint64_t;

struct TableView {
  uint8_t* digests;
  uint64_t* slots;  // record of slot s at slots[2s] (key), slots[2s+1] (score)
  int32_t* bsize;
  unsigned long long* live;
  uint8_t* const* slices;
  uint64_t capacity;
  uint64_t buckets;
  uint64_t qd_magic;   // h mod capacity by magic multiply when not a power of 2
  uint64_t qd_shift;
  uint32_t B;          // slots per bucket (power of 2)
  uint32_t bshift;     // log2(B)
  uint32_t slice_shift;
  uint32_t row_bytes;  // dim * sizeof(V)
  uint32_t pow2;       // capacity is a power of two
};

__device__ __forceinline__ g64& slot_key(const TableView& t, uint64_t s) {
  return G(t.slots)[2 * s];
}
__device__ __forceinline__ g64& slot_score(const TableView& t, uint64_t s) {
  return G(t.slots)[2 * s + 1];
}
// Key (.x) and score (.y) of slot s in one 16-byte load.
__device__ __forceinline__ u64x2 slot_load(const TableView& t, uint64_t s) {
  return G(reinterpret_cast<u64x2*>(t.slots))[s];
}
__device__ __forceinline__ void slot_store(const TableView& t, uint64_t s, uint64_t k,
                                           uint64_t sc) {
  u64x2 v;
  v.x = k;
  v.y = sc;
  G(reinterpret_cast<u64x2*>(t.slots))[s] = v;
}
__device__ __forceinline__ gptr<uint8_t> digest_row(const TableView& t, uint64_t b) {
  return G(t.digests) + b * t.B;
}

// h mod capacity, exactly (reference include/utils.h:86-97 and the divisor
// precomputation in include/table.h:106-127).
__device__ __forceinline__ uint64_t global_idx(const TableView& t, uint64_t h) {
  if (t.pow2) return h & (t.capacity - 1);
  uint64_t q = __umul64hi(h, t.qd_magic);
  q = ((h - q) >> 1) + q;
  return h - (q >> t.qd_shift) * t.capacity;
}

__device__ __forceinline__ gptr<uint8_t> row_ptr(const TableView& t, uint64_t b,
                                                 uint32_t slot) {
  const uint64_t mask = (1ull << t.slice_shift) - 1;
  gptr<uint8_t> base = G(G(t.slices)[b >> t.slice_shift]);
  return base + ((b & mask) * t.B + slot) * (uint64_t)t.row_bytes;
}

// Byte-equality mask of four packed bytes: bit j set when byte j of `w`
// equals the byte replicated in `rep` (exact SWAR test, no cross-byte carry).
__device__ __forceinline__ uint32_t eq_bytes4(uint32_t w, uint32_t rep) {
  const uint32_t x = w ^ rep;
  const uint32_t y = ((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x;
  const uint32_t z = ~y & 0x80808080u;
  return ((z >> 7) & 1u) | ((z >> 14) & 2u) | ((z >> 21) & 4u) | ((z >> 28) & 8u);
}

/* ---- score functors (reference include/score_functor.h) ---------------- */

struct ScoreCtx {
  int strategy;
  uint64_t epoch;
  uint64_t clock;  // one value per API call
};

__device__ __forceinline__ uint64_t score_desired(const ScoreCtx& c, bool has_in,
                                                  uint64_t in) {
  switch (c.strategy) {
    case kLru: return c.clock;
    case kLfu: return kMaxScore;
    case kEpochLru:
      if (c.epoch == kIgnoredEpoch && has_in) return in;
      return (c.epoch << 32) | ((c.clock >> 20) & kScoreMask);
    case kEpochLfu:
      if (c.epoch == kIgnoredEpoch) return in;
      return (c.epoch << 32) | (in & kScoreMask);
    default: return in;
  }
}

// Score of a newly placed key; *w=false when the functor writes nothing.
__device__ __forceinline__ uint64_t score_new(const ScoreCtx& c, bool has_in,
                                              uint64_t in, uint64_t des,
                                              uint64_t old, bool* w) {
  *w = true;
  if (c.strategy == kLfu) {
    if (!has_in) { *w = false; return old; }
    return in;
  }
  return des;
}

// Score of a key found present (update_score_only / update_with_digest with
// new_insert = false).
__device__ __forceinline__ uint64_t score_hit(const ScoreCtx& c, bool has_in,
                                              uint64_t in, uint64_t des,
                                              uint64_t old, bool* w) {
  *w = true;
  if (c.strategy == kLfu) {
    if (!has_in) { *w = false; return old; }
    return in + old;
  }
  if (c.strategy == kEpochLfu) {
    const uint64_t lo = old & kScoreMask;
    if (0xFFFFFFFFull - lo > (des & kScoreMask)) return lo + des;
    return (des & kEpochMask) | 0xFFFFFFFFull;
  }
  return des;
}

// update_without_missed (assign_scores).
__device__ __forceinline__ uint64_t score_wo_missed(const ScoreCtx& c,
                                                    bool has_in, uint64_t in,
                                                    uint64_t old, bool* w) {
  *w = true;
  switch (c.strategy) {
    case kLru: return c.clock;
    case kLfu:
      if (!has_in) { *w = false; return old; }
      return in + old;
    case kEpochLru: return (c.epoch << 32) | ((c.clock >> 20) & kScoreMask);
    case kEpochLfu: {
      if (!has_in) { *w = false; return old; }
      const uint64_t lo = old & kScoreMask;
      if (0xFFFFFFFFull - lo > (in & kScoreMask))
        return lo + ((c.epoch << 32) | (in & kScoreMask));
      return (c.epoch << 32) | 0xFFFFFFFFull;
    }
    default:
      if (!has_in) { *w = false; return old; }
      return in;
  }
}

/* ---- lane helpers ------------------------------------------------------- */

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src, int width) {
  const uint32_t lo = __shfl((uint32_t)v, src, width);
  const uint32_t hi = __shfl((uint32_t)(v >> 32), src, width);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m, int width) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, width);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, width);
  return ((uint64_t)hi << 32) | lo;
}

// Minimum over the 16 lanes of a group.
__device__ __forceinline__ uint32_t group_min_u32(uint32_t v) {
#pragma unroll
  for (int m = 8; m > 0; m >>= 1) {
    const uint32_t o = __shfl_xor(v, m, 16);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ uint32_t bitrev4(uint32_t x) {
  return ((x & 1u) << 3) | ((x & 2u) << 1) | ((x & 4u) >> 1) | ((x & 8u) >> 3);
}

/* ---- cooperative row copies --------------------------------------------- */

template <int U>
struct UnitT;
template <> struct UnitT<16> { using T = u32x4; };
template <> struct UnitT<8> { using T = u32x2; };
template <> struct UnitT<4> { using T = uint32_t; };
template <> struct UnitT<2> { using T = uint16_t; };
template <> struct UnitT<1> { using T = uint8_t; };

// `nl` lanes (rank `r` among them) copy `bytes` from src to dst in U-byte
// units.  Rows are streamed (non-temporal loads and stores), which keeps the
// bucket metadata in the L2 cache.
template <int U>
__device__ __forceinline__ void copy_units(gptr<uint8_t> dst, gptr<const uint8_t> src,
                                           uint32_t bytes, uint32_t r, uint32_t nl) {
  using T = typename UnitT<U>::T;
  const uint32_t units = bytes / U;
  gptr<T> d = (gptr<T>)dst;
  gptr<const T> s = (gptr<const T>)src;
  uint32_t u = r;
  for (; u + 3 * nl < units; u += 4 * nl) {
    const T a = __builtin_nontemporal_load(&s[u]), b = __builtin_nontemporal_load(&s[u + nl]),
            c = __builtin_nontemporal_load(&s[u + 2 * nl]),
            e = __builtin_nontemporal_load(&s[u + 3 * nl]);
    __builtin_nontemporal_store(a, &d[u]);
    __builtin_nontemporal_store(b, &d[u + nl]);
    __builtin_nontemporal_store(c, &d[u + 2 * nl]);
    __builtin_nontemporal_store(e, &d[u + 3 * nl]);
  }
  // At most three units per lane remain: every load is issued before the
  // first store, so the remainder costs one memory round trip.
  if (u < units) {
    const bool o1 = u + nl < units, o2 = u + 2 * nl < units;
    const T a = __builtin_nontemporal_load(&s[u]);
    T b{}, c{};
    if (o1) b = __builtin_nontemporal_load(&s[u + nl]);
    if (o2) c = __builtin_nontemporal_load(&s[u + 2 * nl]);
    __builtin_nontemporal_store(a, &d[u]);
    if (o1) __builtin_nontemporal_store(b, &d[u + nl]);
    if (o2) __builtin_nontemporal_store(c, &d[u + 2 * nl]);
  }
}

// Eviction's two row moves in one pass: the victim's row (at `row`) goes to
// `out` and the input row takes its place.  Both rows load before any store
// (`out`, `row` and `in` are distinct rows), four units per lane per round.
template <int U>
__device__ __forceinline__ void swap_units(gptr<uint8_t> out, gptr<uint8_t> row,
                                           gptr<const uint8_t> in, uint32_t bytes, uint32_t r,
                                           uint32_t nl) {
  using T = typename UnitT<U>::T;
  const uint32_t units = bytes / U;
  gptr<T> o = (gptr<T>)out;
  gptr<T> w = (gptr<T>)row;
  gptr<const T> s = (gptr<const T>)in;
  for (uint32_t u0 = r; u0 < units; u0 += 4 * nl) {
    T v[4], x[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t u = u0 + q * nl;
      if (u < units) {
        v[q] = __builtin_nontemporal_load(&w[u]);
        x[q] = __builtin_nontemporal_load(&s[u]);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t u = u0 + q * nl;
      if (u < units) {
        __builtin_nontemporal_store(v[q], &o[u]);
        __builtin_nontemporal_store(x[q], &w[u]);
      }
    }
  }
}

__device__ __forceinline__ void copy_row(gptr<uint8_t> dst, gptr<const uint8_t> src,
                                         uint32_t bytes, int unit, uint32_t r,
                                         uint32_t nl) {
  switch (unit) {
    case 16: copy_units<16>(dst, src, bytes, r, nl); break;
    case 8: copy_units<8>(dst, src, bytes, r, nl); break;
    case 4: copy_units<4>(dst, src, bytes, r, nl); break;
    case 2: copy_units<2>(dst, src, bytes, r, nl); break;
    default: copy_units<1>(dst, src, bytes, r, nl); break;
  }
}

}  // namespace hkv
