// hkv_kernels.hip -- gfx950 (wave64) kernels of the HierarchicalKV table.
//
// Read-only and idempotent operations (find, find missed, erase, export,
// size, clear) run one thread per key or per slot.  Every mutating batch
// operation (insert_or_assign, find_or_insert, insert_and_evict,
// accum_or_assign, assign_scores) is applied as if its keys ran one at a
// time in increasing batch index, each by the reference kernel's per-key
// algorithm (slot placement and eviction tie-breaks included):
//   1. partition: the batch is grouped by partition (256 consecutive
//      buckets) in batch-chunk order (k_pcount, k_pscan, k_pscatter);
//   2. apply: one workgroup owns each partition, so no atomic touches table
//      memory.  k_apply_fast applies a partition key-parallel where that
//      provably gives the sequential outcome and hands evictions to
//      k_apply_deferred (a 16-lane group per bucket); k_apply_part takes the
//      partitions it leaves: duplicate-heavy buckets folded per distinct key,
//      the rest by a lane-per-bucket walk in batch order.
// Tables of any size take this pipeline: one with more partitions than the
// counting kernels' LDS histogram holds is counted in several passes.
#include <hip/hip_runtime.h>

#include "hkv_kernels.h"

namespace hkv {

namespace {

constexpr int kBlock = 256;
constexpr uint32_t kNone = 0xFFFFFFFFu;

__host__ __device__ inline uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

/* ------------------------------------------------------------------------ */
/* init / clear                                                              */
/* ------------------------------------------------------------------------ */

// include/kernels/init_table_kernel/init_table_kernel.h:77-106 (digests =
// empty digest, keys = EMPTY, scores = 0) and bucket sizes = 0.
__global__ void k_init_slots(TableView t, uint64_t s0, uint64_t s1, uint64_t b0,
                             uint64_t b1, int reset_scores) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t s = s0 + blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; s < s1;
       s += stride) {
    G(t.digests)[s] = kEmptyDigest;
    if (reset_scores) slot_store(t, s, kEmptyKey, 0);
    else slot_key(t, s) = kEmptyKey;
  }
  for (uint64_t b = b0 + blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < b1;
       b += stride)
    G(t.bsize)[b] = 0;
}

/* ------------------------------------------------------------------------ */
/* find                                                                      */
/* ------------------------------------------------------------------------ */

// Key-first probing pays off while the table is at most 3/4 full.
__device__ __forceinline__ bool use_key_first(const TableView& t) {
  return *G(t.live) * 4 < t.capacity * 3;
}

// Wave-cooperative copy of up to 64 rows.  Row r belongs to lane
// lds_rows[r]: it is copied from that lane's `src` to
// dst_base + (lane_base + lane) * row_bytes.  The wave is split into groups of
// lpr lanes, one row per group; each pass moves four rows per group with all
// loads issued before the stores.  Rows past `rows` load row lds_rows[0]
// (valid) and store nothing.  Rows are streamed with non-temporal loads and
// stores, which keeps the probed metadata lines in the L2 cache.
template <int U>
__device__ __forceinline__ void wave_copy_rows(uint32_t rows, const uint32_t* lds_rows,
                                               gptr<const uint8_t> src, uint8_t* dst_base,
                                               uint64_t lane_base, uint32_t row_bytes) {
  using T = typename UnitT<U>::T;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t units = row_bytes / U;
  uint32_t lpr = 64;
  while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;  // lanes per row
  const uint32_t rpi = 64 / lpr;                    // rows per pass and quarter
  const uint32_t sub = lane % lpr;
  const uint64_t sp = (uint64_t)(uintptr_t)src;
  for (uint32_t r0 = 0; r0 < rows; r0 += 4 * rpi) {
    const uint32_t r = r0 + lane / lpr;
    const bool ok0 = r < rows, ok1 = r + rpi < rows, ok2 = r + 2 * rpi < rows,
               ok3 = r + 3 * rpi < rows;
    const uint32_t l0 = lds_rows[ok0 ? r : 0], l1 = lds_rows[ok1 ? r + rpi : 0],
                   l2 = lds_rows[ok2 ? r + 2 * rpi : 0], l3 = lds_rows[ok3 ? r + 3 * rpi : 0];
    gptr<const T> s0 = G<const T>((uintptr_t)shfl_u64(sp, (int)l0, 64));
    gptr<const T> s1 = G<const T>((uintptr_t)shfl_u64(sp, (int)l1, 64));
    gptr<const T> s2 = G<const T>((uintptr_t)shfl_u64(sp, (int)l2, 64));
    gptr<const T> s3 = G<const T>((uintptr_t)shfl_u64(sp, (int)l3, 64));
    gptr<T> d0 = G(reinterpret_cast<T*>(dst_base + (lane_base + l0) * row_bytes));
    gptr<T> d1 = G(reinterpret_cast<T*>(dst_base + (lane_base + l1) * row_bytes));
    gptr<T> d2 = G(reinterpret_cast<T*>(dst_base + (lane_base + l2) * row_bytes));
    gptr<T> d3 = G(reinterpret_cast<T*>(dst_base + (lane_base + l3) * row_bytes));
    for (uint32_t u = sub; u < units; u += lpr) {
      const T v0 = __builtin_nontemporal_load(&s0[u]), v1 = __builtin_nontemporal_load(&s1[u]),
              v2 = __builtin_nontemporal_load(&s2[u]), v3 = __builtin_nontemporal_load(&s3[u]);
      if (ok0) __builtin_nontemporal_store(v0, &d0[u]);
      if (ok1) __builtin_nontemporal_store(v1, &d1[u]);
      if (ok2) __builtin_nontemporal_store(v2, &d2[u]);
      if (ok3) __builtin_nontemporal_store(v3, &d3[u]);
    }
  }
}

struct KeyPos {
  uint64_t b;
  uint32_t start, d;
};

__device__ __forceinline__ KeyPos key_pos(const TableView& t, uint64_t k) {
  const uint64_t h = murmur3(k);
  const uint64_t gi = global_idx(t, h);
  return KeyPos{gi >> t.bshift, (uint32_t)(gi & (t.B - 1)), key_digest(h)};
}

constexpr uint64_t kLocMask = (1ull << 56) - 1;

// Per-wave LDS of wave_probe.
struct ProbeLds {
  uint64_t key[64];
  uint64_t loc[64];    // digest << 56 | (b * B + start) of the lane's key; ~0 when none
  uint32_t dm[64][8];  // per listed key and 16-slot chunk: match bits | EMPTY bits << 16
  uint32_t list[64];   // lanes whose keys the digest pass probes
};

// 128-bit mask (lo, hi) rotated right by r < 128: bit i becomes bit i - r.
__device__ __forceinline__ void rot128(uint64_t& lo, uint64_t& hi, uint32_t r) {
  if (r & 64) {
    const uint64_t x = lo;
    lo = hi;
    hi = x;
  }
  r &= 63;
  if (r) {
    const uint64_t l = (lo >> r) | (hi << (64 - r));
    const uint64_t h = (hi >> r) | (lo << (64 - r));
    lo = l;
    hi = h;
  }
}

// Wave-cooperative lookup of one key per lane (find_without_lock,
// include/find_utils.h:31-86); returns the slot of the lane's key (bucket in
// *bk) or -1.  Buckets hold 128 slots.
//  1. Key-first (kf, the table at most 3/4 full): in each of four loads,
//     lanes 4q..4q+3 read the keys of the first probe group of key q (one
//     64-byte request per key); two ballots give every key the group's hit
//     and EMPTY slots.  The group decides when it holds the key or an EMPTY
//     slot at or after start.
//  2. The other keys: lanes 8q..8q+7 read the eight 16-byte chunks of key
//     q's digest line (one 128-byte request per key) and leave match and
//     EMPTY masks in LDS.  The owner lane rotates them into probe order from
//     align4(start), cuts them after the group of the first EMPTY slot (in
//     the first group only at or after start), and confirms the digest
//     matches in that order with key loads.  This visits slots in the order
//     of the reference's group loop and stops where it stops.
// A slot's digest is the empty digest exactly when its key is EMPTY.
__device__ __forceinline__ int wave_probe(const TableView& t, uint64_t k, bool valid, bool kf,
                                          ProbeLds& L, uint64_t* bk) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t B = t.B;
  uint64_t b = 0;
  uint32_t start = 0, d = 0;
  if (valid) {
    const KeyPos q = key_pos(t, k);
    b = q.b;
    start = q.start;
    d = q.d;
  }
  *bk = b;
  L.key[lane] = k;
  L.loc[lane] = valid ? ((uint64_t)d << 56) | (b * B + start) : ~0ull;
  __builtin_amdgcn_wave_barrier();
  int slot = -1;
  bool done = !valid;
  if (kf) {
    uint64_t hit[4], emp[4];
#pragma unroll
    for (uint32_t j = 0; j < 4; j++) {
      const uint32_t o = j * 16 + (lane >> 2);
      const uint64_t raw = L.loc[o];
      const uint64_t ok = L.key[o];
      const bool live = raw != ~0ull;
      const uint64_t loc = raw & kLocMask;
      const uint32_t pos = lane & 3;
      uint64_t kk = 0;
      if (live) kk = slot_key(t, (loc & ~3ull) + pos);
      hit[j] = __ballot(live && kk == ok);
      emp[j] = __ballot(live && kk == kEmptyKey && pos >= (uint32_t)(loc & 3));
    }
    const uint32_t j = lane >> 4, sh = 4 * (lane & 15);
    const uint64_t H = j == 0 ? hit[0] : j == 1 ? hit[1] : j == 2 ? hit[2] : hit[3];
    const uint64_t E = j == 0 ? emp[0] : j == 1 ? emp[1] : j == 2 ? emp[2] : emp[3];
    const uint32_t h4 = (uint32_t)(H >> sh) & 15u, e4 = (uint32_t)(E >> sh) & 15u;
    if (!done && h4) {
      slot = (int)((start & ~3u) + __builtin_ctz(h4));
      done = true;
    } else if (!done && e4) {
      done = true;
    }
  }
  const uint64_t pend = __ballot(!done);
  const uint32_t cnt = __popcll(pend);
  if (cnt == 0) return slot;
  const uint32_t my = __popcll(pend & ((1ull << lane) - 1));
  if (!done) L.list[my] = lane;
  __builtin_amdgcn_wave_barrier();
  {
    const uint32_t c = lane & 7;
    u32x4 w[8];
#pragma unroll
    for (uint32_t r = 0; r < 8; r++) {
      const uint32_t idx = r * 8 + (lane >> 3);
      w[r] = u32x4{0, 0, 0, 0};
      if (idx < cnt) {
        const uint64_t loc = L.loc[L.list[idx]] & kLocMask;
        w[r] = *(gptr<const u32x4>)(G(t.digests) + (loc & ~(uint64_t)(B - 1)) + c * 16);
      }
    }
    const uint32_t erep = (uint32_t)kEmptyDigest * 0x01010101u;
#pragma unroll
    for (uint32_t r = 0; r < 8; r++) {
      const uint32_t idx = r * 8 + (lane >> 3);
      if (idx < cnt) {
        const uint32_t rep = (uint32_t)(L.loc[L.list[idx]] >> 56) * 0x01010101u;
        const uint32_t m = eq_bytes4(w[r].x, rep) | (eq_bytes4(w[r].y, rep) << 4) |
                           (eq_bytes4(w[r].z, rep) << 8) | (eq_bytes4(w[r].w, rep) << 12);
        const uint32_t e = eq_bytes4(w[r].x, erep) | (eq_bytes4(w[r].y, erep) << 4) |
                           (eq_bytes4(w[r].z, erep) << 8) | (eq_bytes4(w[r].w, erep) << 12);
        L.dm[idx][c] = m | (e << 16);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (done) return slot;
  uint64_t mlo = 0, mhi = 0, elo = 0, ehi = 0;
#pragma unroll
  for (uint32_t c = 0; c < 8; c++) {
    const uint32_t v = L.dm[my][c];
    const uint64_t m = v & 0xFFFFu, e = v >> 16;
    if (c < 4) {
      mlo |= m << (16 * c);
      elo |= e << (16 * c);
    } else {
      mhi |= m << (16 * (c - 4));
      ehi |= e << (16 * (c - 4));
    }
  }
  const uint32_t a = start & ~3u;
  rot128(mlo, mhi, a);
  rot128(elo, ehi, a);
  elo &= ~((1ull << (start - a)) - 1);  // first group: EMPTY only at or after start
  if (kf) mlo &= ~0xFull;               // the first group was read by key
  // Keep the matches up to the end of the first EMPTY slot's group.
  if (elo) {
    const uint32_t lim = ((__builtin_ctzll(elo) >> 2) + 1) * 4;
    mlo &= lim >= 64 ? ~0ull : ((1ull << lim) - 1);
    mhi = 0;
  } else if (ehi) {
    const uint32_t lim = ((__builtin_ctzll(ehi) >> 2) + 1) * 4;
    mhi &= lim >= 64 ? ~0ull : ((1ull << lim) - 1);
  }
  const uint64_t base = b * B;
  while (mlo | mhi) {
    uint32_t i;
    if (mlo) {
      i = __builtin_ctzll(mlo);
      mlo &= mlo - 1;
    } else {
      i = 64 + __builtin_ctzll(mhi);
      mhi &= mhi - 1;
    }
    const uint32_t p = (a + i) & (B - 1);
    if (slot_key(t, base + p) == k) return (int)p;
  }
  return -1;
}

// One key per lane, probed by the wave together (wave_probe); the wave then
// copies its hit rows.  Find is bound by HBM traffic (a metadata line plus
// the row in and out per hit).  The missed-keys variant runs 1024-thread
// blocks and appends a block's missed keys, collected in LDS, with one
// atomic.
template <int U, bool MISSED, int BLK>
__global__ __launch_bounds__(BLK) void k_find(TableView t, const uint64_t* __restrict__ keys,
                                              uint64_t n, uint8_t* __restrict__ values,
                                              uint8_t* __restrict__ founds,
                                              uint64_t* __restrict__ scores,
                                              uint64_t* __restrict__ missed_keys,
                                              int32_t* __restrict__ missed_idx,
                                              int32_t* __restrict__ missed_size) {
  constexpr uint32_t kMissCap = MISSED ? BLK : 1;
  __shared__ uint32_t s_rows[BLK / 64][64];
  __shared__ ProbeLds s_probe[BLK / 64];
  __shared__ uint64_t s_mkey[kMissCap];
  __shared__ uint32_t s_midx[kMissCap];
  __shared__ uint32_t s_mcnt, s_mbase;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wv = threadIdx.x >> 6;
  const bool kf = use_key_first(t);
  if (MISSED && threadIdx.x == 0) s_mcnt = 0;
  if (MISSED) __syncthreads();
  const uint64_t wave_base = ((uint64_t)blockIdx.x * (BLK / 64) + wv) * 64;
  const uint64_t i = wave_base + lane;
  const uint64_t k = i < n ? keys[i] : 0;
  const bool valid = i < n && !is_reserved(k);
  uint64_t b = 0;
  const int p = wave_probe(t, k, valid, kf, s_probe[wv], &b);
  const bool found = p >= 0;
  gptr<const uint8_t> src = nullptr;
  if (found) {
    src = row_ptr(t, b, (uint32_t)p);
    if (scores) scores[i] = slot_score(t, b * t.B + p);
  }
  if (!MISSED && founds && i < n) founds[i] = found ? 1 : 0;
  if (MISSED && i < n && !found) {
    const uint32_t r = atomicAdd(&s_mcnt, 1u);
    s_mkey[r] = k;
    s_midx[r] = (uint32_t)i;
  }
  const uint64_t hm = __ballot(found);
  if (found) s_rows[wv][__popcll(hm & ((1ull << lane) - 1))] = lane;
  __builtin_amdgcn_wave_barrier();
  const uint32_t rows = __popcll(hm);
  if (rows) wave_copy_rows<U>(rows, s_rows[wv], src, values, wave_base, t.row_bytes);
  if (MISSED) {
    __syncthreads();
    const uint32_t cnt = s_mcnt;
    if (threadIdx.x == 0 && cnt)
      s_mbase = atomicAdd(reinterpret_cast<uint32_t*>(missed_size), cnt);
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < cnt; r += BLK) {
      missed_keys[s_mbase + r] = s_mkey[r];
      missed_idx[s_mbase + r] = (int32_t)s_midx[r];
    }
  }
}

/* ------------------------------------------------------------------------ */
/* erase                                                                     */
/* ------------------------------------------------------------------------ */

// include/kernels/remove_kernel/remove_kernel.h:31-113: every digest group
// is scanned (no early stop); a matching key becomes RECLAIM with score 0
// and the reclaim digest.  The slot is claimed with a CAS so that a key
// repeated in one batch is erased once, as if applied in batch order.
__device__ __forceinline__ bool erase_key(const TableView& t, uint64_t k) {
  if (is_reserved(k)) return false;
  const uint32_t B = t.B;
  const uint64_t h = murmur3(k);
  const uint64_t gi = global_idx(t, h);
  const uint64_t b = gi >> t.bshift;
  const uint32_t start = (uint32_t)(gi & (B - 1));
  const uint32_t rep = key_digest(h) * 0x01010101u;
  gptr<uint8_t> dg = digest_row(t, b);
  const uint32_t a = start & ~3u;
  bool erased = false;
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t w = *(gptr<const uint32_t>)(dg + g);
    uint32_t m = eq_bytes4(w, rep);
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      g64& key = slot_key(t, b * B + g + j);
      if (key == k) {
        if (atomicCAS((unsigned long long*)&key, (unsigned long long)k,
                      (unsigned long long)kReclaimKey) == (unsigned long long)k) {
          slot_score(t, b * B + g + j) = 0;
          dg[g + j] = kReclaimDigest;
          atomicSub(t.bsize + b, 1);
          erased = true;
        }
        break;
      }
    }
  }
  return erased;
}

__global__ __launch_bounds__(kBlock) void k_erase(TableView t, const uint64_t* __restrict__ keys,
                                                  uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const bool erased = i < n && erase_key(t, keys[i]);
  const uint64_t m = __ballot(erased);
  if ((threadIdx.x & 63) == 0 && m) atomicAdd(t.live, 0ull - (unsigned long long)__popcll(m));
}

/* ------------------------------------------------------------------------ */
/* bucket owner state and per-key apply (all mutating batch operations)    */
/* ------------------------------------------------------------------------ */

enum Outcome : uint32_t { R_DUP = 1, R_EMPTY = 2, R_RECLAIMED = 3, R_EVICT = 4, R_REFUSED = 5 };

// State of one bucket held by a 16-lane group: lane l owns slots l + 16*j
// (j = 0..7) and keeps their digests (packed in two words), keys and scores
// in registers for as long as the group applies keys to the bucket, so an
// evicting key scans no memory.  Only the owner lane reads or writes a slot,
// which keeps the registers current; writes go through to the table.
struct Bucket16 {
  uint32_t b;  // bucket (bucket counts stay below 2^32)
  uint32_t l;
  uint32_t dg0, dg1;  // digest of slot l+16j in byte j (dg0: j<4, dg1: j>=4)
  int32_t bsz, bsz0;
  uint64_t key[8], score[8];  // record of slot l+16j
};

// Element j of a lane's eight records (j is not a compile-time constant).
// Written as mask arithmetic: a chain of selects would be turned into an
// indexed stack array.
__device__ __forceinline__ uint64_t rec_get(const uint64_t (&v)[8], uint32_t j) {
  uint64_t r = 0;
#pragma unroll
  for (uint32_t q = 0; q < 8; q++) r |= v[q] & (0ull - (uint64_t)(j == q));
  return r;
}

__device__ __forceinline__ void rec_set(uint64_t (&v)[8], uint32_t j, uint64_t x) {
#pragma unroll
  for (uint32_t q = 0; q < 8; q++) {
    const uint64_t m = 0ull - (uint64_t)(j == q);
    v[q] = (v[q] & ~m) | (x & m);
  }
}

__device__ __forceinline__ uint32_t dg_of(const Bucket16& S, uint32_t j) {
  return ((j < 4 ? S.dg0 : S.dg1) >> (8 * (j & 3))) & 0xFFu;
}

__device__ __forceinline__ void dg_set(Bucket16& S, uint32_t j, uint32_t d) {
  const uint32_t sh = 8 * (j & 3);
  const uint32_t m = ~(0xFFu << sh);
  if (j < 4) S.dg0 = (S.dg0 & m) | (d << sh);
  else S.dg1 = (S.dg1 & m) | (d << sh);
}

__device__ __forceinline__ void bucket_load(const TableView& t, Bucket16& S, uint64_t b,
                                            uint32_t l) {
  S.b = (uint32_t)b;
  S.l = l;
  const uint64_t base = b * (uint64_t)t.B;
  gptr<const uint8_t> dg = G(t.digests) + base + l;
  S.dg0 = (uint32_t)dg[0] | ((uint32_t)dg[16] << 8) | ((uint32_t)dg[32] << 16) |
          ((uint32_t)dg[48] << 24);
  S.dg1 = (uint32_t)dg[64] | ((uint32_t)dg[80] << 8) | ((uint32_t)dg[96] << 16) |
          ((uint32_t)dg[112] << 24);
#pragma unroll
  for (uint32_t j = 0; j < 8; j++) {
    const u64x2 r = slot_load(t, base + l + 16 * j);
    S.key[j] = r.x;
    S.score[j] = r.y;
  }
  S.bsz = S.bsz0 = G(t.bsize)[b];
}

// First slot of the bucket a group holds.
__device__ __forceinline__ uint64_t sbase(const TableView& t, const Bucket16& S) {
  return (uint64_t)S.b * t.B;
}

// Group-wide minimum of (score, rank) carrying the slot and its key.
__device__ __forceinline__ void group_min_victim(uint64_t& s, uint32_t& rank, uint32_t& pos,
                                                 uint64_t& key) {
#pragma unroll
  for (int m = 8; m > 0; m >>= 1) {
    const uint64_t os = shfl_xor_u64(s, m, 16);
    const uint32_t orank = __shfl_xor(rank, m, 16);
    const uint32_t opos = __shfl_xor(pos, m, 16);
    const uint64_t okey = shfl_xor_u64(key, m, 16);
    if (os < s || (os == s && orank < rank)) {
      s = os;
      rank = orank;
      pos = opos;
      key = okey;
    }
  }
}

template <typename V>
__device__ __forceinline__ void accum_units(gptr<uint8_t> dst, gptr<const uint8_t> delta,
                                            uint32_t bytes, uint32_t r, uint32_t nl) {
  gptr<V> d = (gptr<V>)dst;
  gptr<const V> s = (gptr<const V>)delta;
  const uint32_t cntv = bytes / sizeof(V);
  // Four elements per lane per round, every load before the first store
  // (delta and dst are different rows).
  for (uint32_t u0 = r; u0 < cntv; u0 += 4 * nl) {
    V v[4], o[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t u = u0 + q * nl;
      if (u < cntv) {
        v[q] = s[u];
        o[q] = d[u];
      }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t u = u0 + q * nl;
      if (u < cntv) {
        v[q] += o[q];  // `val = delta; val += dst` (accum_or_assign_kernel.h:41-49)
        d[u] = v[q];
      }
    }
  }
}

__device__ __forceinline__ void accum_row(gptr<uint8_t> dst, gptr<const uint8_t> delta,
                                          uint32_t bytes, int vt, uint32_t r, uint32_t nl) {
  switch (vt) {
    case 0: accum_units<float>(dst, delta, bytes, r, nl); break;           // f32
    case 8: accum_units<int32_t>(dst, delta, bytes, r, nl); break;         // i32
    case 10: case 11: accum_units<uint64_t>(dst, delta, bytes, r, nl); break;  // i64/u64
    default: break;
  }
}

// Output position of the eviction record of batch key `i` (all 16 lanes of
// the group call this): the key's own batch index, flagged for the
// compaction kernels, or (without a flag bitmap) the next value of the
// record counter.
__device__ __forceinline__ uint64_t ev_slot(const ApplyArgs& a, uint64_t i, uint32_t l) {
  if (a.ev_bits) {
    if (l == 0) atomicOr(&a.ev_bits[i >> 5], 1u << (i & 31));
    return i;
  }
  uint64_t j = 0;
  if (l == 0) j = atomicAdd(reinterpret_cast<unsigned long long*>(a.ev_counter), 1ull);
  return shfl_u64(j, 0, 16);
}

// Applies batch key `i` to the bucket held by the group (all 16 lanes call
// this with the same i).  Restates, for one key, the reference kernels
// insert_or_assign_kernel.h:76-303 (unique keys) and find_and_lock
// (find_utils.h:94-227) with its callers (non-unique keys and accum).
// Row moves of one applied key, for callers that queue them instead of
// running them in place (kRows = false): a read into the key's output row
// (the slot's row, or the key's own input row) and a write of the slot (the
// key's input row copied in, or its delta added).
constexpr uint32_t kRdNone = 0, kRdSlot = 1, kRdSelf = 2, kRdFwd = 3;
constexpr uint32_t kWrNone = 0, kWrCopy = 1, kWrAcc = 2;
struct RowAct {
  uint32_t rd, wr, pos;
};

template <int OP, int U, bool kRows = true>
__device__ __forceinline__ RowAct apply_key_in(const TableView& t, Bucket16& S,
                                               const ApplyArgs& a, uint64_t i, uint64_t k,
                                               uint64_t in) {
  RowAct act{kRdNone, kWrNone, 0};
  constexpr int SPL = 8;
  const uint32_t B = t.B;
  const uint32_t l = S.l;
  const bool has_in = a.in_scores != nullptr;
  const uint64_t h = murmur3(k);
  const uint64_t gi = global_idx(t, h);
  const uint32_t start = (uint32_t)(gi & (B - 1));
  const uint32_t d = key_digest(h);
  const uint64_t des = score_desired(a.sc, has_in, in);

  // 1. Is the key present?  Candidates are digest matches.
  const uint32_t a4 = start & ~3u;
  uint32_t best = kNone;
#pragma unroll
  for (int j = 0; j < SPL; j++) {
    if (dg_of(S, j) == d && S.key[j] == k) {
      const uint32_t p = l + 16 * j;
      const uint32_t rk = (((p - a4) & (B - 1)) << 8) | p;
      best = rk < best ? rk : best;
    }
  }
  best = group_min_u32(best);

  uint32_t res = 0;
  uint32_t pos = 0;
  uint64_t victim_key = 0, victim_score = 0;
  if (best != kNone) {
    res = R_DUP;
    pos = best & 0xFFu;
  } else if (OP == OP_ASSIGN_SCORES) {
    return act;  // absent keys are a no-op
  } else {
    // 2. First EMPTY slot (empty digest) in circular order from `start`.
    if (S.bsz < (int32_t)B) {
      uint32_t rl = kNone;
#pragma unroll
      for (int j = 0; j < SPL; j++) {
        if (dg_of(S, j) == kEmptyDigest) {
          const uint32_t r = (l + 16 * j - start) & (B - 1);
          rl = r < rl ? r : rl;
        }
      }
      const uint32_t r = group_min_u32(rl);
      if (r != kNone) {
        res = R_EMPTY;
        pos = (start + r) & (B - 1);
      }
    }
    if (res == 0) {
      // 3. Eviction over every slot of the bucket.
      uint64_t ms = kMaxScore, mk = 0;
      uint32_t mr = kNone, mp = start;
#pragma unroll
      for (int j = 0; j < SPL; j++) {
        const uint32_t p = l + 16 * j;
        const uint64_t kj = S.key[j];
        const uint64_t sj = S.score[j];
        uint32_t rank;
        bool elig;
        if (a.rule == RULE_DIGEST16) {
          // Lane (p & 15) of the reference's 16-lane group scans p, p+16, ...;
          // the xor-butterfly prefers, on ties, lanes whose xor with the
          // deciding lane (batch index mod 16) is smallest bit-reversed.
          elig = kj != kEmptyKey && kj != kLockedKey;
          rank = bitrev4(l ^ (uint32_t)(i & 15)) * SPL + j;
        } else {
          // find_and_lock: lane r%32 scans r, r+32, ...; lowest lane wins.
          elig = kj != kEmptyKey;
          const uint32_t r = (p - start) & (B - 1);
          rank = (r & 31) * (B / 32) + (r >> 5);
        }
        if (elig && sj < kMaxScore && (sj < ms || (sj == ms && rank < mr))) {
          ms = sj;
          mr = rank;
          mp = p;
          mk = kj;
        }
      }
      group_min_victim(ms, mr, mp, mk);
      if (mr == kNone) {
        // Every eligible score is MAX_SCORE: the start slot is taken.
        mp = start;
        uint64_t kk = 0;
        if (l == (start & 15u)) kk = rec_get(S.key, start >> 4);
        mk = shfl_u64(kk, (int)(start & 15u), 16);
      }
      if (des < ms || mk == kLockedKey) {
        // A LOCKED victim is never taken: the reference kernels wait for it
        // to be unlocked.
        res = R_REFUSED;
      } else {
        pos = mp;
        victim_key = mk;
        victim_score = ms;
        res = victim_key == kReclaimKey ? R_RECLAIMED : R_EVICT;
      }
    }
  }

  // 4. Effects.
  const uint32_t R = t.row_bytes;
  gptr<const uint8_t> in_row = a.in_values ? G(a.in_values) + i * (uint64_t)R : nullptr;
  if (OP == OP_ACCUM_OR_ASSIGN) {
    if (res == R_REFUSED) return act;
    const bool is_accum = G(a.accum_flags)[i] != 0;
    if ((is_accum && res != R_DUP) || (!is_accum && res == R_DUP)) return act;
  }
  if (res == R_REFUSED) {
    if (OP == OP_INSERT_AND_EVICT) {
      const uint64_t j = ev_slot(a, i, l);
      if (l == 0) {
        G(a.ev_keys)[j] = k;
        if (a.ev_scores) G(a.ev_scores)[j] = des;
      }
      if (kRows) copy_units<U>(G(a.ev_values) + j * R, in_row, R, l, 16);
      act.rd = kRdSelf;
    }
    return act;
  }
  gptr<uint8_t> trow = row_ptr(t, S.b, pos);
  const bool swapped = OP == OP_INSERT_AND_EVICT && res == R_EVICT;
  if (swapped) {
    const uint64_t j = ev_slot(a, i, l);
    if (l == 0) {
      G(a.ev_keys)[j] = victim_key;
      if (a.ev_scores) G(a.ev_scores)[j] = victim_score;
    }
    // victim row out and input row in, one pass
    if (kRows) swap_units<U>(G(a.ev_values) + j * R, trow, in_row, R, l, 16);
    act.rd = kRdSlot;
    act.wr = kWrCopy;
  }
  if (res == R_EMPTY || res == R_RECLAIMED) S.bsz++;

  if (OP == OP_FIND_OR_INSERT_PTR || swapped) {
    // No row moves (the caller goes through the returned address), or both
    // moves done above.
  } else if (res == R_DUP) {
    if (OP == OP_FIND_OR_INSERT) {
      if (kRows) copy_units<U>(G(a.io_values) + i * (uint64_t)R, trow, R, l, 16);
      act.rd = kRdSlot;
    } else if (OP == OP_ACCUM_OR_ASSIGN) {
      if (kRows) accum_row(trow, in_row, R, a.value_type, l, 16);
      act.wr = kWrAcc;
    } else if (OP != OP_ASSIGN_SCORES) {
      if (kRows) copy_units<U>(trow, in_row, R, l, 16);
      act.wr = kWrCopy;
    }
  } else {
    if (kRows) copy_units<U>(trow, in_row, R, l, 16);
    act.wr = kWrCopy;
  }
  act.pos = pos;

  const uint32_t owner = pos & 15u, jj = pos >> 4;
  if (l == owner) {
    uint64_t old = 0;
    if (res == R_DUP && (a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu))
      old = rec_get(S.score, jj);
    else if (res != R_DUP && a.sc.strategy == kLfu && !has_in)
      old = rec_get(S.score, jj);
    bool w;
    uint64_t ns;
    if (OP == OP_ASSIGN_SCORES) {
      ns = score_wo_missed(a.sc, has_in, in, old, &w);
    } else if (res == R_DUP) {
      ns = score_hit(a.sc, has_in, in, des, old, &w);
    } else {
      ns = score_new(a.sc, has_in, in, des, old, &w);
    }
    // The pointer find_or_insert with unique keys holds every slot it claims
    // or finds LOCKED for the rest of the batch (find_or_insert_ptr_kernel_v2.h:38-285):
    // later keys neither match nor evict it.
    const bool lk = OP == OP_FIND_OR_INSERT_PTR && a.lock;
    const uint64_t wk = lk ? kLockedKey : k;
    if (res == R_DUP) {
      if (w) {
        slot_score(t, sbase(t, S) + pos) = ns;
        rec_set(S.score, jj, ns);
      }
      if (lk) {
        slot_key(t, sbase(t, S) + pos) = kLockedKey;
        rec_set(S.key, jj, kLockedKey);
      }
    } else if (w) {
      slot_store(t, sbase(t, S) + pos, wk, ns);
      G(t.digests)[sbase(t, S) + pos] = (uint8_t)d;
      dg_set(S, jj, d);
      rec_set(S.key, jj, wk);
      rec_set(S.score, jj, ns);
    } else {
      slot_key(t, sbase(t, S) + pos) = wk;
      rec_set(S.key, jj, wk);
    }
    if (OP == OP_FIND_OR_INSERT_PTR)
      G(a.slot_out)[i] = (sbase(t, S) + pos + 1) | (res == R_DUP ? kSlotFound : 0ull);
  }
  return act;
}

// apply_key_in with the key's input score loaded here.
template <int OP, int U>
__device__ __forceinline__ void apply_key(const TableView& t, Bucket16& S, const ApplyArgs& a,
                                          uint64_t i, uint64_t k) {
  const uint64_t in = a.in_scores ? G(a.in_scores)[i] : 0;
  apply_key_in<OP, U>(t, S, a, i, k, in);
}

__device__ __forceinline__ void bucket_finish(const TableView& t, Bucket16& S) {
  if (S.l == 0 && S.bsz != S.bsz0) {
    G(t.bsize)[S.b] = S.bsz;
    atomicAdd(t.live, (unsigned long long)(int64_t)(S.bsz - S.bsz0));
  }
}

// Row tasks queued by a wave of the lane pass, executed cooperatively.  The
// destination pointer's top bit marks an accumulate task.
constexpr uint64_t kAccumBit = 1ull << 63;

template <int U, int Q>
__device__ __forceinline__ void flush_tasks(uint32_t ntask, const uint64_t* s_src,
                                            const uint64_t* s_dst, uint32_t row_bytes,
                                            int vt) {
  using T = typename UnitT<U>::T;  // Q rows in flight per lane group: 2, 4 or 8
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t units = row_bytes / U;
  uint32_t lpr = 64;
  while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;
  const uint32_t rpi = 64 / lpr;
  const uint32_t sub = lane % lpr;
  // Rows beyond ntask read task 0's source (valid) and store nothing.
  const uint64_t any_src = s_src[0] & ~kAccumBit;
  for (uint32_t r0 = 0; r0 < ntask; r0 += Q * rpi) {
    gptr<const T> s[Q];
    gptr<T> d[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
      const uint32_t r = r0 + q * rpi + lane / lpr;
      const bool ok = r < ntask;
      uint64_t dp = ok ? s_dst[r] : 0;
      const uint64_t sp = ok ? s_src[r] : any_src;
      if (dp & kAccumBit) {
        accum_row(G<uint8_t>((uintptr_t)(dp & ~kAccumBit)), G<const uint8_t>((uintptr_t)sp),
                  row_bytes, vt, sub, lpr);
        dp = 0;
      }
      s[q] = G<const T>((uintptr_t)(dp ? sp : any_src));
      d[q] = G<T>((uintptr_t)dp);
    }
    for (uint32_t u = sub; u < units; u += lpr) {
      if constexpr (Q == 2) {
        const T v0 = s[0][u], v1 = s[1][u];
        if (d[0]) d[0][u] = v0;
        if (d[1]) d[1][u] = v1;
      } else if constexpr (Q == 4) {
        const T v0 = s[0][u], v1 = s[1][u], v2 = s[2][u], v3 = s[3][u];
        if (d[0]) d[0][u] = v0;
        if (d[1]) d[1][u] = v1;
        if (d[2]) d[2][u] = v2;
        if (d[3]) d[3][u] = v3;
      } else {
        const T v0 = s[0][u], v1 = s[1][u], v2 = s[2][u], v3 = s[3][u];
        const T v4 = s[4][u], v5 = s[5][u], v6 = s[6][u], v7 = s[7][u];
        if (d[0]) d[0][u] = v0;
        if (d[1]) d[1][u] = v1;
        if (d[2]) d[2][u] = v2;
        if (d[3]) d[3][u] = v3;
        if (d[4]) d[4][u] = v4;
        if (d[5]) d[5][u] = v5;
        if (d[6]) d[6][u] = v6;
        if (d[7]) d[7][u] = v7;
      }
    }
  }
}

// Digest probe of one key by one lane (insert_or_assign_kernel.h:105-183):
// returns the slot holding `k` (dup=1), else the first EMPTY slot in circular
// order from `start` when the bucket is not full (dup=0), else -1.
__device__ __forceinline__ int probe_upsert(const TableView& t, uint64_t base, uint32_t start,
                                            uint32_t d, uint64_t k, bool not_full, int* dup) {
  const uint32_t B = t.B;
  gptr<const uint8_t> dg = G(t.digests) + base;
  const uint32_t a = start & ~3u;
  const uint32_t rep = d * 0x01010101u;
  const uint32_t erep = (uint32_t)kEmptyDigest * 0x01010101u;
  uint32_t cur = kNone;
  u32x4 chunk = {0, 0, 0, 0};
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t c = g >> 4;
    if (c != cur) {
      chunk = *(gptr<const u32x4>)(dg + (c << 4));
      cur = c;
    }
    const uint32_t wi = (g >> 2) & 3;
    const uint32_t w = wi == 0 ? chunk.x : wi == 1 ? chunk.y : wi == 2 ? chunk.z : chunk.w;
    uint32_t m = eq_bytes4(w, rep);
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      if (slot_key(t, base + g + j) == k) {
        *dup = 1;
        return (int)(g + j);
      }
    }
    if (!not_full) continue;
    uint32_t e = eq_bytes4(w, erep);
    while (e) {
      const uint32_t j = __builtin_ctz(e);
      e &= e - 1;
      const uint32_t p = g + j;
      if (off == 0 && p < start) continue;
      *dup = 0;  // the empty digest marks an EMPTY slot
      return (int)p;
    }
  }
  return -1;
}

// Workgroup barrier that orders LDS only (global stores stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// probe_upsert on a copy of the bucket's digests in LDS (`dg` = 32 words, the
// digests of slots 4w..4w+3 in word w), kept current by the bucket's owner.
__device__ __forceinline__ int probe_upsert_lds(const TableView& t, const uint32_t* dg,
                                                uint64_t base, uint32_t start, uint32_t d,
                                                uint64_t k, bool not_full, int* dup) {
  const uint32_t B = t.B;
  const uint32_t a = start & ~3u;
  const uint32_t rep = d * 0x01010101u;
  const uint32_t erep = (uint32_t)kEmptyDigest * 0x01010101u;
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t w = dg[g >> 2];
    uint32_t m = eq_bytes4(w, rep);
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      if (slot_key(t, base + g + j) == k) {
        *dup = 1;
        return (int)(g + j);
      }
    }
    if (!not_full) continue;
    uint32_t e = eq_bytes4(w, erep);
    while (e) {
      const uint32_t j = __builtin_ctz(e);
      e &= e - 1;
      const uint32_t p = g + j;
      if (off == 0 && p < start) continue;
      *dup = 0;
      return (int)p;
    }
  }
  return -1;
}

// Result bits of lane_apply.
constexpr uint32_t kLaneDigest = 1;  // a new key's digest was written at the slot
constexpr uint32_t kLaneRead = 2;    // the task reads the table row (a find_or_insert hit)

// Effects of one key whose probe returned slot p (dup: the key is present),
// for the lane that owns the bucket (`base` = its first slot, `rows0` = the
// row of its slot 0).  Metadata is updated in place; the row movement is
// returned as a task (*src -> *dst, dst = 0 for none; an accumulate task has
// kAccumBit set in dst).
template <int OP>
__device__ __forceinline__ uint32_t lane_apply(const TableView& t, const ApplyArgs& a,
                                               uint64_t base, gptr<uint8_t> rows0, int p,
                                               int dup, uint64_t i, uint64_t k, uint64_t in,
                                               bool has_in, uint32_t d, int32_t& bsz,
                                               uint64_t& src, uint64_t& dst) {
  const uint32_t R = t.row_bytes;
  src = dst = 0;
  const uint64_t des = score_desired(a.sc, has_in, in);
  if (OP == OP_ACCUM_OR_ASSIGN) {
    const bool is_accum = G(a.accum_flags)[i] != 0;
    if (is_accum != (dup != 0)) return 0;
  }
  gptr<uint8_t> trow = rows0 + (uint64_t)p * R;
  gptr<const uint8_t> in_row = a.in_values ? G(a.in_values) + i * (uint64_t)R : nullptr;
  bool w;
  uint32_t res = 0;
  if (dup) {
    uint64_t old = 0;
    if (a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu) old = slot_score(t, base + p);
    const uint64_t ns = OP == OP_ASSIGN_SCORES ? score_wo_missed(a.sc, has_in, in, old, &w)
                                               : score_hit(a.sc, has_in, in, des, old, &w);
    if (w) slot_score(t, base + p) = ns;
    if (OP == OP_FIND_OR_INSERT) {
      src = (uint64_t)(uintptr_t)trow;
      dst = (uint64_t)(uintptr_t)(G(a.io_values) + i * (uint64_t)R);
      res |= kLaneRead;
    } else if (OP == OP_ACCUM_OR_ASSIGN) {
      src = (uint64_t)(uintptr_t)in_row;
      dst = (uint64_t)(uintptr_t)trow | kAccumBit;
    } else if (OP != OP_ASSIGN_SCORES) {
      src = (uint64_t)(uintptr_t)in_row;
      dst = (uint64_t)(uintptr_t)trow;
    }
  } else {
    // The old score matters only to Lfu without input scores.
    const uint64_t old = (a.sc.strategy == kLfu && !has_in) ? slot_score(t, base + p) : 0;
    const uint64_t ns = score_new(a.sc, has_in, in, des, old, &w);
    if (w) {
      slot_store(t, base + p, k, ns);
      G(t.digests)[base + p] = (uint8_t)d;
      res |= kLaneDigest;
    } else {
      slot_key(t, base + p) = k;
    }
    bsz++;
    src = (uint64_t)(uintptr_t)in_row;
    dst = (uint64_t)(uintptr_t)trow;
  }
  return res;
}

// One key applied by the lane that owns bucket b, probing the digests in
// memory, unless it needs the eviction path: then nothing is changed and the
// function returns false.  *slot is the slot of the key's task.
template <int OP>
__device__ __forceinline__ bool lane_step(const TableView& t, const ApplyArgs& a, uint64_t b,
                                          uint64_t base, uint64_t i, uint64_t k, uint64_t in,
                                          bool has_in, int32_t& bsz, uint64_t& src,
                                          uint64_t& dst, int& slot) {
  const uint32_t B = t.B;
  const uint64_t h = murmur3(k);
  const uint64_t gi = global_idx(t, h);
  const uint32_t start = (uint32_t)(gi & (B - 1));
  const uint32_t d = key_digest(h);
  int dup = 0;
  const bool may_insert = OP != OP_ASSIGN_SCORES;
  const int p = probe_upsert(t, base, start, d, k, may_insert && bsz < (int32_t)B, &dup);
  src = dst = 0;
  slot = p;
  if (p < 0) return !may_insert;  // absent keys are a no-op for assign_scores
  lane_apply<OP>(t, a, base, row_ptr(t, b, 0), p, dup, i, k, in, has_in, d, bsz, src, dst);
  return true;
}

/* ------------------------------------------------------------------------ */
/* partitioned apply (all mutating batch operations)                         */
/* ------------------------------------------------------------------------ */
//
// 1. k_pcount: per 1024-key chunk g of the batch, the number of keys of each
//    partition p (256 consecutive buckets), counted in LDS.
// 2. k_pscan: per partition, its total and the offset of every segment
//    (g, p); partitions that fit their fixed region are placed there, larger
//    ones in a spill area.  Segments of a partition are consecutive and in
//    chunk order, so all keys of segment g precede those of g + 1 in batch
//    order.
// 3. k_pscatter: every key writes {key, batch index} into its segment.
// 4. k_apply_fast: one workgroup per partition of at most kFastLds entries,
//    key-parallel with batch-order results; buckets that need the eviction
//    path go to k_apply_deferred(_q) (one 16-lane group per bucket), larger
//    partitions and buckets with more than kLaneMax keys to k_apply_part.
// 5. k_apply_part: one workgroup per listed partition, taken from a counter.
//    It folds the heavy buckets' repeated keys, then loads the other entries
//    into LDS (in runs of whole segments when they do not fit at once),
//    groups them by bucket and applies each bucket's keys in batch order:
//    one lane per bucket while no eviction is needed, then one 16-lane group
//    per bucket that needs the eviction path or holds many keys.
//    k_big_count / k_big_fold / k_big_tasks do its per-entry passes over the
//    whole GPU for the largest partitions of batches with repeated keys.
// 6. find_or_insert's per-occurrence row copies (k_rowtasks) and
//    insert_and_evict's record compaction (k_evc_*).
// No atomics touch table memory: a bucket has exactly one owner at a time.

constexpr uint32_t kPartLds = kPartChunk;  // entries one LDS load holds
constexpr uint32_t kDgStride = 33;         // words per bucket digest row in LDS
constexpr uint32_t kLaneMax = 32;          // keys per bucket the lane pass takes
// Listed-partition flag: k_apply_fast applied every bucket of the partition
// with at most kLaneMax keys, and k_apply_part takes only the others.
constexpr uint32_t kPartLongOnly = 0x80000000u;
constexpr uint32_t kPartTaskCap = 128;     // queued row tasks per wave

__device__ __forceinline__ uint64_t bucket_of(const TableView& t, uint64_t k) {
  return global_idx(t, murmur3(k)) >> t.bshift;
}

// Partition of each of a thread's keys (kNone for reserved keys and keys past
// the batch).
__device__ __forceinline__ void chunk_parts(const TableView& t, const uint64_t* __restrict__ keys,
                                            uint64_t n, uint64_t i0, uint64_t (&kq)[kPartChunk / kBlock],
                                            uint32_t (&pq)[kPartChunk / kBlock]) {
#pragma unroll
  for (uint32_t q = 0; q < kPartChunk / kBlock; q++) {
    const uint64_t i = i0 + threadIdx.x + q * kBlock;
    kq[q] = i < n ? keys[i] : kEmptyKey;
  }
#pragma unroll
  for (uint32_t q = 0; q < kPartChunk / kBlock; q++)
    pq[q] = is_reserved(kq[q]) ? kNone : (uint32_t)(bucket_of(t, kq[q]) / kPartBuckets);
}

// Chunk of block b of nb: workgroups are dispatched round-robin over the
// chip's 8 XCDs, so this gives the blocks of one XCD a contiguous range of
// chunks.  A partition's segments from neighbouring chunks are adjacent in
// the entry array, so its cache lines are then written through one XCD's L2
// (and the scatter finds the chunk's keys in the L2 the count read them
// through).
__device__ __forceinline__ uint32_t xcd_chunk(uint32_t b, uint32_t nb) {
  constexpr uint32_t kXcds = 8;
  const uint32_t full = nb / kXcds * kXcds;
  return b < full ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
}

// The LDS histogram holds ps.prange partitions; a table with more partitions
// is counted in several passes over the chunk's keys, which stay in registers.
__global__ __launch_bounds__(kBlock) void k_pcount(TableView t, const uint64_t* __restrict__ keys,
                                                   uint64_t n, PartScratch ps) {
  extern __shared__ uint32_t s_h[];
  constexpr uint32_t kPer = kPartChunk / kBlock;
  const uint32_t NP = ps.np;
  const uint32_t g = xcd_chunk(blockIdx.x, gridDim.x);
  const uint64_t i0 = (uint64_t)g * kPartChunk;
  uint64_t kq[kPer];
  uint32_t pq[kPer];
  chunk_parts(t, keys, n, i0, kq, pq);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *ps.spill_top = 0;
    ps.dctr[0] = 0;
    ps.dctr[1] = 0;
    ps.dctr[2] = 0;
    ps.dctr[3] = 0;
    ps.dctr[4] = 0;
    ps.dctr[5] = 0;
  }
  // insert_and_evict flags a record per batch index; the flags of this
  // batch start clear.  Chunk g's indices are words [32 g, 32 g + 32) of
  // the bitmap, which holds n / 32 + 1 words.
  if (ps.ev_bits && threadIdx.x < kPartChunk / 32) {
    const uint64_t w = (uint64_t)g * (kPartChunk / 32) + threadIdx.x;
    if (w <= n / 32) ps.ev_bits[w] = 0;
  }
  uint32_t* H = ps.hist + (uint64_t)g * NP;
  for (uint32_t p0 = 0; p0 < NP; p0 += ps.prange) {
    const uint32_t w = NP - p0 < ps.prange ? NP - p0 : ps.prange;
    for (uint32_t q = threadIdx.x; q < w; q += kBlock) s_h[q] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++)
      if (pq[q] - p0 < w) atomicAdd(&s_h[pq[q] - p0], 1u);  // kNone never falls in range
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < w; q += kBlock) H[p0 + q] = s_h[q];
    __syncthreads();
  }
}

// kScanCols partitions per block of 1024 threads; thread (segment group sg,
// column c) handles chunks [sg * per, (sg + 1) * per) of partition c, so that
// each block row reads 128 contiguous bytes (one whole cache line) per chunk.
constexpr uint32_t kScanCols = 32;
constexpr uint32_t kScanGroups = 1024 / kScanCols;

__global__ __launch_bounds__(1024) void k_pscan(PartScratch ps) {
  constexpr uint32_t kReg = 32;  // column values a thread keeps in registers
  __shared__ uint32_t s_part[kScanGroups][kScanCols];
  __shared__ uint32_t s_base[kScanCols];
  const uint32_t c = threadIdx.x % kScanCols, sg = threadIdx.x / kScanCols;
  const uint32_t p = blockIdx.x * kScanCols + c;
  const uint32_t NP = ps.np, NG = ps.chunks;
  const uint32_t per = (NG + kScanGroups - 1) / kScanGroups;
  const uint32_t g0 = sg * per < NG ? sg * per : NG;
  const uint32_t g1 = g0 + per < NG ? g0 + per : NG;
  const bool live = p < NP;
  const bool in_reg = per <= kReg;
  gptr<uint32_t> col = G(ps.hist) + p;
  uint32_t v[kReg];
  uint32_t sum = 0;
  if (live && in_reg) {
#pragma unroll
    for (uint32_t j = 0; j < kReg; j++) {
      v[j] = g0 + j < g1 ? col[(uint64_t)(g0 + j) * NP] : 0u;
      sum += v[j];
    }
  } else if (live) {
#pragma unroll 8
    for (uint32_t g = g0; g < g1; g++) sum += col[(uint64_t)g * NP];
  }
  s_part[sg][c] = sum;
  __syncthreads();
  if (sg == 0 && live) {
    uint32_t tot = 0;
    for (uint32_t q = 0; q < kScanGroups; q++) tot += s_part[q][c];
    const uint32_t base =
        tot <= ps.cap ? p * ps.cap : NP * ps.cap + atomicAdd(ps.spill_top, tot);
    ps.pinfo[2 * p] = base;
    ps.pinfo[2 * p + 1] = tot;
    s_base[c] = base;
  }
  __syncthreads();
  if (live) {
    uint32_t off = s_base[c];
    for (uint32_t q = 0; q < sg; q++) off += s_part[q][c];
    if (in_reg) {
#pragma unroll
      for (uint32_t j = 0; j < kReg; j++) {
        if (g0 + j < g1) col[(uint64_t)(g0 + j) * NP] = off;
        off += v[j];
      }
    } else {
#pragma unroll 8
      for (uint32_t g = g0; g < g1; g++) {
        const uint32_t x = col[(uint64_t)g * NP];
        col[(uint64_t)g * NP] = off;
        off += x;
      }
    }
  }
}

__global__ __launch_bounds__(kBlock) void k_pscatter(TableView t,
                                                     const uint64_t* __restrict__ keys,
                                                     uint64_t n, PartScratch ps) {
  extern __shared__ uint32_t s_o[];
  constexpr uint32_t kPer = kPartChunk / kBlock;
  const uint32_t NP = ps.np;
  const uint32_t g = xcd_chunk(blockIdx.x, gridDim.x);
  const uint64_t i0 = (uint64_t)g * kPartChunk;
  uint64_t kq[kPer];
  uint32_t pq[kPer];
  chunk_parts(t, keys, n, i0, kq, pq);
  const uint32_t* H = ps.hist + (uint64_t)g * NP;
  gptr<u64x2> ent = G(reinterpret_cast<u64x2*>(ps.ent));
  for (uint32_t p0 = 0; p0 < NP; p0 += ps.prange) {
    const uint32_t w = NP - p0 < ps.prange ? NP - p0 : ps.prange;
    for (uint32_t q = threadIdx.x; q < w; q += kBlock) s_o[q] = H[p0 + q];
    __syncthreads();
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      if (pq[q] - p0 >= w) continue;  // other pass, reserved key or past the batch
      const uint32_t pos = atomicAdd(&s_o[pq[q] - p0], 1u);
      u64x2 v;
      v.x = kq[q];
      v.y = i0 + threadIdx.x + q * kBlock;
      ent[pos] = v;
    }
    __syncthreads();
  }
}

// Row tasks recorded by the lane pass, one word per batch index (0 = none),
// executed in batch order by k_rowcopy.  The top two bits give the kind:
//   kTaskIn:  input row i -> the table row at the address in the low bits
//   kTaskOut: the table row at the address -> output row i
//   kTaskFwd: output row j (low bits) -> output row i  (find_or_insert hit on
//             a row that key j inserted earlier in the same batch)
constexpr uint64_t kTaskIn = 1ull << 62;
constexpr uint64_t kTaskOut = 2ull << 62;
constexpr uint64_t kTaskFwd = 3ull << 62;
constexpr uint64_t kTaskMask = (1ull << 62) - 1;
constexpr uint8_t kNoSlot = 0xFF;

// Copies one row per lane that has a task (dst != 0), from src to dst; the
// wave copies the rows cooperatively, four rows per lane group in flight.
// `s_rows` is 64 words of LDS owned by the wave.
template <int U>
__device__ __forceinline__ void wave_copy_pairs(uint64_t src, uint64_t dst, uint32_t row_bytes,
                                                uint32_t* s_rows) {
  using T = typename UnitT<U>::T;
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t hm = __ballot(dst != 0);
  if (dst) s_rows[__popcll(hm & ((1ull << lane) - 1))] = lane;
  __builtin_amdgcn_wave_barrier();
  const uint32_t rows = __popcll(hm);
  const uint32_t units = row_bytes / U;
  uint32_t lpr = 64;
  while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;  // lanes per row
  const uint32_t rpi = 64 / lpr;
  const uint32_t sub = lane % lpr;
  for (uint32_t r0 = 0; r0 < rows; r0 += 4 * rpi) {
    const uint32_t r = r0 + lane / lpr;
    const bool ok0 = r < rows, ok1 = r + rpi < rows, ok2 = r + 2 * rpi < rows,
               ok3 = r + 3 * rpi < rows;
    const uint32_t l0 = s_rows[ok0 ? r : 0], l1 = s_rows[ok1 ? r + rpi : 0],
                   l2 = s_rows[ok2 ? r + 2 * rpi : 0], l3 = s_rows[ok3 ? r + 3 * rpi : 0];
    gptr<const T> s0 = G<const T>((uintptr_t)shfl_u64(src, (int)l0, 64));
    gptr<const T> s1 = G<const T>((uintptr_t)shfl_u64(src, (int)l1, 64));
    gptr<const T> s2 = G<const T>((uintptr_t)shfl_u64(src, (int)l2, 64));
    gptr<const T> s3 = G<const T>((uintptr_t)shfl_u64(src, (int)l3, 64));
    gptr<T> d0 = G<T>((uintptr_t)shfl_u64(dst, (int)l0, 64));
    gptr<T> d1 = G<T>((uintptr_t)shfl_u64(dst, (int)l1, 64));
    gptr<T> d2 = G<T>((uintptr_t)shfl_u64(dst, (int)l2, 64));
    gptr<T> d3 = G<T>((uintptr_t)shfl_u64(dst, (int)l3, 64));
    for (uint32_t u = sub; u < units; u += lpr) {
      const T v0 = s0[u], v1 = s1[u], v2 = s2[u], v3 = s3[u];
      if (ok0) d0[u] = v0;
      if (ok1) d1[u] = v1;
      if (ok2) d2[u] = v2;
      if (ok3) d3[u] = v3;
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// wave_copy_pairs with Q rows per lane group in flight: all loads of a round
// are issued before its first store, and rows past the end are not touched.
// The rows are streamed with non-temporal loads and stores, so that they do
// not evict the bucket metadata other keys of the call are probing from the
// L2 cache.
template <int U, int Q>
__device__ __forceinline__ void wave_copy_pairs_q(uint64_t src, uint64_t dst, uint32_t row_bytes,
                                                  uint32_t* s_rows) {
  using T = typename UnitT<U>::T;
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t hm = __ballot(dst != 0);
  if (dst) s_rows[__popcll(hm & ((1ull << lane) - 1))] = lane;
  __builtin_amdgcn_wave_barrier();
  const uint32_t rows = __popcll(hm);
  const uint32_t units = row_bytes / U;
  uint32_t lpr = 64;
  while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;  // lanes per row
  const uint32_t rpi = 64 / lpr;
  const uint32_t sub = lane % lpr;
  for (uint32_t r0 = 0; r0 < rows; r0 += Q * rpi) {
    gptr<const T> s[Q];
    gptr<T> d[Q];
    bool ok[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
      const uint32_t r = r0 + q * rpi + lane / lpr;
      ok[q] = r < rows;
      const uint32_t l = s_rows[ok[q] ? r : 0];
      s[q] = G<const T>((uintptr_t)shfl_u64(src, (int)l, 64));
      d[q] = G<T>((uintptr_t)shfl_u64(dst, (int)l, 64));
    }
    for (uint32_t u = sub; u < units; u += lpr) {
      T v[Q];
#pragma unroll
      for (int q = 0; q < Q; q++)
        if (ok[q]) v[q] = __builtin_nontemporal_load(&s[q][u]);
#pragma unroll
      for (int q = 0; q < Q; q++)
        if (ok[q]) __builtin_nontemporal_store(v[q], &d[q][u]);
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// Lane `u`'s copy unit, broadcast to the wave (u is wave-uniform).
__device__ __forceinline__ u32x4 bcast_unit(u32x4 v, uint32_t u) {
  u32x4 r;
  r.x = __builtin_amdgcn_readlane(v.x, u);
  r.y = __builtin_amdgcn_readlane(v.y, u);
  r.z = __builtin_amdgcn_readlane(v.z, u);
  r.w = __builtin_amdgcn_readlane(v.w, u);
  return r;
}
__device__ __forceinline__ u32x2 bcast_unit(u32x2 v, uint32_t u) {
  u32x2 r;
  r.x = __builtin_amdgcn_readlane(v.x, u);
  r.y = __builtin_amdgcn_readlane(v.y, u);
  return r;
}
__device__ __forceinline__ uint32_t bcast_unit(uint32_t v, uint32_t u) {
  return __builtin_amdgcn_readlane(v, u);
}
__device__ __forceinline__ uint16_t bcast_unit(uint16_t v, uint32_t u) {
  return (uint16_t)__builtin_amdgcn_readlane((uint32_t)v, u);
}
__device__ __forceinline__ uint8_t bcast_unit(uint8_t v, uint32_t u) {
  return (uint8_t)__builtin_amdgcn_readlane((uint32_t)v, u);
}

// Row copies of N tasks per lane (dst == 0: none), for task sets where many
// tasks read one row (the occurrences of a hot key read its table row, or
// its first occurrence's input): the source of the wave's first task is
// loaded once and written by every lane whose task reads it; the other
// tasks are copied pairwise.
template <int U, int N>
__device__ __forceinline__ void wave_copy_tasks(uint64_t (&src)[N], uint64_t (&dst)[N],
                                                uint32_t row_bytes, uint32_t* s_rows) {
  using T = typename UnitT<U>::T;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t units = row_bytes / U;
  uint64_t lead = 0;
#pragma unroll
  for (int r = 0; r < N; r++) {
    const uint64_t m = __ballot(dst[r] != 0);
    if (m && !lead) lead = shfl_u64(src[r], __ffsll((unsigned long long)m) - 1, 64);
  }
  if (lead && units <= 64) {
    // lpr lanes per row, one unit each; rpi rows per store instruction, so
    // every instruction writes whole lines.
    uint32_t lpr = 64;
    while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;
    const uint32_t rpi = 64 / lpr, sub = lane % lpr;
    const T v = sub < units ? __builtin_nontemporal_load(G<const T>((uintptr_t)lead) + sub) : T{};
#pragma unroll
    for (int r = 0; r < N; r++) {
      const bool use = dst[r] != 0 && src[r] == lead;
      const uint64_t hm = __ballot(use);
      if (use) s_rows[__popcll(hm & ((1ull << lane) - 1))] = lane;
      __builtin_amdgcn_wave_barrier();
      const uint32_t rows = __popcll(hm);
      for (uint32_t r0 = 0; r0 < rows; r0 += rpi) {
        const uint32_t row = r0 + lane / lpr;
        const uint32_t ol = s_rows[row < rows ? row : 0];
        const uint64_t d = shfl_u64(dst[r], (int)ol, 64);
        if (row < rows && sub < units) __builtin_nontemporal_store(v, G<T>((uintptr_t)d) + sub);
      }
      __builtin_amdgcn_wave_barrier();
      if (use) dst[r] = 0;
    }
  }
#pragma unroll
  for (int r = 0; r < N; r++) wave_copy_pairs<U>(src[r], dst[r], row_bytes, s_rows);
}

// Executes and clears the row tasks of batch indices `i`, one per lane (a
// lane with valid == false takes part without a task).
template <int U>
__device__ __forceinline__ void wave_run_tasks(const ApplyArgs& a, gptr<uint64_t> trow,
                                               uint64_t i, bool valid, uint32_t row_bytes,
                                               uint32_t* s_rows) {
  const uint64_t R = row_bytes;
  uint64_t tv = 0;
  if (valid) {
    tv = trow[i];
    if (tv) trow[i] = 0;
  }
  uint64_t src = 0, dst = 0;
  if (tv) {
    const uint64_t kind = tv & ~kTaskMask, val = tv & kTaskMask;
    if (kind == kTaskIn) {
      src = (uint64_t)(uintptr_t)(a.in_values + i * R);
      dst = val;
    } else if (kind == kTaskOut) {
      src = val;
      dst = (uint64_t)(uintptr_t)(a.io_values + i * R);
    } else {
      src = (uint64_t)(uintptr_t)(a.io_values + val * R);
      dst = (uint64_t)(uintptr_t)(a.io_values + i * R);
    }
  }
  wave_copy_pairs<U>(src, dst, row_bytes, s_rows);
}

// Heavy buckets: buckets that receive more than kHeavyMin keys of a partition
// (duplicate-heavy batches such as Zipf traffic, where one key can occur
// tens of thousands of times).  When the distinct keys of such a bucket that
// are absent from the table fit its EMPTY slots, no key of the call can
// evict or be refused, and the batch-order outcome depends only on
//   * the order of the new keys' first occurrences (each takes the first
//     EMPTY slot in circular order from its start slot, as one key would),
//   * per distinct key, a fold of its occurrences' scores:
//       Lfu:       sum of the inputs (added to the old score of a present key);
//       EpochLfu:  (epoch << 32) | min(old low word + sum of input low words,
//                  0xFFFFFFFF) -- consecutive saturating adds compose into one;
//                  with the epoch ignored the high word is the last input's;
//       others:    the desired score of the last occurrence,
//   * and per occurrence a row copy that the fold fixes: find_or_insert
//     returns the table row of a present key, or the first occurrence's input
//     for a new key; the upserts write the last occurrence's input.
// Such a bucket costs one pass of its distinct keys instead of one serial
// step per occurrence.  Buckets where that condition fails (or whose keys do
// not fit the block's key map) keep the serial batch-order walk.
constexpr uint32_t kMapCap = 1024;   // distinct keys of a partition's heavy buckets
constexpr uint32_t kMapProbe = 64;   // linear-probe limit of the key map
constexpr uint32_t kItemCap = 128;   // distinct keys of a bucket without eviction (<= B)
constexpr uint32_t kHvPer = 8;       // entries per thread per tile of the streaming passes
constexpr uint32_t kHeavyMin = 8;    // a bucket with more entries in its partition is folded
constexpr uint8_t kHvNone = 0, kHvDone = 1, kHvSerial = 2;
constexpr uint16_t kMapNew = 0x100;     // key map result: new key ...
constexpr uint16_t kMapPlaced = 0x200;  // ... placed at the slot in the low byte

__device__ __forceinline__ void group_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ uint32_t map_home(uint64_t h) {
  return (uint32_t)(h ^ (h >> 29)) & (kMapCap - 1);
}

// Final score of a heavy-bucket key from the fold of its occurrences (see
// above); `sum` is the sum of the inputs (Lfu) or of their low words
// (EpochLfu), `in_last` the input of the last occurrence.
template <int OP>
__device__ __forceinline__ uint64_t heavy_score(const ScoreCtx& c, bool has_in, bool is_new,
                                                uint64_t old, uint64_t sum, uint64_t in_last) {
  const uint64_t old_lo = is_new ? 0 : (old & kScoreMask);
  if (OP == OP_ASSIGN_SCORES) {
    switch (c.strategy) {
      case kLru: return c.clock;
      case kLfu: return old + sum;
      case kEpochLru: return (c.epoch << 32) | ((c.clock >> 20) & kScoreMask);
      case kEpochLfu: {
        const uint64_t lo = old_lo + sum;
        return (c.epoch << 32) | (lo < kScoreMask ? lo : kScoreMask);
      }
      default: return in_last;
    }
  }
  switch (c.strategy) {
    case kLfu: return is_new ? sum : old + sum;
    case kEpochLfu: {
      const uint64_t hi = c.epoch == kIgnoredEpoch ? (in_last >> 32) : c.epoch;
      const uint64_t lo = old_lo + sum;
      return (hi << 32) | (lo < kScoreMask ? lo : kScoreMask);
    }
    default: return score_desired(c, has_in, in_last);
  }
}

template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_apply_part(TableView t, ApplyArgs a, PartScratch ps) {
  // accum_or_assign accumulates in place, in batch order, inside this kernel;
  // the other operations record their row movements for k_rowcopy.
  constexpr bool kDeferRows = OP != OP_ACCUM_OR_ASSIGN;
  constexpr uint32_t kQ = kDeferRows ? 1 : kPartTaskCap;
  __shared__ uint64_t s_key[kPartLds];
  __shared__ uint32_t s_idx[kPartLds];
  __shared__ uint8_t s_slot[kPartLds];  // slot whose row the step wrote
  __shared__ uint32_t s_cnt[kPartBuckets], s_off[kPartBuckets], s_fill[kPartBuckets];
  __shared__ uint32_t s_defer[kPartBuckets];
  __shared__ uint32_t s_perm[kPartBuckets];  // buckets by decreasing key count
  __shared__ uint32_t s_cls[64];             // buckets per key count class
  __shared__ uint32_t s_rows[kBlock / 64][64];
  // Digest rows of the buckets (run loop); before the run loop, the key map
  // and item lists of the heavy-bucket pass.
  __shared__ __align__(16) uint32_t s_dg[kPartBuckets * kDgStride];
  __shared__ uint32_t s_wsum[kBlock / 64];
  __shared__ uint64_t s_src[kBlock / 64][kQ];
  __shared__ uint64_t s_dst[kBlock / 64][kQ];
  __shared__ uint32_t s_ndefer, s_c1;
  __shared__ uint32_t s_tot[kPartBuckets];  // entries per bucket over the partition
  __shared__ uint8_t s_hst[kPartBuckets];   // heavy-bucket state
  __shared__ uint8_t s_hlist[kPartBuckets];
  __shared__ uint32_t s_icnt[kBlock / 16];
  __shared__ uint32_t s_nheavy, s_mfull, s_kept, s_li;
  __shared__ uint32_t s_head[kPartBuckets];  // first key map entry of each heavy bucket
  __shared__ uint64_t s_rbase[kPartBuckets];  // row 0 of each bucket (heavy-bucket copies)
  __shared__ uint32_t s_hw[kHvPer][kBlock / 64];  // kept entries per sub-tile and wave
  __shared__ int32_t s_bslot;     // big slot of the partition (-1: none)
  __shared__ uint32_t s_anyser;   // a heavy bucket was left to the serial walk
  // Key map {key, fold sum, first / last batch index, result, bucket}.
  uint64_t* const mkey = reinterpret_cast<uint64_t*>(s_dg);
  uint64_t* const msum = mkey + kMapCap;
  uint32_t* const mfirst = reinterpret_cast<uint32_t*>(msum + kMapCap);
  uint32_t* const mlast = mfirst + kMapCap;
  uint16_t* const mres = reinterpret_cast<uint16_t*>(mlast + kMapCap);
  uint8_t* const mbk = reinterpret_cast<uint8_t*>(mres + kMapCap);
  uint16_t* const items = reinterpret_cast<uint16_t*>(mbk + kMapCap);  // [16][kItemCap]
  uint16_t* const mnext = items + (kBlock / 16) * kItemCap;  // next entry of the bucket
  static_assert(kMapCap * (8 + 8 + 4 + 4 + 2 + 1 + 2) + (kBlock / 16) * kItemCap * 2 <=
                    sizeof(uint32_t) * kPartBuckets * kDgStride,
                "key map fits the digest rows");
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t B = t.B;
  const uint32_t R = t.row_bytes;
  const bool has_in = a.in_scores != nullptr;
  gptr<const u64x2> ent = G(reinterpret_cast<const u64x2*>(ps.ent));
  gptr<u64x2> ent_w = G(reinterpret_cast<u64x2*>(ps.ent));  // in-place compaction
  gptr<uint64_t> trow = G(ps.trow);
  uint32_t added = 0;
  // The partitions k_apply_fast left (usually none: then every block leaves
  // without touching the shared counter): whole partitions from the front of
  // the list, long-bucket-only ones from its back.
  const uint32_t nwhole = *(volatile uint32_t*)&ps.dctr[2];
  const uint32_t nlist = nwhole + *(volatile uint32_t*)&ps.dctr[5];
  if (nlist == 0) return;
  // Blocks take partitions from a counter, so that a block holding a large
  // partition is not also given a fixed share of the others.  The whole
  // partitions, which take a block two to three times as long, go first:
  // taken last, one of them would set the kernel's end.
  for (;;) {
    if (tid == 0) s_li = atomicAdd(&ps.dctr[3], 1u);
    __syncthreads();
    const uint32_t li = s_li;
    if (li >= nlist) break;  // block-uniform
    const uint32_t pl = li < nwhole ? ps.plist[li] : ps.plist[ps.np - 1 - (li - nwhole)];
    // kPartLongOnly: k_apply_fast applied the buckets with at most kLaneMax
    // entries; only the longer ones are folded (or walked) here.
    const bool long_only = (pl & kPartLongOnly) != 0;
    const uint32_t p = pl & ~kPartLongOnly;
    const uint32_t hmin = long_only ? kLaneMax : kHeavyMin;  // heavy: more entries than this
    const uint32_t base_e = ps.pinfo[2 * p], m = ps.pinfo[2 * p + 1];
    const uint64_t part_b0 = (uint64_t)p * kPartBuckets;
    uint32_t m_run = m;  // entries left to the run loop
    gptr<const u64x2> rent = ent;  // entries of the run loop
    uint32_t run_base = base_e;
    if constexpr (kDeferRows) {
      // A big partition's counts and key map were built grid-wide.
      if (tid == 0) {
        s_bslot = -1;
        s_anyser = 0;
      }
      __syncthreads();
      if (ps.big) {
        uint32_t nbb = *(volatile uint32_t*)&ps.dctr[4];
        nbb = nbb < kBigMax ? nbb : kBigMax;
        for (uint32_t q = tid; q < nbb; q += kBlock)
          if (ps.big_part[q] == p) s_bslot = (int32_t)q;
      }
      __syncthreads();
      const int32_t bslot = s_bslot;
      BigSlot* const bs = bslot >= 0 ? ps.big + bslot : nullptr;
      /* H0. Entries per bucket over the whole partition (a wave adds the
         count of its leading lane's bucket with one atomic). */
      s_tot[tid] = bs ? bs->tot[tid] : 0u;
      s_hst[tid] = kHvNone;
      s_rbase[tid] = part_b0 + tid < t.buckets
                         ? (uint64_t)(uintptr_t)row_ptr(t, part_b0 + tid, 0) : 0;
      if (tid == 0) {
        s_nheavy = 0;
        s_mfull = 0;
        s_kept = 0;
      }
      __syncthreads();
      for (uint32_t e0 = 0; !bs && e0 < m; e0 += kBlock * kHvPer) {
        uint64_t kq[kHvPer];
#pragma unroll
        for (uint32_t r = 0; r < kHvPer; r++) {
          const uint32_t e = e0 + tid + r * kBlock;
          kq[r] = e < m ? ent[base_e + e].x : kEmptyKey;
        }
#pragma unroll
        for (uint32_t r = 0; r < kHvPer; r++) {
          const bool v = e0 + tid + r * kBlock < m;
          const uint32_t bk = v ? (uint32_t)(bucket_of(t, kq[r]) % kPartBuckets) : 0u;
          const uint64_t act = __ballot(v);
          if (act) {
            const int ld = __ffsll((unsigned long long)act) - 1;
            const uint32_t lb = __shfl(bk, ld, 64);
            const uint64_t same = __ballot(v && bk == lb);
            if ((int)lane == ld) atomicAdd(&s_tot[lb], (uint32_t)__popcll(same));
            if (v && bk != lb) atomicAdd(&s_tot[bk], 1u);
          }
        }
      }
      __syncthreads();
      s_head[tid] = kNone;
      if (s_tot[tid] > hmin) s_hlist[atomicAdd(&s_nheavy, 1u)] = (uint8_t)tid;
      __syncthreads();
      const uint32_t nheavy = s_nheavy;
      if (long_only && !nheavy) m_run = 0;  // nothing left (not expected)
      if (nheavy) {
        const bool sum_in = a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu;
        const bool fold_ok =
            has_in || !(sum_in || a.sc.strategy == kCustomized);
        /* H1. Fold the heavy buckets' entries into the key map (for a big
           partition: load the map folded grid-wide and link its keys into
           their buckets' lists). */
        for (uint32_t q = tid; q < kMapCap; q += kBlock) {
          mkey[q] = bs ? bs->mkey[q] : kEmptyKey;
          msum[q] = bs ? bs->msum[q] : 0;
          mfirst[q] = bs ? bs->mfirst[q] : kNone;
          mlast[q] = bs ? bs->mlast[q] : 0;
        }
        if (bs && tid == 0) s_mfull = bs->mfull;
        __syncthreads();
        if (bs) {
          for (uint32_t q = tid; q < kMapCap; q += kBlock) {
            const uint64_t k = mkey[q];
            if (k != kEmptyKey) {
              const uint32_t bk = (uint32_t)(bucket_of(t, k) % kPartBuckets);
              mnext[q] = (uint16_t)atomicExch(&s_head[bk], q);
              mbk[q] = (uint8_t)bk;
            }
          }
          __syncthreads();
        }
        // The next tile's entries load while this tile's input scores are
        // gathered (their addresses depend on the entries).
        u64x2 nq[kHvPer];
#pragma unroll
        for (uint32_t r = 0; r < kHvPer; r++) {
          const uint32_t e = tid + r * kBlock;
          nq[r].x = kEmptyKey;
          nq[r].y = 0;
          if (!bs && e < m) nq[r] = ent[base_e + e];
        }
        for (uint32_t e0 = 0; !bs && e0 < m; e0 += kBlock * kHvPer) {
          if (*(volatile uint32_t*)&s_mfull) break;  // block-uniform: set before a barrier
          u64x2 eq[kHvPer];
          uint64_t hq_[kHvPer], cq[kHvPer];
          bool hvq[kHvPer];
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            eq[r] = nq[r];
            const uint32_t e = e0 + kBlock * kHvPer + tid + r * kBlock;
            nq[r].x = kEmptyKey;
            nq[r].y = 0;
            if (e < m) nq[r] = ent[base_e + e];
          }
          // Input scores of every entry of the tile, issued before the
          // hashing that tells which entries are heavy.
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            cq[r] = 0;
            if (sum_in && has_in && e0 + tid + r * kBlock < m) cq[r] = G(a.in_scores)[eq[r].y];
          }
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            hq_[r] = murmur3(eq[r].x);
            const uint32_t bk = (uint32_t)((global_idx(t, hq_[r]) >> t.bshift) % kPartBuckets);
            hvq[r] = e0 + tid + r * kBlock < m && s_tot[bk] > hmin;
          }
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            const uint64_t in = cq[r];
            cq[r] = !hvq[r] ? 0 : a.sc.strategy == kLfu ? in : (in & kScoreMask);
          }
          // The wave's leading key (first heavy entry of the tile) is folded
          // over all of the tile's sub-rounds with one reduction.
          uint64_t lk = 0;
          bool have_lead = false;
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            const uint64_t act = __ballot(hvq[r]);
            if (act && !have_lead) {
              lk = shfl_u64(eq[r].x, __ffsll((unsigned long long)act) - 1, 64);
              have_lead = true;
            }
          }
          uint32_t l1 = kNone, l2 = 0;
          uint64_t l3 = 0;
          if (have_lead) {
#pragma unroll
            for (uint32_t r = 0; r < kHvPer; r++) {
              if (hvq[r] && eq[r].x == lk) {
                const uint32_t i = (uint32_t)eq[r].y;
                l1 = i < l1 ? i : l1;
                l2 = i > l2 ? i : l2;
                l3 += cq[r];
                hvq[r] = false;  // folded into the leader's update
              }
            }
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) {
              const uint32_t o1 = __shfl_xor(l1, d, 64), o2 = __shfl_xor(l2, d, 64);
              l1 = o1 < l1 ? o1 : l1;
              l2 = o2 > l2 ? o2 : l2;
              l3 += shfl_xor_u64(l3, d, 64);
            }
          }
          // Map updates: the leader's folded occurrences (lane 0), then every
          // other heavy entry on its own.
#pragma unroll
          for (uint32_t r = 0; r <= kHvPer; r++) {
            bool mine;
            uint64_t k, h, csum;
            uint32_t fmin, fmax;
            if (r == kHvPer) {
              mine = have_lead && lane == 0;
              k = lk;
              h = murmur3(lk);
              fmin = l1;
              fmax = l2;
              csum = l3;
            } else {
              mine = hvq[r];
              k = eq[r].x;
              h = hq_[r];
              fmin = fmax = (uint32_t)eq[r].y;
              csum = cq[r];
            }
            if (mine) {
              const uint32_t bk = (uint32_t)((global_idx(t, h) >> t.bshift) % kPartBuckets);
              uint32_t q = map_home(h);
              bool ok = false;
              for (uint32_t pr = 0; pr < kMapProbe; pr++) {
                const uint64_t cur = atomicCAS(reinterpret_cast<unsigned long long*>(&mkey[q]),
                                               (unsigned long long)kEmptyKey,
                                               (unsigned long long)k);
                if (cur == kEmptyKey || cur == k) {
                  // The lane that installs the key links it into its bucket's list.
                  if (cur == kEmptyKey) mnext[q] = (uint16_t)atomicExch(&s_head[bk], q);
                  ok = true;
                  break;
                }
                q = (q + 1) & (kMapCap - 1);
              }
              if (!ok) {
                s_mfull = 1;
              } else {
                atomicMin(&mfirst[q], fmin);
                atomicMax(&mlast[q], fmax);
                if (csum) atomicAdd(reinterpret_cast<unsigned long long*>(&msum[q]),
                                    (unsigned long long)csum);
                mbk[q] = (uint8_t)bk;
              }
            }
          }
          __syncthreads();
        }
        __syncthreads();
        /* H2. One 16-lane group per heavy bucket: the bucket in registers,
           its distinct keys looked up, and, when the new ones fit its EMPTY
           slots, placed in first-occurrence order with folded scores. */
        const uint32_t gi = tid >> 4, gl = tid & 15;
        const bool mfull = s_mfull != 0;
        for (uint32_t hq = gi; hq < nheavy; hq += kBlock / 16) {
          const uint32_t bk = s_hlist[hq];
          const uint64_t b = part_b0 + bk;
          uint16_t* const it = items + gi * kItemCap;
          bool serial = mfull || !fold_ok;
          if (gl == 0) s_icnt[gi] = 0;
          group_sync();
          if (!serial) {
            if (gl == 0) {
              uint32_t c = 0;
              for (uint32_t q = s_head[bk]; q != 0xFFFFu && q != kNone; q = mnext[q]) {
                if (c < kItemCap) it[c] = (uint16_t)q;
                c++;
              }
              s_icnt[gi] = c;
            }
            group_sync();
          }
          const uint32_t ni = s_icnt[gi];
          if (ni > kItemCap) serial = true;
          if (serial) {
            if (gl == 0) s_hst[bk] = kHvSerial;
            continue;
          }
          Bucket16 S;
          bucket_load(t, S, b, gl);
          uint32_t ne = 0;
#pragma unroll
          for (uint32_t j = 0; j < 8; j++) ne += dg_of(S, j) == kEmptyDigest ? 1u : 0u;
#pragma unroll
          for (int d = 8; d > 0; d >>= 1) ne += __shfl_xor(ne, d, 16);
          // Present keys keep their slot; new keys are marked.
          uint32_t nnew = 0;
          for (uint32_t x = 0; x < ni; x++) {
            const uint32_t q = it[x];
            const uint64_t k = mkey[q];
            const uint32_t d = key_digest(murmur3(k));
            uint32_t best = kNone;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
              if (dg_of(S, j) == d && S.key[j] == k) best = gl + 16 * j;
            best = group_min_u32(best);
            if (gl == 0) mres[q] = best == kNone ? kMapNew : (uint16_t)best;
            nnew += best == kNone ? 1u : 0u;
          }
          group_sync();
          if (OP == OP_ASSIGN_SCORES) nnew = 0;  // absent keys are a no-op
          if (nnew > ne) {
            if (gl == 0) s_hst[bk] = kHvSerial;
            continue;
          }
          // New keys in order of first occurrence: first EMPTY slot in
          // circular order from the start slot.
          for (uint32_t r = 0; r < nnew; r++) {
            uint32_t bf = kNone, bq = 0;
            for (uint32_t x = gl; x < ni; x += 16) {
              const uint32_t q = it[x];
              if (mres[q] == kMapNew && mfirst[q] < bf) {
                bf = mfirst[q];
                bq = q;
              }
            }
#pragma unroll
            for (int d = 8; d > 0; d >>= 1) {
              const uint32_t of = __shfl_xor(bf, d, 16), oq = __shfl_xor(bq, d, 16);
              if (of < bf) {
                bf = of;
                bq = oq;
              }
            }
            const uint64_t k = mkey[bq];
            const uint64_t h = murmur3(k);
            const uint32_t start = (uint32_t)(global_idx(t, h) & (B - 1));
            const uint32_t d = key_digest(h);
            uint32_t rl = kNone;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
              if (dg_of(S, j) == kEmptyDigest) {
                const uint32_t rr = (gl + 16 * j - start) & (B - 1);
                rl = rr < rl ? rr : rl;
              }
            const uint32_t pos = (start + group_min_u32(rl)) & (B - 1);
            if (gl == (pos & 15u)) {
              dg_set(S, pos >> 4, d);
              rec_set(S.key, pos >> 4, k);
            }
            if (gl == 0) mres[bq] = (uint16_t)(kMapNew | kMapPlaced | pos);
            group_sync();
          }
          // Folded scores and the slots' records.  The last occurrence's
          // input score of item x sits in lane x % 16, register x / 16.
          uint64_t inl[8];
#pragma unroll
          for (uint32_t j = 0; j < 8; j++) {
            const uint32_t x = gl + 16 * j;
            inl[j] = (has_in && x < ni) ? G(a.in_scores)[mlast[it[x]]] : 0;
          }
          int32_t nadd = 0;
          for (uint32_t x = 0; x < ni; x++) {
            const uint32_t q = it[x];
            const uint32_t rs = mres[q];
            const bool is_new = (rs & kMapNew) != 0;
            const uint64_t in_last = shfl_u64(rec_get(inl, x >> 4), (int)(x & 15u), 16);
            if (OP == OP_ASSIGN_SCORES && is_new) continue;
            const uint32_t pos = rs & 0xFFu;
            if (gl == (pos & 15u)) {
              const uint64_t old = rec_get(S.score, pos >> 4);
              const uint64_t ns = heavy_score<OP>(a.sc, has_in, is_new, old, msum[q], in_last);
              if (is_new) {
                const uint64_t k = mkey[q];
                slot_store(t, sbase(t, S) + pos, k, ns);
                G(t.digests)[sbase(t, S) + pos] = (uint8_t)key_digest(murmur3(k));
              } else {
                slot_score(t, sbase(t, S) + pos) = ns;
              }
            }
            nadd += is_new ? 1 : 0;
          }
          if (gl == 0) {
            if (nadd) {
              G(t.bsize)[b] = S.bsz + nadd;
              added += (uint32_t)nadd;
            }
            s_hst[bk] = kHvDone;
          }
        }
        __syncthreads();
        if (s_hst[tid] == kHvSerial) s_anyser = 1;
        __syncthreads();
        // A big partition whose heavy buckets were all folded and whose other
        // entries fit one run leaves the row work to k_big_tasks and runs the
        // entries k_big_fold listed.
        const bool big_fast = bs && !s_mfull && !s_anyser && bs->nlight <= kBigLight;
        if (big_fast) {
          for (uint32_t q = tid; q < kMapCap; q += kBlock)
            if (mkey[q] != kEmptyKey) bs->mres[q] = mres[q];
          if (tid == 0) bs->fast = 1;
          rent = G(reinterpret_cast<const u64x2*>(bs->light));
          run_base = 0;
          m_run = bs->nlight;
        }
        /* H3. Row copies of the folded buckets' occurrences (find_or_insert:
           row tasks), and the other entries compacted in place (order kept)
           for the run loop. */
        for (uint32_t e0 = 0; !big_fast && e0 < m; e0 += kBlock * kHvPer) {
          u64x2 eq[kHvPer];
          uint64_t srcq[kHvPer], dstq[kHvPer];
          bool keepq[kHvPer];
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            const uint32_t e = e0 + tid + r * kBlock;
            eq[r].x = kEmptyKey;
            eq[r].y = 0;
            if (e < m) eq[r] = ent[base_e + e];
          }
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            const uint64_t k = eq[r].x;
            const uint64_t i = eq[r].y;
            const bool v = e0 + tid + r * kBlock < m;
            const uint64_t h = murmur3(k);
            const uint32_t bk = (uint32_t)((global_idx(t, h) >> t.bshift) % kPartBuckets);
            const bool done = v && s_hst[bk] == kHvDone;
            uint64_t src = 0, dst = 0;
            if (done && OP != OP_ASSIGN_SCORES) {
              uint32_t q = map_home(h);
              while (mkey[q] != k) q = (q + 1) & (kMapCap - 1);  // present: inserted in H1
              const uint32_t rs = mres[q];
              const uint64_t trow_a = s_rbase[bk] + (uint64_t)(rs & 0xFFu) * R;
              if (OP == OP_FIND_OR_INSERT) {
                // One copy per occurrence: recorded for k_rowtasks, which
                // spreads them over the whole GPU.
                trow[i] = !(rs & kMapNew) ? (kTaskOut | trow_a)
                          : i == mfirst[q] ? (kTaskIn | trow_a)
                                           : (kTaskFwd | (uint64_t)mfirst[q]);
              } else if (i == mlast[q]) {
                src = (uint64_t)(uintptr_t)(a.in_values + i * R);
                dst = trow_a;
              }
            }
            srcq[r] = src;
            dstq[r] = dst;
            keepq[r] = v && !done && (!long_only || s_tot[bk] > kLaneMax);
          }
          uint64_t kmq[kHvPer];
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            kmq[r] = __ballot(keepq[r]);
            if (lane == 0) s_hw[r][wv] = (uint32_t)__popcll(kmq[r]);
          }
          __syncthreads();  // every entry of this tile has been read
          // Entries of sub-tile r precede those of sub-tile r + 1; a kept
          // entry moves to the number of kept entries before it.
          uint32_t run = s_kept;
#pragma unroll
          for (uint32_t r = 0; r < kHvPer; r++) {
            uint32_t pre = run;
#pragma unroll
            for (uint32_t q = 0; q < kBlock / 64; q++) {
              pre += q < wv ? s_hw[r][q] : 0u;
              run += s_hw[r][q];
            }
            if (keepq[r])
              ent_w[base_e + pre + (uint32_t)__popcll(kmq[r] & ((1ull << lane) - 1))] = eq[r];
          }
          wave_copy_tasks<U, kHvPer>(srcq, dstq, R, s_rows[wv]);
          __syncthreads();
          if (tid == 0) s_kept = run;
        }
        __syncthreads();
        if (!big_fast) m_run = s_kept;
        __syncthreads();
      }
    }
    uint32_t c0 = run_base;
    const uint32_t end_e = run_base + m_run;
    while (c0 < end_e) {
      // This run of entries: the whole list when it fits, else whole
      // segments in chunk order.  A segment holds at most kPartChunk =
      // kPartLds entries of one chunk, so (c0, c0 + kPartLds] holds a chunk
      // boundary; the run ends at the last one.
      if (end_e - c0 > kPartLds) {
        if (tid == 0) s_c1 = c0;
        __syncthreads();
        for (uint32_t x = c0 + 1 + tid; x <= c0 + kPartLds; x += kBlock)
          if (rent[x].y / kPartChunk != rent[x - 1].y / kPartChunk) atomicMax(&s_c1, x);
        __syncthreads();
      }
      if (tid == 0) {
        if (end_e - c0 <= kPartLds) s_c1 = end_e;
        s_ndefer = 0;
      }
      s_cnt[tid] = 0;
      if (tid < 64) s_cls[tid] = 0;
      __syncthreads();
      const uint32_t c1 = s_c1;
      const uint32_t mc = c1 - c0;
      // Group the run's entries by bucket.
      for (uint32_t e = tid; e < mc; e += kBlock)
        atomicAdd(&s_cnt[bucket_of(t, rent[c0 + e].x) % kPartBuckets], 1u);
      __syncthreads();
      {
        const uint32_t v = s_cnt[tid];
        uint32_t x = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const uint32_t y = __shfl_up(x, d, 64);
          if (lane >= (uint32_t)d) x += y;
        }
        if (lane == 63) s_wsum[wv] = x;
        __syncthreads();
        uint32_t pre = 0;
        for (uint32_t q = 0; q < wv; q++) pre += s_wsum[q];
        s_off[tid] = pre + x - v;
        s_fill[tid] = pre + x - v;
      }
      __syncthreads();
      for (uint32_t e = tid; e < mc; e += kBlock) {
        const u64x2 v = rent[c0 + e];
        const uint32_t pos = atomicAdd(&s_fill[bucket_of(t, v.x) % kPartBuckets], 1u);
        s_key[pos] = v.x;
        s_idx[pos] = (uint32_t)v.y;
      }
      if (kDeferRows) {
        // Digest rows of the partition's buckets (one contiguous region).
        gptr<const u32x4> dsrc = (gptr<const u32x4>)(G(t.digests) + part_b0 * B);
        const uint32_t nbk =
            t.buckets - part_b0 < kPartBuckets ? (uint32_t)(t.buckets - part_b0) : kPartBuckets;
        for (uint32_t q = tid; q < nbk * 8; q += kBlock) {
          const u32x4 v = dsrc[q];
          uint32_t* row = s_dg + (q >> 3) * kDgStride + (q & 7) * 4;
          row[0] = v.x;
          row[1] = v.y;
          row[2] = v.z;
          row[3] = v.w;
        }
      }
      __syncthreads();
      if (kDeferRows) {
        // Lanes take buckets in decreasing order of key count, so that a wave
        // holds buckets of similar work (counts above 63 tie).
        const uint32_t cc = s_cnt[tid] < 63 ? s_cnt[tid] : 63;
        const uint32_t r = atomicAdd(&s_cls[63 - cc], 1u);
        __syncthreads();
        // Exclusive prefix of the 64 count classes, by one wave.
        if (wv == 0) {
          const uint32_t v = s_cls[lane];
          uint32_t x = v;
#pragma unroll
          for (int d = 1; d < 64; d <<= 1) {
            const uint32_t y = __shfl_up(x, d, 64);
            if (lane >= (uint32_t)d) x += y;
          }
          s_defer[lane] = x - v;  // class offsets (s_defer is free here)
        }
        __syncthreads();
        s_perm[s_defer[63 - cc] + r] = tid;
        __syncthreads();
      }

      // Lane pass: the lane owns bucket bk of the partition.
      const uint32_t bk = kDeferRows ? s_perm[tid] : tid;
      const uint64_t b = part_b0 + bk;
      const bool own = b < t.buckets;
      const uint32_t c = own ? s_cnt[bk] : 0;
      const uint32_t o = s_off[bk];
      const bool lane_ok = c > 0 && c <= kLaneMax;
      if (lane_ok) {
        // Batch order within the bucket (insertion sort of a short run).
        for (uint32_t x = 1; x < c; x++) {
          const uint64_t kx = s_key[o + x];
          const uint32_t ix = s_idx[o + x];
          uint32_t y = x;
          while (y > 0 && s_idx[o + y - 1] > ix) {
            s_key[o + y] = s_key[o + y - 1];
            s_idx[o + y] = s_idx[o + y - 1];
            y--;
          }
          s_key[o + y] = kx;
          s_idx[o + y] = ix;
        }
      } else if (c > kLaneMax) {
        s_defer[atomicAdd(&s_ndefer, 1u)] = bk << 16;
      }
      const uint64_t base = b * (uint64_t)B;
      int32_t bsz = lane_ok ? G(t.bsize)[b] : 0;
      const int32_t bsz0 = bsz;
      uint32_t wr0 = 0, wr1 = 0, wr2 = 0, wr3 = 0;
      if constexpr (kDeferRows) {
        if (lane_ok) {
          uint32_t* dg = s_dg + bk * kDgStride;
          const gptr<uint8_t> rows0 = row_ptr(t, b, 0);
          constexpr bool may_insert = OP != OP_ASSIGN_SCORES;
          for (uint32_t step = 0; step < c; step++) {
            const uint64_t k = s_key[o + step];
            const uint64_t i = s_idx[o + step];
            const uint64_t in = has_in ? G(a.in_scores)[i] : 0;
            const uint64_t h = murmur3(k);
            const uint32_t start = (uint32_t)(global_idx(t, h) & (B - 1));
            const uint32_t d = key_digest(h);
            int dup = 0;
            const int slot =
                probe_upsert_lds(t, dg, base, start, d, k, may_insert && bsz < (int32_t)B, &dup);
            if (slot < 0 && may_insert) {
              // Eviction path: the 16-lane pass resumes here, after running the
              // row tasks recorded so far for this bucket.
              s_defer[atomicAdd(&s_ndefer, 1u)] = (bk << 16) | step;
              break;
            }
            uint64_t src = 0, dst = 0;
            uint32_t res = 0;
            if (slot >= 0) {
              res = lane_apply<OP>(t, a, base, rows0, slot, dup, i, k, in, has_in, d, bsz, src,
                                   dst);
              if (res & kLaneDigest) reinterpret_cast<uint8_t*>(dg)[slot] = (uint8_t)d;
            }
            uint64_t task = 0;
            uint8_t wrote = kNoSlot;
            if (dst) {
              const uint32_t sl = (uint32_t)slot;
              const uint32_t bit = 1u << (sl & 31), wq = sl >> 5;
              const uint32_t cur = wq == 0 ? wr0 : wq == 1 ? wr1 : wq == 2 ? wr2 : wr3;
              // Latest earlier step of this bucket that wrote the row of `slot`.
              uint32_t prev = kNone;
              if (cur & bit)
                for (uint32_t x = 0; x < step; x++)
                  if (s_slot[o + x] == (uint8_t)sl) prev = x;
              if (res & kLaneRead) {
                // A hit: read the row, or the input of the key that wrote it.
                task = prev != kNone ? (kTaskFwd | s_idx[o + prev])
                                     : (kTaskOut | (src & kTaskMask));
              } else {
                // The row is written: a later write of the same row supersedes.
                if (prev != kNone) {
                  trow[s_idx[o + prev]] = 0;
                  s_slot[o + prev] = kNoSlot;
                }
                task = kTaskIn | (dst & kTaskMask);
                wrote = (uint8_t)sl;
                wr0 |= wq == 0 ? bit : 0u;
                wr1 |= wq == 1 ? bit : 0u;
                wr2 |= wq == 2 ? bit : 0u;
                wr3 |= wq == 3 ? bit : 0u;
              }
            }
            s_slot[o + step] = wrote;
            if (task) trow[i] = task;
          }
        }
      } else {
        uint32_t maxc = lane_ok ? c : 0;
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) {
          const uint32_t y = __shfl_xor(maxc, d, 64);
          maxc = y > maxc ? y : maxc;
        }
        bool active = lane_ok;
        for (uint32_t step = 0; step < maxc; step++) {
          uint64_t src = 0, dst = 0;
          if (active && step < c) {
            const uint64_t k = s_key[o + step];
            const uint64_t i = s_idx[o + step];
            const uint64_t in = has_in ? G(a.in_scores)[i] : 0;
            int slot = -1;
            if (!lane_step<OP>(t, a, b, base, i, k, in, has_in, bsz, src, dst, slot)) {
              active = false;
              s_defer[atomicAdd(&s_ndefer, 1u)] = (bk << 16) | step;
            }
          }
          // Accumulations run in batch order: each step's tasks are executed
          // before the next step reads rows.
          const uint64_t tm = __ballot(dst != 0);
          if (dst) {
            const uint32_t r = __popcll(tm & ((1ull << lane) - 1));
            s_src[wv][r] = src;
            s_dst[wv][r] = dst;
          }
          __builtin_amdgcn_wave_barrier();
          if (tm) flush_tasks<U, 2>(__popcll(tm), s_src[wv], s_dst[wv], R, a.value_type);
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
          __builtin_amdgcn_wave_barrier();
        }
      }
      if (lane_ok && bsz != bsz0) G(t.bsize)[b] = bsz;
      added += (uint32_t)(bsz - bsz0);
      __syncthreads();

      // 16-lane pass over the buckets handed over: 16 groups per block.
      const uint32_t nd = s_ndefer;
      const uint32_t gl = tid & 15;
      for (uint32_t q = tid >> 4; q < nd; q += kBlock / 16) {
        const uint32_t v = s_defer[q];
        const uint32_t l2 = v >> 16, st = v & 0xFFFFu;
        const uint32_t c2 = s_cnt[l2], o2 = s_off[l2];
        const uint64_t b2 = part_b0 + l2;
        if constexpr (kDeferRows) {
          // Row tasks the lane pass recorded for this bucket, in batch order.
          for (uint32_t x = 0; x < st; x++) {
            const uint64_t i = s_idx[o2 + x];
            const uint64_t tv = trow[i];
            if (tv == 0) continue;
            const uint64_t kind = tv & ~kTaskMask, val = tv & kTaskMask;
            gptr<const uint8_t> src;
            gptr<uint8_t> dst;
            if (kind == kTaskIn) {
              src = G(a.in_values) + i * (uint64_t)R;
              dst = G<uint8_t>((uintptr_t)val);
            } else if (kind == kTaskOut) {
              src = G<const uint8_t>((uintptr_t)val);
              dst = G(a.io_values) + i * (uint64_t)R;
            } else {
              src = G(a.io_values) + val * (uint64_t)R;
              dst = G(a.io_values) + i * (uint64_t)R;
            }
            copy_units<U>(dst, src, R, gl, 16);
            if (gl == 0) trow[i] = 0;
          }
        }
        Bucket16 S;
        bucket_load(t, S, b2, gl);
        if (c2 <= kLaneMax) {
          for (uint32_t step = st; step < c2; step++)
            apply_key<OP, U>(t, S, a, s_idx[o2 + step], s_key[o2 + step]);
        } else {
          // Long run, not sorted: take the entries by increasing batch index.
          uint32_t last = 0;  // batch index + 1 of the previous key
          for (uint32_t step = 0; step < c2; step++) {
            uint32_t mi = kNone, mp = 0;
            for (uint32_t x = gl; x < c2; x += 16) {
              const uint32_t iv = s_idx[o2 + x] + 1u;
              if (iv > last && iv < mi) {
                mi = iv;
                mp = x;
              }
            }
#pragma unroll
            for (int d = 8; d > 0; d >>= 1) {
              const uint32_t om = __shfl_xor(mi, d, 16);
              const uint32_t op = __shfl_xor(mp, d, 16);
              if (om < mi) {
                mi = om;
                mp = op;
              }
            }
            last = mi;
            apply_key<OP, U>(t, S, a, (uint64_t)(mi - 1), s_key[o2 + mp]);
          }
        }
        bucket_finish(t, S);
      }
      __syncthreads();
      if (kDeferRows) {
        // The row tasks of this run, executed before another run can touch
        // the same slots.
        for (uint32_t e0 = 0; e0 < mc; e0 += kBlock) {
          const uint32_t e = e0 + tid;
          wave_run_tasks<U>(a, trow, e < mc ? s_idx[e] : 0, e < mc, R, s_rows[wv]);
        }
        __syncthreads();
      }
      c0 = c1;
    }
    __syncthreads();  // LDS is reused by the next partition
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) added += __shfl_xor(added, d, 64);
  if (lane == 0 && added) atomicAdd(t.live, (unsigned long long)added);
}

/* ------------------------------------------------------------------------ */
/* insert_and_evict record compaction                                        */
/* ------------------------------------------------------------------------ */

// The partition pipeline writes the eviction record of batch key i at
// position i of the caller's output arrays (which hold n records) and flags
// bit i, instead of appending at an atomically incremented counter (one
// atomic per record on one address serialises the whole eviction path).
// These kernels then produce the reference's compact output: with c records
// in all, the k-th record at a position >= c moves into the k-th hole below
// c (sources and destinations are disjoint, so every move runs in
// parallel), and the counter gets c.  The flags stay set until the next
// call's k_pcount clears those of its own batch.
/* ------------------------------------------------------------------------ */
/* big partitions of batches with repeated keys                              */
/* ------------------------------------------------------------------------ */
//
// A partition that receives more than kBigPart entries of a batch with
// repeated keys (Zipf traffic, where one key can occur tens of thousands of
// times) would leave one block of k_apply_part streaming all of its entries
// three times: entries per bucket (H0), the heavy-bucket fold (H1) and the
// per-occurrence row work (H3).  k_apply_fast lists such partitions in
// big slots, and these passes run over the whole GPU instead, with each
// partition's counts and key map in its slot in global memory (the block
// of k_apply_fast that lists a partition resets its slot):
//   k_big_count  adds up entries per bucket;
//   k_big_fold   folds the heavy buckets' entries into the key map (first
//                and last batch index and score sum per key: associative,
//                so the order in which blocks fold does not matter) and
//                lists the other entries;
//   k_apply_part loads the counts and the map, places the heavy buckets'
//                keys (H2) and applies the listed entries in its run loop;
//   k_big_tasks  does H3's work: per-occurrence row tasks (find_or_insert)
//                or the last occurrence's row copy.
// If the map overflows, a heavy bucket cannot be folded (H2 leaves it to the
// serial walk) or the other entries exceed one LDS run, k_apply_part
// finishes the partition with its own H3 and run loop, and k_big_tasks
// skips it.

constexpr uint32_t kBigTile = kBlock * kHvPer;  // entries per tile of the grid-wide passes
static_assert(kBigMapCap == kMapCap && kBigLight == kPartLds && kBigMax == kBlock,
              "big-partition slot layout");

// Tiles of the listed big partitions: s_pre[s] = tiles of slots before s
// (s_pre[nb] = all of them).  Every thread of the block calls this.
__device__ __forceinline__ uint32_t big_tiles(const PartScratch& ps, uint32_t* s_pre,
                                              uint32_t* s_wsum, uint32_t* nb_out) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t nb = *(volatile uint32_t*)&ps.dctr[4];
  nb = nb < kBigMax ? nb : kBigMax;
  uint32_t c = 0;
  if (tid < nb) c = (ps.pinfo[2 * ps.big_part[tid] + 1] + kBigTile - 1) / kBigTile;
  uint32_t x = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(x, d, 64);
    if (lane >= (uint32_t)d) x += y;
  }
  if (lane == 63) s_wsum[wv] = x;
  __syncthreads();
  uint32_t pre = 0;
  for (uint32_t q = 0; q < wv; q++) pre += s_wsum[q];
  s_pre[tid + 1] = pre + x;
  if (tid == 0) s_pre[0] = 0;
  __syncthreads();
  *nb_out = nb;
  return s_pre[nb];
}

// Slot of tile v: the last s with s_pre[s] <= v.
__device__ __forceinline__ uint32_t big_slot_of(const uint32_t* s_pre, uint32_t nb, uint32_t v) {
  uint32_t lo = 0, hi = nb;  // s_pre[lo] <= v < s_pre[hi]
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (s_pre[mid] <= v) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Resets one slot of big-partition state (all kBlock threads of a block).
__device__ __forceinline__ void big_slot_reset(BigSlot& S, uint32_t tid) {
  S.tot[tid] = 0;
  for (uint32_t q = tid; q < kBigMapCap; q += kBlock) {
    S.mkey[q] = kEmptyKey;
    S.msum[q] = 0;
    S.mfirst[q] = kNone;
    S.mlast[q] = 0;
  }
  if (tid == 0) {
    S.mfull = 0;
    S.nlight = 0;
    S.fast = 0;
  }
}

__global__ __launch_bounds__(kBlock) void k_big_count(TableView t, PartScratch ps) {
  __shared__ uint32_t s_pre[kBigMax + 1], s_wsum[kBlock / 64], s_cnt[kPartBuckets];
  const uint32_t tid = threadIdx.x;
  uint32_t nb;
  const uint32_t total = big_tiles(ps, s_pre, s_wsum, &nb);
  gptr<const u64x2> ent = G(reinterpret_cast<const u64x2*>(ps.ent));
  for (uint32_t v = blockIdx.x; v < total; v += gridDim.x) {
    const uint32_t sl = big_slot_of(s_pre, nb, v);
    const uint32_t p = ps.big_part[sl];
    const uint32_t base_e = ps.pinfo[2 * p], m = ps.pinfo[2 * p + 1];
    const uint32_t e0 = (v - s_pre[sl]) * kBigTile;
    uint64_t kq[kHvPer];
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const uint32_t e = e0 + tid + r * kBlock;
      kq[r] = e < m ? ent[base_e + e].x : kEmptyKey;
    }
    s_cnt[tid] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++)
      if (e0 + tid + r * kBlock < m) atomicAdd(&s_cnt[bucket_of(t, kq[r]) % kPartBuckets], 1u);
    __syncthreads();
    if (s_cnt[tid]) atomicAdd(&ps.big[sl].tot[tid], s_cnt[tid]);
    __syncthreads();
  }
}

template <int OP>
__global__ __launch_bounds__(kBlock) void k_big_fold(TableView t, ApplyArgs a, PartScratch ps) {
  __shared__ uint32_t s_pre[kBigMax + 1], s_wsum[kBlock / 64], s_tot[kPartBuckets];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  uint32_t nb;
  const uint32_t total = big_tiles(ps, s_pre, s_wsum, &nb);
  gptr<const u64x2> ent = G(reinterpret_cast<const u64x2*>(ps.ent));
  const bool has_in = a.in_scores != nullptr;
  const bool sum_in = a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu;
  for (uint32_t v = blockIdx.x; v < total; v += gridDim.x) {
    const uint32_t sl = big_slot_of(s_pre, nb, v);
    BigSlot& S = ps.big[sl];
    const uint32_t p = ps.big_part[sl];
    const uint32_t base_e = ps.pinfo[2 * p], m = ps.pinfo[2 * p + 1];
    const uint32_t e0 = (v - s_pre[sl]) * kBigTile;
    u64x2 eq[kHvPer];
    uint64_t hq_[kHvPer], cq[kHvPer];
    bool hvq[kHvPer], ltq[kHvPer];
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const uint32_t e = e0 + tid + r * kBlock;
      eq[r].x = kEmptyKey;
      eq[r].y = 0;
      if (e < m) eq[r] = ent[base_e + e];
    }
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      cq[r] = 0;
      if (sum_in && has_in && e0 + tid + r * kBlock < m) cq[r] = G(a.in_scores)[eq[r].y];
    }
    s_tot[tid] = S.tot[tid];
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const bool valid = e0 + tid + r * kBlock < m;
      hq_[r] = murmur3(eq[r].x);
      const uint32_t bk = (uint32_t)((global_idx(t, hq_[r]) >> t.bshift) % kPartBuckets);
      hvq[r] = valid && s_tot[bk] > kHeavyMin;
      ltq[r] = valid && !hvq[r];
      const uint64_t in = cq[r];
      cq[r] = !hvq[r] ? 0 : a.sc.strategy == kLfu ? in : (in & kScoreMask);
    }
    // Other buckets' entries: listed, one atomic per wave and sub-tile.
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const uint64_t lm = __ballot(ltq[r]);
      if (lm) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&S.nlight, (uint32_t)__popcll(lm));
        base = __shfl(base, 0, 64);
        const uint32_t pos = base + (uint32_t)__popcll(lm & ((1ull << lane) - 1));
        if (ltq[r] && pos < kBigLight) {
          S.light[2 * pos] = eq[r].x;
          S.light[2 * pos + 1] = eq[r].y;
        }
      }
    }
    // Heavy entries: the wave's leading key folded over the tile with one
    // reduction, then the map updated once for it and once per other entry.
    uint64_t lk = 0;
    bool have_lead = false;
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const uint64_t act = __ballot(hvq[r]);
      if (act && !have_lead) {
        lk = shfl_u64(eq[r].x, __ffsll((unsigned long long)act) - 1, 64);
        have_lead = true;
      }
    }
    uint32_t l1 = kNone, l2 = 0;
    uint64_t l3 = 0;
    if (have_lead) {
#pragma unroll
      for (uint32_t r = 0; r < kHvPer; r++) {
        if (hvq[r] && eq[r].x == lk) {
          const uint32_t i = (uint32_t)eq[r].y;
          l1 = i < l1 ? i : l1;
          l2 = i > l2 ? i : l2;
          l3 += cq[r];
          hvq[r] = false;
        }
      }
#pragma unroll
      for (int d = 32; d > 0; d >>= 1) {
        const uint32_t o1 = __shfl_xor(l1, d, 64), o2 = __shfl_xor(l2, d, 64);
        l1 = o1 < l1 ? o1 : l1;
        l2 = o2 > l2 ? o2 : l2;
        l3 += shfl_xor_u64(l3, d, 64);
      }
    }
#pragma unroll
    for (uint32_t r = 0; r <= kHvPer; r++) {
      bool mine;
      uint64_t k, h, csum;
      uint32_t fmin, fmax;
      if (r == kHvPer) {
        mine = have_lead && lane == 0;
        k = lk;
        h = murmur3(lk);
        fmin = l1;
        fmax = l2;
        csum = l3;
      } else {
        mine = hvq[r];
        k = eq[r].x;
        h = hq_[r];
        fmin = fmax = (uint32_t)eq[r].y;
        csum = cq[r];
      }
      if (mine) {
        uint32_t q = map_home(h);
        bool ok = false;
        for (uint32_t pr = 0; pr < kMapProbe; pr++) {
          const uint64_t cur = atomicCAS(reinterpret_cast<unsigned long long*>(&S.mkey[q]),
                                         (unsigned long long)kEmptyKey, (unsigned long long)k);
          if (cur == kEmptyKey || cur == k) {
            ok = true;
            break;
          }
          q = (q + 1) & (kBigMapCap - 1);
        }
        if (!ok) {
          atomicOr(&S.mfull, 1u);
        } else {
          atomicMin(&S.mfirst[q], fmin);
          atomicMax(&S.mlast[q], fmax);
          if (csum) atomicAdd(reinterpret_cast<unsigned long long*>(&S.msum[q]),
                              (unsigned long long)csum);
        }
      }
    }
    __syncthreads();  // s_tot of the next tile
  }
}

template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_big_tasks(TableView t, ApplyArgs a, PartScratch ps) {
  __shared__ uint32_t s_pre[kBigMax + 1], s_wsum[kBlock / 64], s_tot[kPartBuckets];
  __shared__ uint32_t s_rows[kBlock / 64][64];
  const uint32_t tid = threadIdx.x, wv = tid >> 6;
  uint32_t nb;
  const uint32_t total = big_tiles(ps, s_pre, s_wsum, &nb);
  gptr<const u64x2> ent = G(reinterpret_cast<const u64x2*>(ps.ent));
  gptr<uint64_t> trow = G(ps.trow);
  const uint32_t R = t.row_bytes;
  for (uint32_t v = blockIdx.x; v < total; v += gridDim.x) {
    const uint32_t sl = big_slot_of(s_pre, nb, v);
    const BigSlot& S = ps.big[sl];
    if (!*(volatile const uint32_t*)&S.fast) continue;  // block-uniform
    const uint32_t p = ps.big_part[sl];
    const uint32_t base_e = ps.pinfo[2 * p], m = ps.pinfo[2 * p + 1];
    const uint64_t part_b0 = (uint64_t)p * kPartBuckets;
    const uint32_t e0 = (v - s_pre[sl]) * kBigTile;
    u64x2 eq[kHvPer];
    uint64_t srcq[kHvPer], dstq[kHvPer];
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const uint32_t e = e0 + tid + r * kBlock;
      eq[r].x = kEmptyKey;
      eq[r].y = 0;
      if (e < m) eq[r] = ent[base_e + e];
    }
    s_tot[tid] = S.tot[tid];
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < kHvPer; r++) {
      const uint64_t k = eq[r].x, i = eq[r].y;
      const uint64_t h = murmur3(k);
      const uint64_t gb = global_idx(t, h) >> t.bshift;
      const uint32_t bk = (uint32_t)(gb % kPartBuckets);
      srcq[r] = dstq[r] = 0;
      // In a slot left to this kernel every heavy bucket was folded.
      if (e0 + tid + r * kBlock < m && s_tot[bk] > kHeavyMin) {
        uint32_t q = map_home(h);
        uint32_t pr = 0;
        while (S.mkey[q] != k && pr < kBigMapCap) {  // present: folded
          q = (q + 1) & (kBigMapCap - 1);
          pr++;
        }
        if (S.mkey[q] != k) continue;
        const uint32_t rs = S.mres[q];
        const uint64_t trow_a = (uint64_t)(uintptr_t)row_ptr(t, part_b0 + bk, rs & (t.B - 1));
        if (OP == OP_FIND_OR_INSERT) {
          const uint32_t first = S.mfirst[q];
          trow[i] = !(rs & kMapNew) ? (kTaskOut | trow_a)
                    : i == first ? (kTaskIn | trow_a)
                                 : (kTaskFwd | (uint64_t)first);
        } else if (i == S.mlast[q]) {
          srcq[r] = (uint64_t)(uintptr_t)(a.in_values + i * R);
          dstq[r] = trow_a;
        }
      }
    }
    wave_copy_tasks<U, kHvPer>(srcq, dstq, R, s_rows[wv]);
    __syncthreads();  // s_tot of the next tile
  }
}

constexpr uint32_t kEvBlkWords = 256;  // bitmap words per block of the count kernel

__device__ __forceinline__ uint32_t block_excl_scan256(uint32_t v, uint32_t* s_w,
                                                        uint32_t* total) {
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(x, d, 64);
    if (lane >= (uint32_t)d) x += y;
  }
  if (lane == 63) s_w[wv] = x;
  __syncthreads();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (uint32_t q = 0; q < kBlock / 64; q++) {
    pre += q < wv ? s_w[q] : 0u;
    tot += s_w[q];
  }
  __syncthreads();
  *total = tot;
  return pre + x - v;
}

// Set bits before each word within its block, and each block's total.
__global__ __launch_bounds__(kBlock) void k_evc_count(const uint32_t* __restrict__ bits,
                                                      uint32_t nw, uint32_t* __restrict__ wpre,
                                                      uint32_t* __restrict__ blk) {
  __shared__ uint32_t s_w[kBlock / 64];
  const uint32_t w = blockIdx.x * kEvBlkWords + threadIdx.x;
  const uint32_t c = w < nw ? (uint32_t)__popc(bits[w]) : 0u;
  uint32_t tot;
  const uint32_t ex = block_excl_scan256(c, s_w, &tot);
  if (w < nw) wpre[w] = ex;
  if (threadIdx.x == 0) blk[blockIdx.x] = tot;
}

__device__ __forceinline__ uint32_t ev_bits_before_word(const uint32_t* blk, const uint32_t* wpre,
                                                        uint32_t w) {
  return blk[w / kEvBlkWords] + wpre[w];
}

// One block: exclusive scan of the block totals; then blk[nb] = c, the
// record count, and blk[nb + 1] = the records at positions below c; the
// caller's counter gets c.
__global__ __launch_bounds__(kBlock) void k_evc_scan(uint32_t* __restrict__ blk, uint32_t nb,
                                                     const uint32_t* __restrict__ bits,
                                                     const uint32_t* __restrict__ wpre,
                                                     uint32_t nw, uint64_t* counter) {
  __shared__ uint32_t s_w[kBlock / 64];
  uint32_t carry = 0;
  for (uint32_t b0 = 0; b0 < nb; b0 += kBlock) {
    const uint32_t b = b0 + threadIdx.x;
    const uint32_t v = b < nb ? blk[b] : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan256(v, s_w, &tot);
    if (b < nb) blk[b] = carry + ex;
    carry += tot;
  }
  __syncthreads();  // the scanned offsets are read below
  if (threadIdx.x == 0) {
    const uint32_t c = carry;
    const uint32_t w = c / 32;
    const uint32_t below =
        w < nw ? ev_bits_before_word(blk, wpre, w) + (uint32_t)__popc(bits[w] & ((1u << (c & 31)) - 1u))
               : c;
    blk[nb] = c;
    blk[nb + 1] = below;
    atomicAdd(reinterpret_cast<unsigned long long*>(counter), (unsigned long long)c);
  }
}

// Moves every record at a position >= c into a hole below c.
template <int U>
__global__ __launch_bounds__(kBlock) void k_evc_move(const uint32_t* __restrict__ bits,
                                                     uint32_t nw,
                                                     const uint32_t* __restrict__ wpre,
                                                     const uint32_t* __restrict__ blk, uint32_t nb,
                                                     uint64_t n, uint64_t* keys, uint8_t* vals,
                                                     uint64_t* scores, uint32_t row_bytes) {
  __shared__ uint32_t s_rows[kBlock / 64][64];
  const uint32_t wv = threadIdx.x >> 6;
  const uint32_t c = blk[nb], below = blk[nb + 1];
  for (uint64_t i0 = (uint64_t)blockIdx.x * kBlock; i0 < n; i0 += (uint64_t)gridDim.x * kBlock) {
    const uint64_t i = i0 + threadIdx.x;
    uint64_t src = 0, dst = 0;
    if (i < n && i >= c) {
      const uint32_t w = (uint32_t)(i >> 5), word = bits[w];
      if ((word >> (i & 31)) & 1u) {
        // rank among the records at positions >= c = rank of its hole
        const uint32_t r = ev_bits_before_word(blk, wpre, w) +
                           (uint32_t)__popc(word & ((1u << (i & 31)) - 1u)) - below;
        // last word x <= (c - 1) / 32 with (holes before x) <= r
        uint32_t lo = 0, hi = (c - 1) / 32;
        while (lo < hi) {
          const uint32_t mid = (lo + hi + 1) / 2;
          if (32 * mid - ev_bits_before_word(blk, wpre, mid) <= r) lo = mid;
          else hi = mid - 1;
        }
        uint32_t inv = ~bits[lo];
        for (uint32_t k = r - (32 * lo - ev_bits_before_word(blk, wpre, lo)); k > 0; k--)
          inv &= inv - 1;
        const uint64_t h = 32ull * lo + (uint32_t)(__ffs(inv) - 1);
        keys[h] = keys[i];
        if (scores) scores[h] = scores[i];
        src = (uint64_t)(uintptr_t)(vals + i * row_bytes);
        dst = (uint64_t)(uintptr_t)(vals + h * row_bytes);
      }
    }
    wave_copy_pairs<U>(src, dst, row_bytes, s_rows[wv]);
  }
}

// Executes the row tasks k_apply_part left in the task words (the
// find_or_insert copies of folded heavy buckets; zero elsewhere), over the
// whole GPU, and clears them.  The tasks of one call are independent: they
// read input rows, present keys' table rows or rows no task writes.
template <int U>
__global__ __launch_bounds__(kBlock) void k_rowtasks(TableView t, ApplyArgs a, PartScratch ps) {
  __shared__ uint32_t s_rows[kBlock / 64][64];
  const uint32_t wv = threadIdx.x >> 6;
  gptr<uint64_t> trow = G(ps.trow);
  for (uint64_t i0 = (uint64_t)blockIdx.x * kBlock; i0 < a.n; i0 += (uint64_t)gridDim.x * kBlock) {
    const uint64_t i = i0 + threadIdx.x;
    wave_run_tasks<U>(a, trow, i < a.n ? i : 0, i < a.n, t.row_bytes, s_rows[wv]);
  }
}

// Single-run apply of a partition whose entries fit one LDS load (kFastLds)
// and whose buckets receive at most kLaneMax keys each (every partition, for
// uniform keys); other partitions are listed for k_apply_part.
//
// The batch-order semantics (keys applied one at a time in increasing batch
// index, each by the reference's per-key algorithm) are reproduced with the
// keys processed in parallel, one thread per key:
//  B. every key probes the table as it was before the call, over the two
//     16-slot digest chunks from its start group: the key is present at a
//     slot, or absent with a first EMPTY slot, or undecided;
//  C. per bucket, the first key in batch order whose outcome could depend on
//     earlier keys of the call: the same key met again, two absent keys with
//     the same first EMPTY slot, an absent key that would find the bucket
//     full, or an undecided probe.  Up to that key the parallel outcomes are
//     the sequential ones: a probe ends at its first EMPTY slot, so an
//     earlier key's new slot lies on a later key's probe only when both are
//     that slot;
//  S. the rest of such a bucket, by one lane in batch order, probing the
//     digests in memory and the call's own insertions in LDS.  At a key that
//     needs the eviction path the lane hands the rest of the bucket to
//     k_apply_deferred;
//  W. the metadata of every applied key (one record per slot), then the
//     block copies the rows of all its tasks.
// No global store precedes the last global load of a phase that waits on it
// (gfx9 counts loads and stores on one in-order counter, so a load issued
// after stores would wait for them).
constexpr uint32_t kFastLds = 704;  // entries of a partition the fast pass takes

// Per-entry flags of the fast pass: the metadata record (bits 0-1), the row
// task (bits 2-3) and the outcome on the table before the call (bits 4-5).
constexpr uint8_t kMetaKey = 1;     // new key: key and score written at the slot
constexpr uint8_t kMetaScore = 2;   // present key: score written
constexpr uint8_t kMetaMask = 3;
constexpr uint32_t kSerialKeys = 4;     // keys one serial lane of k_apply_fast applies ...
constexpr uint32_t kSerialCapFrom = 40;  // ... when its block has more serial buckets,
constexpr uint32_t kSerialLong = 6;      // or (find_or_insert, whose duplicate-heavy
                                         // batches make long lanes) its bucket has more
                                         // keys left
constexpr uint8_t kTkIn = 1 << 2;   // input row -> table row
constexpr uint8_t kTkOut = 2 << 2;  // table row -> output row
constexpr uint8_t kTkAcc = kTkOut;  // accum_or_assign: input delta added into the table row
constexpr uint8_t kTkFwd = 3 << 2;  // input row of the earlier key that wrote the slot -> output row
constexpr uint8_t kTkMask = 3 << 2;
constexpr uint8_t kResNew = 1 << 4;   // absent; the slot is the probe's first EMPTY slot
constexpr uint8_t kResDup = 2 << 4;   // present at the slot
constexpr uint8_t kResSlow = 3 << 4;  // undecided by the window (or needs the serial lane)
constexpr uint8_t kResMask = 3 << 4;
constexpr uint8_t kRepeat = 1 << 6;  // a later occurrence of a key met earlier in its bucket
constexpr uint8_t kRest = 1 << 7;    // the window held neither the key nor an EMPTY slot (step B2)

__device__ __forceinline__ uint32_t sel4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                         uint32_t q) {
  return q == 0 ? w0 : q == 1 ? w1 : q == 2 ? w2 : w3;
}

// Probe of one key in the order of find_without_lock /
// insert_or_assign_kernel.h:105-183: 4-slot groups from start's group,
// circularly; in each group first the digest matches, then the EMPTY slots
// (in the first group only at or after start).  The first two digest matches
// met before the probe ends are recorded: their keys decide whether the key
// is present.  A probe the window does not decide goes to the serial lane.
// After the first EMPTY slot the scan records the next EMPTY slots of the
// window: a key absent before the call ends its probe at the first of them
// that no earlier key of the call has taken (digest matches past the first
// EMPTY slot belong to other keys, since a key always sits before the first
// EMPTY slot of its probe).
constexpr uint32_t kMoreEmpty = 1;  // EMPTY slots recorded after the first

struct WinProbe {
  uint32_t slot;                // first EMPTY slot of the probe (when found)
  uint32_t c0, c1;              // first two digest matches (kNone: none)
  uint32_t more[kMoreEmpty];    // the next EMPTY slots in probe order (kNone: none)
  uint32_t nmore;
  bool found;                   // the probe reached an EMPTY slot
  bool over;                    // more than two digest matches
};

// One group (digests w, first slot gs) of a probe.
__device__ __forceinline__ void probe_group(WinProbe& r, uint32_t w, uint32_t gs, uint32_t rep,
                                            uint32_t emask) {
  uint32_t m = eq_bytes4(w, rep);
  uint32_t e = eq_bytes4(w, (uint32_t)kEmptyDigest * 0x01010101u) & emask;
  if (!r.found) {
    while (m) {
      const uint32_t p = gs + __builtin_ctz(m);
      m &= m - 1;
      if (r.c0 == kNone) r.c0 = p;
      else if (r.c1 == kNone) r.c1 = p;
      else r.over = true;
    }
    if (!e) return;
    r.found = true;
    r.slot = gs + __builtin_ctz(e);
    e &= e - 1;
  }
  while (e && r.nmore < kMoreEmpty) {
    const uint32_t p = gs + __builtin_ctz(e);
    e &= e - 1;
#pragma unroll
    for (uint32_t j = 0; j < kMoreEmpty; j++)
      if (j == r.nmore) r.more[j] = p;
    r.nmore++;
  }
}

// The probe over its first two 16-slot digest chunks: w0 (the chunk of
// start's group) and w1 (the next one, circularly).  `empties` = false scans
// for the key only (a full bucket).
__device__ __forceinline__ WinProbe probe_window(u32x4 w0, u32x4 w1, uint32_t start, uint32_t d,
                                                 uint32_t B, bool empties) {
  const uint32_t a = start & ~3u;
  const uint32_t cbase = a & ~15u;    // first slot of chunk w0
  const uint32_t g0 = (a >> 2) & 3u;  // start's group inside w0
  const uint32_t rep = d * 0x01010101u;
  const uint32_t emask = empties ? 0xFu : 0u;
  const uint32_t first_mask = ~((1u << (start - a)) - 1u) & emask;
  const uint32_t words[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  WinProbe r{0, kNone, kNone, {kNone}, 0, false, false};
#pragma unroll
  for (uint32_t q = 0; q < 8; q++) {
    if (q < g0 || r.nmore == kMoreEmpty) continue;
    probe_group(r, words[q], (cbase + 4 * q) & (B - 1), rep, q == g0 ? first_mask : emask);
  }
  return r;
}

// Probe of key k for the serial lane, over the bucket's digests in memory.
// Slots filled by the call's earlier keys (bit set in f0..f3) still show the
// empty digest in memory and are skipped: the caller has already looked for
// k among the keys those earlier keys placed (its scan of the bucket's
// earlier entries), so only slots placed before the call can hold k here.
// Returns the slot holding k (*dup = 1), else the first EMPTY slot when
// `empties` (*dup = 0), else -1.  Digests load 32 slots (two 16-byte
// chunks, in probe order) per memory round trip.
__device__ __forceinline__ int probe_serial(const TableView& t, uint64_t base, uint32_t f0,
                                            uint32_t f1, uint32_t f2, uint32_t f3,
                                            uint32_t start, uint32_t d, uint64_t k, bool empties,
                                            int* dup) {
  const uint32_t B = t.B;
  const uint32_t nch = B / 16;
  gptr<const u32x4> drow = (gptr<const u32x4>)(G(t.digests) + base);
  const uint32_t a = start & ~3u;
  const uint32_t rep = d * 0x01010101u;
  const uint32_t erep = (uint32_t)kEmptyDigest * 0x01010101u;
  uint32_t cur = kNone;  // chunk held in c0; c1 holds the next one
  u32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t ch = g >> 4;
    if (cur == kNone || (ch != cur && ch != ((cur + 1) & (nch - 1)))) {
      cur = ch;
      c0 = drow[ch];
      c1 = drow[(ch + 1) & (nch - 1)];
    }
    const u32x4 chunk = ch == cur ? c0 : c1;
    const uint32_t wi = (g >> 2) & 3;
    const uint32_t w = wi == 0 ? chunk.x : wi == 1 ? chunk.y : wi == 2 ? chunk.z : chunk.w;
    const uint32_t fm = (sel4(f0, f1, f2, f3, g >> 5) >> (g & 31)) & 0xFu;
    uint32_t m = eq_bytes4(w, rep) & ~fm;
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      if (slot_key(t, base + g + j) == k) {
        *dup = 1;
        return (int)(g + j);
      }
    }
    if (!empties) continue;
    uint32_t em = eq_bytes4(w, erep) & ~fm;
    if (off == 0) em &= ~((1u << (start - a)) - 1u);
    if (em) {
      *dup = 0;
      return (int)(g + __builtin_ctz(em));
    }
  }
  return -1;
}

// Element-wise dst += src over one U-byte unit, for the value types
// accum_or_assign supports (f32, i32, i64/u64), in the reference's order
// (`val = delta; val += dst`, accum_or_assign_kernel.h:41-49).
template <typename T>
__device__ __forceinline__ T add_unit(T row, T delta, int vt) {
  constexpr int W = sizeof(T) / 4;  // 32-bit words in the unit (>= 1)
  uint32_t r[W > 0 ? W : 1], d[W > 0 ? W : 1];
  __builtin_memcpy(r, &row, sizeof(T));
  __builtin_memcpy(d, &delta, sizeof(T));
  if (vt == 0) {  // f32
#pragma unroll
    for (int j = 0; j < W; j++) {
      float v = __uint_as_float(d[j]);
      v += __uint_as_float(r[j]);
      r[j] = __float_as_uint(v);
    }
  } else if (vt == 8) {  // i32
#pragma unroll
    for (int j = 0; j < W; j++) r[j] = (uint32_t)((int32_t)d[j] + (int32_t)r[j]);
  } else {  // i64 / u64
#pragma unroll
    for (int j = 0; j + 1 < W; j += 2) {
      const uint64_t v = (((uint64_t)d[j + 1] << 32) | d[j]) + (((uint64_t)r[j + 1] << 32) | r[j]);
      r[j] = (uint32_t)v;
      r[j + 1] = (uint32_t)(v >> 32);
    }
  }
  T out;
  __builtin_memcpy(&out, r, sizeof(T));
  return out;
}

// Wave-cooperative accumulation: the lane with dst != 0 has its row of
// deltas (src) added into the table row dst; lpr lanes per row, one unit each.
// Different lanes name different table rows.
template <int U>
__device__ __forceinline__ void wave_accum_pairs(uint64_t src, uint64_t dst, uint32_t row_bytes,
                                                 int vt, uint32_t* s_rows) {
  using T = typename UnitT<U>::T;
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t hm = __ballot(dst != 0);
  if (!hm) return;
  if (dst) s_rows[__popcll(hm & ((1ull << lane) - 1))] = lane;
  __builtin_amdgcn_wave_barrier();
  const uint32_t rows = __popcll(hm);
  const uint32_t units = row_bytes / U;
  uint32_t lpr = 64;
  while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;
  const uint32_t rpi = 64 / lpr, sub = lane % lpr;
  for (uint32_t r0 = 0; r0 < rows; r0 += rpi) {
    const uint32_t r = r0 + lane / lpr;
    const uint32_t l = s_rows[r < rows ? r : 0];
    gptr<const T> sp = G<const T>((uintptr_t)shfl_u64(src, (int)l, 64));
    gptr<T> dp = G<T>((uintptr_t)shfl_u64(dst, (int)l, 64));
    if (r < rows)
      for (uint32_t u = sub; u < units; u += lpr) dp[u] = add_unit<T>(dp[u], sp[u], vt);
  }
  __builtin_amdgcn_wave_barrier();
}

// Does entry e carry a record or (pointer find_or_insert) a slot word?
template <int OP>
__device__ __forceinline__ bool emits_meta(uint8_t fl) {
  if (fl & kMetaMask) return true;
  const uint32_t res = fl & kResMask;
  return OP == OP_FIND_OR_INSERT_PTR && (res == kResNew || res == kResDup);
}

// The metadata record of entry e at global slot s.  The pointer
// find_or_insert also writes every applied key's slot word (slot + 1, found
// flag) and, with unique keys, holds the slot LOCKED for the rest of the
// batch, as the reference does.
template <int OP>
__device__ __forceinline__ void emit_record(const TableView& t, const ApplyArgs& a, uint32_t e,
                                            uint64_t k, uint64_t h, uint64_t s,
                                            const uint32_t* s_idx, const uint64_t* s_sc,
                                            const uint8_t* s_fl) {
  const uint8_t fl = s_fl[e];
  const uint32_t f = fl & kMetaMask;
  const bool lk = OP == OP_FIND_OR_INSERT_PTR && a.lock;
  const bool dup = (fl & kResMask) == kResDup;
  if (f == kMetaKey) {
    slot_store(t, s, lk ? kLockedKey : k, s_sc[e]);
    G(t.digests)[s] = (uint8_t)key_digest(h);
  } else if (f == kMetaScore) {
    if (lk) slot_store(t, s, kLockedKey, s_sc[e]);
    else slot_score(t, s) = s_sc[e];
  } else if (lk && dup) {
    slot_key(t, s) = kLockedKey;
  }
  if (OP == OP_FIND_OR_INSERT_PTR && emits_meta<OP>(fl))
    G(a.slot_out)[s_idx[e]] = (s + 1) | (dup ? kSlotFound : 0ull);
}

// Metadata records (at most one per slot) and row copies of the entries of a
// k_apply_fast block whose bucket's serial flag equals `ser` (2: every
// bucket), by the threads
// t0 .. t0 + nthr - 1 of the block (whole waves; nthr a multiple of 64).
// Tasks of different keys name different rows (a superseded write was
// dropped), except that a forwarded read takes an input row that is only
// read, so they run in any order.
// Source and destination rows of entry e's row task tk (bucket gb) in a
// k_apply_fast block: a copy (src -> dst) or, for accum_or_assign, an
// accumulation (asrc into adst).
template <int OP>
__device__ __forceinline__ void fast_row_task(const TableView& t, const ApplyArgs& a, uint32_t e,
                                              uint64_t gb, uint32_t tk, const uint32_t* s_idx,
                                              const uint8_t* s_slot, const uint8_t* s_fl,
                                              const uint32_t* s_off, uint64_t& src,
                                              uint64_t& dst, uint64_t& asrc, uint64_t& adst) {
  const uint64_t R64 = t.row_bytes;
  const uint64_t i = s_idx[e];
  const uint32_t sl = s_slot[e];
  const uint64_t trow = (uint64_t)(uintptr_t)row_ptr(t, gb, sl);
  if (tk == kTkIn) {
    src = (uint64_t)(uintptr_t)(a.in_values + i * R64);
    dst = trow;
  } else if (tk == kTkOut && OP == OP_ACCUM_OR_ASSIGN) {
    asrc = (uint64_t)(uintptr_t)(a.in_values + i * R64);  // kTkAcc
    adst = trow;
  } else if (tk == kTkOut) {
    src = trow;
    dst = (uint64_t)(uintptr_t)(a.io_values + i * R64);
  } else {
    // The latest earlier key of the bucket whose input row was queued for
    // this slot.
    uint32_t xs = e;
    for (uint32_t x = s_off[gb % kPartBuckets]; x < e; x++)
      if (s_slot[x] == sl && (s_fl[x] & kTkMask) == kTkIn) xs = x;
    src = (uint64_t)(uintptr_t)(a.io_values + (uint64_t)s_idx[xs] * R64);
    dst = (uint64_t)(uintptr_t)(a.io_values + i * R64);
  }
}

// With with_rows false only the metadata records are written.
template <int OP, int U, bool kMovesRows>
__device__ __forceinline__ void emit_fast(const TableView& t, const ApplyArgs& a, uint32_t m,
                                          uint64_t part_b0, uint32_t t0, uint32_t nthr,
                                          uint8_t ser, const uint64_t* s_key,
                                          const uint32_t* s_idx, const uint64_t* s_sc,
                                          const uint8_t* s_slot, const uint8_t* s_fl,
                                          const uint32_t* s_off, const uint32_t* s_cnt,
                                          const uint8_t* s_isser, uint32_t* s_rows,
                                          bool with_rows = true) {
  const uint32_t B = t.B;
  for (uint32_t e = t0; e < m; e += nthr) {
    if (!emits_meta<OP>(s_fl[e])) continue;
    const uint64_t k = s_key[e];
    const uint64_t h = murmur3(k);
    const uint64_t gb = global_idx(t, h) >> t.bshift;
    const uint32_t lbk = (uint32_t)(gb % kPartBuckets);
    if (ser != 2 && s_isser[lbk] != ser) continue;
    if (e - s_off[lbk] >= s_cnt[lbk]) continue;  // left to k_apply_deferred
    emit_record<OP>(t, a, e, k, h, gb * B + s_slot[e], s_idx, s_sc, s_fl);
  }
  if (!kMovesRows || !with_rows) return;
  for (uint32_t e0 = 0; e0 < m; e0 += nthr) {
    const uint32_t e = e0 + t0;
    uint64_t src = 0, dst = 0, asrc = 0, adst = 0;
    uint32_t tk = e < m ? (s_fl[e] & kTkMask) : 0u;
    uint64_t gb = 0;
    if (tk) {
      gb = bucket_of(t, s_key[e]);
      const uint32_t lbk = (uint32_t)(gb % kPartBuckets);
      if ((ser != 2 && s_isser[lbk] != ser) || e - s_off[lbk] >= s_cnt[lbk]) tk = 0;
    }
    if (tk)
      fast_row_task<OP>(t, a, e, gb, tk, s_idx, s_slot, s_fl, s_off, src, dst, asrc, adst);
    wave_copy_pairs_q<U, 4>(src, dst, t.row_bytes, s_rows);
    if (OP == OP_ACCUM_OR_ASSIGN) wave_accum_pairs<U>(asrc, adst, t.row_bytes, a.value_type, s_rows);
  }
}

// emit_fast for the buckets the parallel pass applied whole (serial flag 0),
// by whole waves that take 64-entry chunks from the LDS counter *next (zero
// beforehand): the waves that ran serial lanes join when those are done, so
// every wave of the block copies rows.
template <int OP, int U, bool kMovesRows>
__device__ __forceinline__ void emit_fast_dyn(const TableView& t, const ApplyArgs& a, uint32_t m,
                                              uint64_t part_b0, const uint64_t* s_key,
                                              const uint32_t* s_idx, const uint64_t* s_sc,
                                              const uint8_t* s_slot, const uint8_t* s_fl,
                                              const uint32_t* s_off, const uint32_t* s_cnt,
                                              const uint8_t* s_isser, uint32_t* s_rows,
                                              uint32_t* next) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t B = t.B;
  for (;;) {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(next, 1u);
    c = __shfl(c, 0, 64);
    if (c * 64 >= m) break;  // wave-uniform
    const uint32_t e = c * 64 + lane;
    uint64_t k = 0, h = 0, gb = 0;
    bool f = false;
    uint32_t tk = 0;
    if (e < m) {
      k = s_key[e];
      h = murmur3(k);
      gb = global_idx(t, h) >> t.bshift;
      const uint32_t lbk = (uint32_t)(gb % kPartBuckets);
      if (s_isser[lbk] == 0 && e - s_off[lbk] < s_cnt[lbk]) {
        f = emits_meta<OP>(s_fl[e]);
        tk = s_fl[e] & kTkMask;
      }
    }
    if (kMovesRows) {
      uint64_t src = 0, dst = 0, asrc = 0, adst = 0;
      if (tk)
        fast_row_task<OP>(t, a, e, gb, tk, s_idx, s_slot, s_fl, s_off, src, dst, asrc, adst);
      wave_copy_pairs_q<U, 4>(src, dst, t.row_bytes, s_rows);
      if (OP == OP_ACCUM_OR_ASSIGN) wave_accum_pairs<U>(asrc, adst, t.row_bytes, a.value_type, s_rows);
    }
    if (f) emit_record<OP>(t, a, e, k, h, gb * B + s_slot[e], s_idx, s_sc, s_fl);
  }
}

template <int OP, int U>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_apply_fast(TableView t, ApplyArgs a, PartScratch ps) {
  constexpr uint32_t kPer = (kFastLds + kBlock - 1) / kBlock;  // entries per thread
  // accum_or_assign and the pointer find_or_insert list a partition with a
  // long bucket whole (k_apply_part and k_apply_seq take it).
  constexpr bool kSplitLong = OP != OP_ACCUM_OR_ASSIGN && OP != OP_FIND_OR_INSERT_PTR;
  constexpr bool may_insert = OP != OP_ASSIGN_SCORES;
  constexpr bool moves_rows = OP != OP_ASSIGN_SCORES && OP != OP_FIND_OR_INSERT_PTR;
  constexpr bool reads_rows = OP == OP_FIND_OR_INSERT;
  // Entries of the partition, grouped by bucket and in batch order inside a
  // bucket: the rank of entry e of bucket [lo, hi) in the batch is e - lo.
  __shared__ uint64_t s_key[kFastLds];
  __shared__ uint64_t s_sc[kFastLds];     // input score, then the score of the record
  __shared__ uint32_t s_idx[kFastLds];    // batch index
  __shared__ uint8_t s_slot[kFastLds];    // slot of the outcome (kNoSlot: none)
  __shared__ uint8_t s_fl[kFastLds];      // outcome, metadata record and row task
  __shared__ uint8_t s_more[kMoreEmpty][kFastLds];  // next EMPTY slots of the window (kNoSlot: none)
  __shared__ uint32_t s_cnt[kPartBuckets];  // keys per bucket, fill pointers, then stops
  __shared__ uint32_t s_off[kPartBuckets + 1];  // first entry of each bucket
  __shared__ uint8_t s_bsz[kPartBuckets];   // bucket sizes before the call
  // Row lists of the copies (own storage: copies run while the serial lanes
  // still read and write the scores).
  __shared__ uint32_t s_rows[kBlock / 64][64];
  __shared__ uint32_t s_wsum[kBlock / 64];
  __shared__ uint32_t s_big;
  __shared__ uint8_t s_long[kPartBuckets];  // buckets left to k_apply_part (long buckets)
  __shared__ uint32_t s_nrec, s_npool;  // hand-over records and pool entries of the block
  __shared__ uint8_t s_serial[kPartBuckets];  // buckets left to the serial lanes
  __shared__ uint8_t s_isser[kPartBuckets];   // 1 for those buckets
  __shared__ uint32_t s_nser;
  __shared__ uint32_t s_enext;  // next 64-entry chunk of the emit
  __shared__ uint32_t s_rbase, s_pbase;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t p = blockIdx.x;
  const uint32_t base_e = ps.pinfo[2 * p], m_all = ps.pinfo[2 * p + 1];
  if (m_all > kFastLds) {
    // k_apply_part takes the partition; a big one also gets a slot of
    // big-partition state, which this block resets for k_big_count.
    __shared__ uint32_t s_slot_big;
    if (tid == 0) {
      ps.plist[atomicAdd(&ps.dctr[2], 1u)] = p;
      s_slot_big = kNone;
      if (ps.big && m_all > kBigPart) {
        const uint32_t sl = atomicAdd(&ps.dctr[4], 1u);
        if (sl < kBigMax) {
          ps.big_part[sl] = p;
          s_slot_big = sl;
        }
      }
    }
    __syncthreads();
    if (s_slot_big != kNone) big_slot_reset(ps.big[s_slot_big], tid);
    return;
  }
  if (m_all == 0) return;
  const uint32_t B = t.B;
  const uint64_t part_b0 = (uint64_t)p * kPartBuckets;
  const bool has_in = a.in_scores != nullptr;
  const bool old_for_hit = a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu;
  const bool old_for_new = a.sc.strategy == kLfu && !has_in;
  // Step B2 runs for assign_scores, and on full buckets for insert_and_evict
  // and accum_or_assign, whose handed-over buckets take the queued eviction
  // kernel: a present key past its window is decided here instead of sending
  // its bucket there.  For the other upserts the scan measured slower on a
  // full table of new keys, which all go to the eviction path anyway.
  constexpr bool kRestScan = OP == OP_ASSIGN_SCORES || OP == OP_INSERT_AND_EVICT ||
                             OP == OP_ACCUM_OR_ASSIGN;
  // Batches with repeated keys: a key's later occurrences in its bucket are
  // applied beside its first one (step F), with the scores folded as the
  // sequential updates would leave them.  The fold needs the input scores of
  // the strategies that add them up (and of kCustomized, whose last one wins).
  const bool fold = (OP == OP_FIND_OR_INSERT || OP == OP_INSERT_OR_ASSIGN) &&
                    a.rule == RULE_TILE32 &&
                    (has_in || !(a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu ||
                                 a.sc.strategy == kCustomized));

  /* A. Entries grouped by bucket (every load issued before the first use;
        indices past m_all read entry m_all - 1 and are ignored).  A bucket
        with more than kLaneMax keys is left to k_apply_part, which folds
        repeated keys: its entries are dropped here (buckets are independent,
        so the rest of the partition is applied as usual), and the partition
        is listed with kPartLongOnly.  accum_or_assign lists the whole
        partition instead (k_apply_part applies its accumulations in batch
        order without a fold). */
  {
    const uint64_t b = part_b0 + tid;
    const uint32_t bsz_own = b < t.buckets ? (uint32_t)G(t.bsize)[b] : 0u;
    gptr<const u64x2> ent = G(reinterpret_cast<const u64x2*>(ps.ent)) + base_e;
    u64x2 ev[kPer];
    uint64_t inq[kPer];
    uint32_t lb[kPer], pos[kPer];
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      ev[q] = ent[e < m_all ? e : m_all - 1];
    }
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) inq[q] = has_in ? G(a.in_scores)[ev[q].y] : 0;
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++)
      lb[q] = (uint32_t)(bucket_of(t, ev[q].x) % kPartBuckets);
    s_cnt[tid] = 0;
    s_bsz[tid] = (uint8_t)bsz_own;
    if (tid == 0) {
      s_big = 0;
      s_nrec = 0;
      s_npool = 0;
      s_nser = 0;
      s_enext = 0;
    }
    lds_barrier();
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++)
      if (tid + q * kBlock < m_all) atomicAdd(&s_cnt[lb[q]], 1u);
    lds_barrier();
    const bool lng = kSplitLong && s_cnt[tid] > kLaneMax;
    const uint32_t c = lng ? 0u : s_cnt[tid];
    s_long[tid] = lng ? 1 : 0;
    if (lng) s_big = 2;
    uint32_t x = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t y = __shfl_up(x, d, 64);
      if (lane >= (uint32_t)d) x += y;
    }
    if (lane == 63) s_wsum[wv] = x;
    if (c > kLaneMax) s_big = 1;
    lds_barrier();
    uint32_t pre = 0;
    for (uint32_t q = 0; q < wv; q++) pre += s_wsum[q];
    const uint32_t o = pre + x - c;
    s_off[tid] = o;
    s_cnt[tid] = o;  // fill pointer (this thread read its count above)
    if (tid == kBlock - 1) s_off[kPartBuckets] = o + c;
    lds_barrier();
    if (s_big == 1) {
      // A long bucket: k_apply_part orders the partition.
      if (tid == 0) ps.plist[atomicAdd(&ps.dctr[2], 1u)] = p;
      return;
    }
    if (s_big == 2 && tid == 0)
      ps.plist[ps.np - 1 - atomicAdd(&ps.dctr[5], 1u)] = p | kPartLongOnly;
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      if (tid + q * kBlock < m_all && !s_long[lb[q]]) {
        s_idx[atomicAdd(&s_cnt[lb[q]], 1u)] = (uint32_t)ev[q].y;
      }
    }
    lds_barrier();
    s_cnt[tid] = kNone;  // first rank the parallel pass does not apply (none yet)
    // Batch order inside each bucket: every entry moves to lo + its rank.
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      if (tid + q * kBlock < m_all && !s_long[lb[q]]) {
        const uint32_t lo = s_off[lb[q]], hi = s_off[lb[q] + 1];
        const uint32_t iv = (uint32_t)ev[q].y;
        uint32_t r = 0;
        for (uint32_t y = lo; y < hi; y++) r += s_idx[y] < iv ? 1u : 0u;
        pos[q] = lo + r;
      }
    }
    lds_barrier();
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      if (tid + q * kBlock < m_all && !s_long[lb[q]]) {
        s_key[pos[q]] = ev[q].x;
        s_idx[pos[q]] = (uint32_t)ev[q].y;
        s_sc[pos[q]] = inq[q];
      }
    }
    lds_barrier();
  }
  // Entries kept here (all of them unless long buckets were dropped).
  const uint32_t m = s_off[kPartBuckets];
  if (m == 0) return;  // block-uniform

  /* B. Outcome of every key on the table before the call, with the score,
        metadata record and row task it has if the parallel pass applies it. */
  {
    u32x4 w0[kPer], w1[kPer];
    uint64_t gi[kPer];
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      w0[q] = w1[q] = u32x4{0, 0, 0, 0};
      gi[q] = 0;
      if (e < m) {
        gi[q] = global_idx(t, murmur3(s_key[e]));
        const uint32_t a4 = (uint32_t)(gi[q] & (B - 1)) & ~3u;
        gptr<const u32x4> drow = (gptr<const u32x4>)(G(t.digests) + (gi[q] >> t.bshift) * B);
        w0[q] = drow[a4 >> 4];
        w1[q] = drow[((a4 >> 4) + 1) & (B / 16 - 1)];
      }
    }
    // accum_or_assign: accumulate (flag set) applies to present keys only,
    // assign (flag clear) to absent keys only; the other cases are no-ops.
    bool flag[kPer];
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      flag[q] = OP == OP_ACCUM_OR_ASSIGN && e < m && G(a.accum_flags)[s_idx[e]] != 0;
    }
    WinProbe wp[kPer];
    uint64_t k0[kPer], k1[kPer];  // keys at the first two digest matches
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      wp[q] = WinProbe{0, kNone, kNone, {kNone}, 0, false, true};
      if (e < m) {
        const uint32_t d = key_digest(murmur3(s_key[e]));
        const uint32_t lbk = (uint32_t)((gi[q] >> t.bshift) % kPartBuckets);
        const bool empties = !may_insert || s_bsz[lbk] < B;
        wp[q] = probe_window(w0[q], w1[q], (uint32_t)(gi[q] & (B - 1)), d, B, empties);
      }
    }
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      k0[q] = k1[q] = 0;
      if (e < m) {
        const uint64_t base = (gi[q] >> t.bshift) * B;
        if (wp[q].c0 != kNone) k0[q] = slot_key(t, base + wp[q].c0);
        if (wp[q].c1 != kNone) k1[q] = slot_key(t, base + wp[q].c1);
      }
    }
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      if (e >= m) continue;
      const uint64_t k = s_key[e];
      const uint64_t in = s_sc[e];
      if (fold) {
        // A repeat takes the outcome of the key's first occurrence (step F);
        // its input score stays in s_sc for the fold.
        const uint32_t lo = s_off[(uint32_t)((gi[q] >> t.bshift) % kPartBuckets)];
        bool rep = false;
        for (uint32_t x = lo; x < e; x++) rep |= s_key[x] == k;
        if (rep) {
          s_slot[e] = kNoSlot;
#pragma unroll
          for (uint32_t j = 0; j < kMoreEmpty; j++) s_more[j][e] = kNoSlot;
          s_fl[e] = kResSlow | kRepeat;
          continue;
        }
      }
      uint8_t fl = kResSlow, slot = kNoSlot;
      uint64_t sc = 0;
      // A verified digest match is the first one in probe order, so the key
      // is present there whether or not the window reached an EMPTY slot.
      const bool hit0 = wp[q].c0 != kNone && k0[q] == k;
      const bool hit1 = !hit0 && wp[q].c1 != kNone && k1[q] == k;
      if (hit0 || hit1 || (wp[q].found && !wp[q].over)) {
        const uint64_t des = score_desired(a.sc, has_in, in);
        bool w;
        if ((hit0 || hit1) && OP == OP_ACCUM_OR_ASSIGN && !flag[q]) {
          fl = 0;  // present, assign requested: a no-op
        } else if (!(hit0 || hit1) && OP == OP_ACCUM_OR_ASSIGN && flag[q]) {
          fl = 0;  // absent, accumulate requested: a no-op
        } else if (hit0 || hit1) {
          const bool first = hit0;
          slot = (uint8_t)(first ? wp[q].c0 : wp[q].c1);
          const uint64_t old =
              old_for_hit ? slot_score(t, (gi[q] >> t.bshift) * B + slot) : 0;
          const uint64_t ns = OP == OP_ASSIGN_SCORES ? score_wo_missed(a.sc, has_in, in, old, &w)
                                                     : score_hit(a.sc, has_in, in, des, old, &w);
          fl = kResDup | (w ? kMetaScore : 0);
          sc = ns;
          if (OP == OP_ACCUM_OR_ASSIGN) fl |= kTkAcc;
          else if (moves_rows) fl |= reads_rows ? kTkOut : kTkIn;
        } else if (!may_insert) {
          fl = 0;  // assign_scores: absent keys are a no-op
        } else if (!old_for_new) {
          slot = (uint8_t)wp[q].slot;
          sc = score_new(a.sc, has_in, in, des, 0, &w);
          fl = kResNew | kMetaKey | kTkIn;
        }
      } else if (kRestScan && !wp[q].over &&
                 (OP == OP_ASSIGN_SCORES ||
                  s_bsz[(uint32_t)((gi[q] >> t.bshift) % kPartBuckets)] >= B)) {
        fl = kResSlow | kRest;  // step B2 reads the rest of the bucket
      }
      s_slot[e] = slot;
#pragma unroll
      for (uint32_t j = 0; j < kMoreEmpty; j++)
        s_more[j][e] = wp[q].more[j] != kNone ? (uint8_t)wp[q].more[j] : kNoSlot;
      s_fl[e] = fl;
      if ((fl & kResMask) != kResSlow) s_sc[e] = sc;
    }
    /* B2 (kRestScan).  A key whose window (two 16-slot chunks) held neither
           the key nor an EMPTY slot, in a full bucket (or for assign_scores,
           in any):
           the rest of its bucket's digest line in probe order (the other six
           chunks, then the start chunk's groups before the start's group).
           Up to two digest matches before the first EMPTY slot are checked
           with one 16-byte record load each; the key is then present at a
           match, or absent (a no-op for assign_scores and for an accumulation,
           the eviction path for the others), and only more matches leave it
           to the serial lane. */
    if (kRestScan) {
#pragma unroll 1
      for (uint32_t q = 0; q < kPer; q++) {
        const uint32_t e = tid + q * kBlock;
        if (e >= m || !(s_fl[e] & kRest)) continue;
        const uint64_t k = s_key[e];
        const uint64_t h = murmur3(k);
        const uint64_t g2 = global_idx(t, h);
        const uint32_t ch = (uint32_t)(g2 & (B - 1)) >> 4;
        const uint64_t base = (g2 >> t.bshift) * B;
        gptr<const u32x4> drow = (gptr<const u32x4>)(G(t.digests) + base);
        // The six chunks after the window, then the groups of the start's
        // chunk before the start's group (last in probe order).
        u32x4 w7[7];
#pragma unroll
        for (uint32_t c = 0; c < 7; c++) w7[c] = drow[(ch + 2 + c) & (B / 16 - 1)];
        const uint32_t g0 = ((uint32_t)(g2 & (B - 1)) >> 2) & 3u;
        const uint32_t rep = key_digest(h) * 0x01010101u;
        WinProbe r{0, kNone, kNone, {kNone}, 0, false, false};
#pragma unroll
        for (uint32_t c = 0; c < 7; c++) {
          const uint32_t cb = ((ch + 2 + c) & (B / 16 - 1)) * 16;
          const uint32_t ng = c < 6 ? 4u : g0;  // groups of this chunk in the rest
          if (ng > 0) probe_group(r, w7[c].x, cb, rep, 0xFu);
          if (ng > 1) probe_group(r, w7[c].y, cb + 4, rep, 0xFu);
          if (ng > 2) probe_group(r, w7[c].z, cb + 8, rep, 0xFu);
          if (ng > 3) probe_group(r, w7[c].w, cb + 12, rep, 0xFu);
        }
        uint8_t fl = kResSlow;
        uint8_t slot = kNoSlot;
        if (!r.over) {
          const u64x2 r0 = r.c0 != kNone ? slot_load(t, base + r.c0) : u64x2{0, 0};
          const u64x2 r1 = r.c1 != kNone ? slot_load(t, base + r.c1) : u64x2{0, 0};
          const bool h0 = r.c0 != kNone && r0.x == k;
          const bool h1 = !h0 && r.c1 != kNone && r1.x == k;
          const bool acc_flag = OP == OP_ACCUM_OR_ASSIGN && G(a.accum_flags)[s_idx[e]] != 0;
          if (h0 || h1) {
            if (OP == OP_ACCUM_OR_ASSIGN && !acc_flag) {
              fl = 0;  // present, assign requested: a no-op
            } else {
              const uint64_t in = s_sc[e];
              const uint64_t old = h0 ? r0.y : r1.y;
              bool w;
              const uint64_t ns =
                  OP == OP_ASSIGN_SCORES
                      ? score_wo_missed(a.sc, has_in, in, old, &w)
                      : score_hit(a.sc, has_in, in, score_desired(a.sc, has_in, in), old, &w);
              slot = (uint8_t)(h0 ? r.c0 : r.c1);
              fl = kResDup | (w ? kMetaScore : 0);
              if (OP == OP_ACCUM_OR_ASSIGN) fl |= kTkAcc;
              else if (moves_rows) fl |= reads_rows ? kTkOut : kTkIn;
              s_sc[e] = ns;
            }
          } else if (OP == OP_ASSIGN_SCORES || acc_flag) {
            fl = 0;  // absent: a no-op
          }
        }
        s_slot[e] = slot;
        s_fl[e] = fl;
      }
    }
  }
  lds_barrier();

  /* C. Per bucket, by its thread in batch order, the first key whose
        outcome the parallel pass cannot decide: an undecided probe, a key
        met again (without the fold of step F), a new key that would find the
        bucket full, or a new key whose recorded EMPTY slots earlier new keys
        of the call all took.  A new key whose first EMPTY slot an earlier
        one took moves to the next EMPTY slot of its window: its probe passes
        the taken slot, and no key is present past an EMPTY slot. */
  {
    const uint32_t bk = tid;
    const uint32_t lo = s_off[bk], hi = s_off[bk + 1];
    uint32_t tk0 = 0, tk1 = 0, tk2 = 0, tk3 = 0;  // slots taken by the call's new keys
    uint32_t nnew = 0, stop = kNone;
    for (uint32_t e = lo; e < hi; e++) {
      const uint8_t f = s_fl[e];
      if (f & kRepeat) continue;  // follows the key's first occurrence
      const uint32_t res = f & kResMask;
      bool bad = res == kResSlow;
      if (!bad && !fold) {
        const uint64_t k = s_key[e];
        for (uint32_t x = lo; x < e; x++) bad |= s_key[x] == k;
      }
      if (!bad && res == kResNew) {
        bad = s_bsz[bk] + nnew >= B;
        uint32_t sl = s_slot[e];
#pragma unroll
        for (uint32_t j = 0; j <= kMoreEmpty; j++) {
          if (bad || sl == kNoSlot) break;
          const uint32_t w = sl >> 5, bit = 1u << (sl & 31);
          const uint32_t cur = w == 0 ? tk0 : w == 1 ? tk1 : w == 2 ? tk2 : tk3;
          if (!(cur & bit)) break;  // free: the key takes it
          sl = j < kMoreEmpty ? s_more[j][e] : kNoSlot;
        }
        if (sl == kNoSlot) bad = true;
        if (!bad) {
          s_slot[e] = (uint8_t)sl;
          const uint32_t w = sl >> 5, bit = 1u << (sl & 31);
          tk0 |= w == 0 ? bit : 0u;
          tk1 |= w == 1 ? bit : 0u;
          tk2 |= w == 2 ? bit : 0u;
          tk3 |= w == 3 ? bit : 0u;
          nnew++;
        }
      }
      if (bad) {
        stop = e - lo;
        break;
      }
    }
    s_cnt[bk] = stop;
  }
  lds_barrier();

  /* F. Repeats below a bucket's stop rank: hits at the slot of the key's
        first occurrence, whose record carries the score the sequential
        updates leave (the first occurrence's score, then the fold of the
        repeats' inputs).  find_or_insert reads the row the first occurrence
        wrote (a new key) or the table row; insert_or_assign keeps the last
        occurrence's row write only. */
  if (fold) {
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++) {
      const uint32_t e = tid + q * kBlock;
      if (e >= m) continue;
      const uint8_t f = s_fl[e];
      const uint32_t res = f & kResMask;
      if ((f & kRepeat) || (res != kResDup && res != kResNew)) continue;
      const uint64_t k = s_key[e];
      const uint32_t lbk = (uint32_t)(bucket_of(t, k) % kPartBuckets);
      const uint32_t lo = s_off[lbk], c = s_off[lbk + 1] - lo;
      const uint32_t end = lo + (s_cnt[lbk] < c ? s_cnt[lbk] : c);
      if (e >= end) continue;
      uint64_t sum = 0, in_last = 0;
      uint32_t last = kNone;
      for (uint32_t x = e + 1; x < end; x++) {
        if (s_key[x] != k) continue;
        const uint64_t in = s_sc[x];
        sum += a.sc.strategy == kLfu ? in : (in & kScoreMask);
        in_last = in;
        last = x;
      }
      if (last == kNone) continue;
      s_sc[e] = heavy_score<OP>(a.sc, has_in, false, s_sc[e], sum, in_last);
      const uint8_t tk = OP == OP_FIND_OR_INSERT ? (res == kResNew ? kTkFwd : kTkOut) : kTkIn;
      for (uint32_t x = e + 1; x < end; x++) {
        if (s_key[x] != k) continue;
        s_slot[x] = s_slot[e];
        s_fl[x] = kResDup | kRepeat | ((OP == OP_INSERT_OR_ASSIGN && x != last) ? 0 : tk);
      }
      if (OP == OP_INSERT_OR_ASSIGN) s_fl[e] = f & (uint8_t)~kTkMask;  // superseded
    }
    lds_barrier();
  }

  /* S. The rest of a bucket whose parallel pass stopped, by one lane.  Such
        buckets are listed so that consecutive lanes take them: the serial
        work (long and divergent) then occupies as few waves as possible,
        instead of a few lanes of every wave of the SIMD. */
  uint32_t added = 0;
  uint32_t hand = kNone;  // hand-over of the bucket this lane took: record << 16 | pool entry
  uint32_t hand_bk = 0;   // that bucket
  {
    const uint32_t bk = tid;
    const uint32_t lo = s_off[bk], hi = s_off[bk + 1], c = hi - lo;
    s_isser[bk] = s_cnt[bk] < c ? 1 : 0;
    if (s_cnt[bk] < c) {
      s_serial[atomicAdd(&s_nser, 1u)] = (uint8_t)bk;
    } else if (lo < hi) {
      // Every key of the bucket was applied in parallel.
      uint32_t bsz = s_bsz[bk];
      for (uint32_t x = lo; x < hi; x++) bsz += (s_fl[x] & kResMask) == kResNew ? 1u : 0u;
      s_cnt[bk] = c;
      if (bsz != s_bsz[bk]) {
        G(t.bsize)[part_b0 + bk] = (int32_t)bsz;
        added = bsz - s_bsz[bk];
      }
    }
  }
  lds_barrier();
  // The waves that hold serial lanes run them; meanwhile the other waves write
  // the records and copy the rows of the buckets the parallel pass applied
  // whole (different buckets, so neither touches what the other reads), in
  // 64-entry chunks from a counter that the serial waves join when done.
  const uint32_t ns_w = (s_nser + 63) / 64;
  if (tid < s_nser) {
    const uint32_t bk = s_serial[tid];
    const uint64_t b = part_b0 + bk;
    const uint32_t lo = s_off[bk], hi = s_off[bk + 1], c = hi - lo;
    uint32_t stop = s_cnt[bk];
    uint32_t bsz = s_bsz[bk];
    uint32_t f0 = 0, f1 = 0, f2 = 0, f3 = 0;  // slots filled by the call so far
    for (uint32_t x = lo; x < lo + stop; x++) {
      if ((s_fl[x] & kResMask) == kResNew) {
        const uint32_t sl = s_slot[x], bit = 1u << (sl & 31), wq = sl >> 5;
        f0 |= wq == 0 ? bit : 0u;
        f1 |= wq == 1 ? bit : 0u;
        f2 |= wq == 2 ? bit : 0u;
        f3 |= wq == 3 ? bit : 0u;
        bsz++;
      }
    }
    const uint64_t base = b * (uint64_t)B;
    // In a block with many serial buckets, a lane takes at most kSerialKeys
    // keys: the block's time is its longest serial lane, so a long bucket's
    // rest goes to k_apply_deferred (a 16-lane group with the bucket in
    // registers), like an evicting one.  Blocks with few serial buckets keep
    // them whole (the hand-over costs more than it saves there).
    const uint32_t r_end =
        (s_nser > kSerialCapFrom || (OP == OP_FIND_OR_INSERT && c - stop > kSerialLong))
            ? stop + kSerialKeys
            : c;
    for (uint32_t r = stop; r < c; r++) {
      if (r >= r_end) {
        stop = r;
        break;
      }
      const uint32_t e = lo + r;
      const uint64_t k = s_key[e];
      const uint64_t i = s_idx[e];
      if (OP == OP_FIND_OR_INSERT_PTR && a.lock) {
        // A key met again while its earlier slot is held LOCKED matches
        // nothing there: the eviction kernel, which reads the bucket back
        // with the lock in place, applies the rest of the bucket.
        bool again = false;
        for (uint32_t x = lo; x < e; x++) again |= s_key[x] == k;
        if (again) {
          stop = r;
          break;
        }
      }
      const uint64_t in = has_in ? G(a.in_scores)[i] : 0;
      const uint64_t h = murmur3(k);
      const uint32_t start = (uint32_t)(global_idx(t, h) & (B - 1));
      const uint32_t d = key_digest(h);
      // Most keys here need no new probe.  A key met earlier in the call is
      // present at that key's slot; a key present before the call still is
      // (nothing is evicted here); and the call only removes EMPTY slots, so
      // a key's first EMPTY slot before the call is still its first one
      // unless an earlier key of the call took it.
      int dup = 0;
      int sl = -1;
      bool known = false;
      for (uint32_t x = lo; x < e; x++) {
        if (s_key[x] == k && s_slot[x] != kNoSlot) {
          sl = s_slot[x];
          dup = 1;
          known = true;
        }
      }
      const uint32_t pres = s_fl[e] & kResMask;  // outcome on the table before the call
      if (!known && pres == kResDup) {
        sl = s_slot[e];
        dup = 1;
        known = true;
      }
      if (!known && may_insert && bsz >= B) {
        // A full bucket: the eviction path (which also finds a present key)
        // takes the rest of it, without a scan of the whole bucket here.
        stop = r;
        break;
      }
      if (!known && pres == kResNew) {
        // The probe ends at the first of the recorded EMPTY slots (the first
        // one, then the window's next ones) that no earlier key took.
        uint32_t cand[1 + kMoreEmpty];
        bool taken[1 + kMoreEmpty];
        cand[0] = s_slot[e];
#pragma unroll
        for (uint32_t j = 0; j < kMoreEmpty; j++) cand[1 + j] = s_more[j][e];
#pragma unroll
        for (uint32_t j = 0; j <= kMoreEmpty; j++) taken[j] = false;
        for (uint32_t x = lo; x < e; x++) {
          if ((s_fl[x] & kResMask) == kResNew) {
            const uint32_t sx = s_slot[x];
#pragma unroll
            for (uint32_t j = 0; j <= kMoreEmpty; j++) taken[j] |= sx == cand[j];
          }
        }
#pragma unroll
        for (uint32_t j = 0; j <= kMoreEmpty; j++) {
          if (!known && cand[j] != kNoSlot && !taken[j]) {
            sl = (int)cand[j];
            known = true;
          }
          if (cand[j] == kNoSlot) break;
        }
      }
      if (!known)
        sl = probe_serial(t, base, f0, f1, f2, f3, start, d, k,
                          !may_insert || bsz < B, &dup);
      if (sl < 0 && may_insert) {
        // The eviction path: the rest of the bucket goes to k_apply_deferred.
        stop = r;
        break;
      }
      if (OP == OP_ACCUM_OR_ASSIGN && sl >= 0 && dup) {
        // An accumulation onto a row an earlier key of the call wrote or
        // accumulated runs after that task: the eviction kernel applies the
        // rest of the bucket in order, after this kernel's row tasks.
        bool chain = false;
        for (uint32_t x = lo; x < e; x++)
          chain |= s_slot[x] == (uint32_t)sl && (s_fl[x] & kTkMask) != 0;
        if (chain && G(a.accum_flags)[i] != 0) {
          stop = r;
          break;
        }
      }
      stop = r + 1;
      uint8_t fl = 0;
      if (sl < 0 || (!may_insert && !dup) ||
          (OP == OP_ACCUM_OR_ASSIGN && (G(a.accum_flags)[i] != 0) != (dup != 0))) {
        // assign_scores: absent; accum_or_assign: the flag does not match
        s_slot[e] = kNoSlot;
        s_fl[e] = 0;
        continue;
      }
      const uint32_t slu = (uint32_t)sl;
      const uint64_t des = score_desired(a.sc, has_in, in);
      bool w;
      // The latest earlier record of the call at this slot, and the latest
      // earlier key whose input row is queued for it.
      uint32_t xrec = kNone, xin = kNone;
      for (uint32_t x = lo; x < e; x++) {
        if (s_slot[x] != slu) continue;
        if (s_fl[x] & kMetaMask) xrec = x;
        if ((s_fl[x] & kTkMask) == kTkIn) xin = x;
      }
      if (dup) {
        uint64_t old = 0;
        if (old_for_hit) old = xrec != kNone ? s_sc[xrec] : slot_score(t, base + slu);
        const uint64_t ns = OP == OP_ASSIGN_SCORES ? score_wo_missed(a.sc, has_in, in, old, &w)
                                                   : score_hit(a.sc, has_in, in, des, old, &w);
        fl = kResDup;
        if (w) {
          if (xrec != kNone) {
            s_sc[xrec] = ns;  // one record per slot: the earlier one carries it
          } else {
            fl |= kMetaScore;
            s_sc[e] = ns;
          }
        }
        if (OP == OP_ACCUM_OR_ASSIGN) {
          fl |= kTkAcc;
        } else if (moves_rows) {
          if (reads_rows) {
            fl |= xin != kNone ? kTkFwd : kTkOut;
          } else {
            if (xin != kNone) s_fl[xin] &= (uint8_t)~kTkMask;  // a later write supersedes
            fl |= kTkIn;
          }
        }
      } else {
        const uint64_t old = old_for_new ? slot_score(t, base + slu) : 0;
        const uint64_t ns = score_new(a.sc, has_in, in, des, old, &w);
        s_sc[e] = w ? ns : old;
        fl = kResNew | kMetaKey | kTkIn;
        const uint32_t bit = 1u << (slu & 31), wq = slu >> 5;
        f0 |= wq == 0 ? bit : 0u;
        f1 |= wq == 1 ? bit : 0u;
        f2 |= wq == 2 ? bit : 0u;
        f3 |= wq == 3 ? bit : 0u;
        bsz++;
      }
      s_slot[e] = (uint8_t)slu;
      s_fl[e] = fl;
    }
    s_cnt[bk] = stop;  // keys of rank < stop are applied here
    // A bucket handed over takes a record and pool entries, counted here in
    // LDS; the block reserves them with one pair of atomics below.
    if (stop < c) {
      hand = (atomicAdd(&s_nrec, 1u) << 16) | atomicAdd(&s_npool, c - stop);
      hand_bk = bk;
    }
    if (bsz != s_bsz[bk]) {
      G(t.bsize)[b] = (int32_t)bsz;
      added += bsz - s_bsz[bk];
    }
  }
  if (ns_w < kBlock / 64)
    emit_fast_dyn<OP, U, moves_rows>(t, a, m, part_b0, s_key, s_idx, s_sc, s_slot, s_fl, s_off,
                                     s_cnt, s_isser, s_rows[wv], &s_enext);
  lds_barrier();

  /* W. Records and rows of the serial buckets; also of the others when
        every wave held serial lanes (none was free to emit them above).
        The serial buckets' row tasks are listed first (in s_sc, whose
        scores the records have consumed) and split evenly over the waves:
        they are a few entries of the block, clustered by bucket, so a pass
        over all entries would leave most lanes idle and some waves with
        most of the rows. */
  const uint8_t wser = ns_w == kBlock / 64 ? 2 : 1;
  const bool wlist = moves_rows && wser == 1;
  emit_fast<OP, U, moves_rows>(t, a, m, part_b0, tid, kBlock, wser, s_key, s_idx, s_sc, s_slot,
                               s_fl, s_off, s_cnt, s_isser, s_rows[wv], !wlist);
  if (wlist) {  // uniform in the block
    __shared__ uint32_t s_nlist;
    if (tid == 0) s_nlist = 0;
    lds_barrier();
    uint16_t* s_list = reinterpret_cast<uint16_t*>(s_sc);  // m <= kFastLds entries fit
    for (uint32_t e0 = 0; e0 < m; e0 += kBlock) {
      const uint32_t e = e0 + tid;
      bool has = false;
      if (e < m && (s_fl[e] & kTkMask)) {
        const uint32_t lbk = (uint32_t)(bucket_of(t, s_key[e]) % kPartBuckets);
        has = s_isser[lbk] == 1 && e - s_off[lbk] < s_cnt[lbk];
      }
      const uint64_t bm = __ballot(has);
      uint32_t at = 0;
      if (lane == 0 && bm) at = atomicAdd(&s_nlist, (uint32_t)__popcll(bm));
      at = (uint32_t)__shfl((int)at, 0, 64);
      if (has) s_list[at + __popcll(bm & ((1ull << lane) - 1))] = (uint16_t)e;
    }
    lds_barrier();
    const uint32_t nl = s_nlist;
    const uint32_t per = (nl + kBlock / 64 - 1) / (kBlock / 64);
    const uint32_t j1 = min(nl, (wv + 1) * per);
    for (uint32_t j = wv * per; j < j1; j += 64) {  // uniform in the wave
      uint64_t src = 0, dst = 0, asrc = 0, adst = 0;
      if (j + lane < j1) {
        const uint32_t e = s_list[j + lane];
        fast_row_task<OP>(t, a, e, bucket_of(t, s_key[e]), s_fl[e] & kTkMask, s_idx, s_slot,
                          s_fl, s_off, src, dst, asrc, adst);
      }
      wave_copy_pairs_q<U, 4>(src, dst, t.row_bytes, s_rows[wv]);
      if (OP == OP_ACCUM_OR_ASSIGN)
        wave_accum_pairs<U>(asrc, adst, t.row_bytes, a.value_type, s_rows[wv]);
    }
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) added += __shfl_xor(added, d, 64);
  if (lane == 0) s_wsum[wv] = added;
  lds_barrier();
  if (tid == 0) {
    uint32_t tot = 0;
    for (uint32_t q = 0; q < kBlock / 64; q++) tot += s_wsum[q];
    if (tot) atomicAdd(t.live, (unsigned long long)tot);
    if (s_nrec) {
      s_rbase = atomicAdd(&ps.dctr[0], s_nrec);
      s_pbase = atomicAdd(&ps.dctr[1], s_npool);
    }
  }
  if (s_nrec) {  // uniform in the block
    lds_barrier();
    // Hand-over records {bucket, keys left, 0, pool offset} and the keys
    // left in batch order, for k_apply_deferred.
    if (hand != kNone) {
      const uint32_t lo = s_off[hand_bk] + s_cnt[hand_bk], hi = s_off[hand_bk + 1];
      const uint32_t po = s_pbase + (hand & 0xFFFFu);
      gptr<uint32_t> rec = G(ps.drec) + 4 * (uint64_t)(s_rbase + (hand >> 16));
      rec[0] = (uint32_t)(part_b0 + hand_bk);
      rec[1] = hi - lo;
      rec[2] = 0;
      rec[3] = po;
      gptr<u64x2> pool = G(reinterpret_cast<u64x2*>(ps.dpool)) + po;
      for (uint32_t x = lo; x < hi; x++) {
        u64x2 v;
        v.x = s_key[x];
        v.y = s_idx[x];
        pool[x - lo] = v;
      }
    }
  }

}

// Element size of the accumulating value types (accum_row): 4 for f32 and
// i32, 8 for i64 / u64, 0 for types that accumulate nothing.
__host__ __device__ __forceinline__ uint32_t acc_elem(int vt) {
  return (vt == 0 || vt == 8) ? 4u : (vt == 10 || vt == 11) ? 8u : 0u;
}

// Row moves of a deferred bucket, queued while its keys are applied and run
// after its last key with every load of a round issued before the round's
// first store.  Key q of the bucket (q < kDefKeys) has an entry held by lane
// q & 15, in half q >> 4:
//   ek: read kind (bits 0-1), write kind (bits 2-3), slot (bits 8-15);
//   ex: batch index of the input row that the read forwards (kRdFwd, or the
//       key itself for kRdSelf) or that the write copies or adds;
//   ei: the key's batch index (its output row).
// All moves that touch one slot sit in one entry, the slot's owner: its read
// of the slot's row as the queue found it, then the slot's last write.  The
// other entries read input rows, which no move writes, and write their own
// output rows; so the entries are independent and run in any order.  A move
// the queue cannot hold that way (a write after two reads of the slot, or
// after a read by another key that reads it again; an addition after any
// earlier move on the slot) runs the queue first.
constexpr uint32_t kDefKeys = 16;
constexpr uint32_t kSsOwner = 0x3F;   // slot state: owner entry + 1
constexpr uint32_t kSsWrite = 0x40;   // the owner writes the slot
constexpr uint32_t kSsMulti = 0x80;   // two or more entries read the slot

struct DeferQ {
  uint32_t ek, ex, ei;  // entry q held by lane q
  uint32_t ss0, ss1;    // state of slot l + 16j in byte j (ss0: j < 4)
};

__device__ __forceinline__ uint32_t dq_get(uint32_t v, uint32_t q) {
  return (uint32_t)__shfl((int)v, (int)q, 16);
}
__device__ __forceinline__ void dq_set(uint32_t& v, uint32_t l, uint32_t q, uint32_t v_new) {
  if (l == q) v = v_new;
}
__device__ __forceinline__ uint32_t ss_get(const DeferQ& Q, uint32_t pos) {
  const uint32_t j = pos >> 4;
  const uint32_t w = (uint32_t)__shfl((int)(j < 4 ? Q.ss0 : Q.ss1), (int)(pos & 15), 16);
  return (w >> (8 * (j & 3))) & 0xFFu;
}
__device__ __forceinline__ void ss_set(DeferQ& Q, uint32_t l, uint32_t pos, uint32_t v) {
  if (l != (pos & 15)) return;
  const uint32_t j = pos >> 4, sh = 8 * (j & 3);
  const uint32_t m = ~(0xFFu << sh);
  if (j < 4) Q.ss0 = (Q.ss0 & m) | (v << sh);
  else Q.ss1 = (Q.ss1 & m) | (v << sh);
}

// Runs the queued moves of entries q < nq (all 16 lanes of the group), two
// entries per round, and empties the queue.
template <int OP, int U>
__device__ __forceinline__ void defer_run(const TableView& t, const ApplyArgs& a, uint64_t b,
                                       uint32_t l, DeferQ& Q, uint32_t nq) {
  using T = typename UnitT<U>::T;
  const uint64_t R = t.row_bytes;
  const uint32_t units = t.row_bytes / U;
  const uint32_t gsh = threadIdx.x & 48;  // the group's first lane in the wave
  const uint64_t b0 = __ballot(Q.ek != 0 && l < nq);
  uint32_t mk = (uint32_t)((b0 >> gsh) & 0xFFFFu);
  const uint64_t in_base = (uint64_t)(uintptr_t)a.in_values;
  const uint64_t out_base =
      (uint64_t)(uintptr_t)(OP == OP_INSERT_AND_EVICT ? a.ev_values : a.io_values);
  const bool acc_any = acc_elem(a.value_type) != 0;
  while (mk) {  // uniform in the group
    uint64_t src[4], dst[4];
    bool acc[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
      src[2 * e] = src[2 * e + 1] = dst[2 * e] = dst[2 * e + 1] = 0;
      acc[e] = false;
      if (!mk) continue;
      const uint32_t q = (uint32_t)__builtin_ctz(mk);
      mk &= mk - 1;
      const uint32_t ek = dq_get(Q.ek, q), ex = dq_get(Q.ex, q),
                     ei = dq_get(Q.ei, q);
      const uint32_t rd = ek & 3u, wr = (ek >> 2) & 3u, pos = (ek >> 8) & 0xFFu;
      const uint64_t slot = (uint64_t)(uintptr_t)row_ptr(t, b, pos);
      if (rd != kRdNone) {
        src[2 * e] = rd == kRdSlot ? slot : in_base + (uint64_t)ex * R;
        dst[2 * e] = out_base + (uint64_t)ei * R;
      }
      if (wr == kWrCopy) {
        src[2 * e + 1] = in_base + (uint64_t)ex * R;
        dst[2 * e + 1] = slot;
      } else if (wr == kWrAcc && acc_any) {
        src[2 * e] = slot;  // the row (no read entry holds an addition)
        src[2 * e + 1] = in_base + (uint64_t)ex * R;  // the delta
        dst[2 * e + 1] = slot;
        acc[e] = true;
      }
    }
    gptr<const T> sp[4];
    gptr<T> dp[4];
#pragma unroll
    for (int x = 0; x < 4; x++) {
      sp[x] = G<const T>((uintptr_t)src[x]);
      dp[x] = G<T>((uintptr_t)dst[x]);
    }
    for (uint32_t u0 = l; u0 < units; u0 += 32) {
      T v[4][2];
#pragma unroll
      for (int x = 0; x < 4; x++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t u = u0 + 16 * h;
          if (src[x] && u < units) v[x][h] = __builtin_nontemporal_load(&sp[x][u]);
        }
#pragma unroll
      for (int e = 0; e < 2; e++)
        if (acc[e])
#pragma unroll
          for (int h = 0; h < 2; h++)
            if (u0 + 16 * h < units)
              v[2 * e + 1][h] = add_unit(v[2 * e][h], v[2 * e + 1][h], a.value_type);
#pragma unroll
      for (int x = 0; x < 4; x++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t u = u0 + 16 * h;
          if (dst[x] && u < units) __builtin_nontemporal_store(v[x][h], &dp[x][u]);
        }
    }
  }
  Q.ek = 0;
  Q.ss0 = Q.ss1 = 0;
}

// defer_run for the queue cut short inside a bucket (rare: a move that
// cannot join it), one entry and one unit per lane at a time, so that it
// adds few registers to the bucket state held across it.
template <int OP, int U>
__device__ __forceinline__ void defer_run_narrow(const TableView& t, const ApplyArgs& a,
                                                 uint64_t b, uint32_t l, DeferQ& Q,
                                                 uint32_t nq) {
  using T = typename UnitT<U>::T;
  const uint64_t R = t.row_bytes;
  const uint32_t units = t.row_bytes / U;
  const uint64_t in_base = (uint64_t)(uintptr_t)a.in_values;
  const uint64_t out_base =
      (uint64_t)(uintptr_t)(OP == OP_INSERT_AND_EVICT ? a.ev_values : a.io_values);
  const bool acc_any = acc_elem(a.value_type) != 0;
  for (uint32_t q = 0; q < nq; q++) {  // uniform in the group
    const uint32_t ek = dq_get(Q.ek, q);
    if (!ek) continue;
    const uint32_t ex = dq_get(Q.ex, q), ei = dq_get(Q.ei, q);
    const uint32_t rd = ek & 3u, wr = (ek >> 2) & 3u, pos = (ek >> 8) & 0xFFu;
    const uint64_t slot = (uint64_t)(uintptr_t)row_ptr(t, b, pos);
    uint64_t sa = 0, da = 0, sb = 0, db = 0;
    bool acc = false;
    if (rd != kRdNone) {
      sa = rd == kRdSlot ? slot : in_base + (uint64_t)ex * R;
      da = out_base + (uint64_t)ei * R;
    }
    if (wr == kWrCopy) {
      sb = in_base + (uint64_t)ex * R;
      db = slot;
    } else if (wr == kWrAcc && acc_any) {
      sa = slot;
      sb = in_base + (uint64_t)ex * R;
      db = slot;
      acc = true;
    }
    for (uint32_t u = l; u < units; u += 16) {
      T va{}, vb{};
      if (sa) va = __builtin_nontemporal_load(&G<const T>((uintptr_t)sa)[u]);
      if (sb) vb = __builtin_nontemporal_load(&G<const T>((uintptr_t)sb)[u]);
      if (acc) vb = add_unit(va, vb, a.value_type);
      if (da) __builtin_nontemporal_store(va, &G<T>((uintptr_t)da)[u]);
      if (db) __builtin_nontemporal_store(vb, &G<T>((uintptr_t)db)[u]);
    }
  }
  Q.ek = 0;
  Q.ss0 = Q.ss1 = 0;
}

// True when the row moves of `act` cannot join the queue as it stands (the
// queue runs first, then they join the emptied queue).
__device__ __forceinline__ bool defer_conflict(const DeferQ& Q, const RowAct& act) {
  if (act.wr == kWrNone) return false;  // reads always join
  const uint32_t s = ss_get(Q, act.pos);
  if (!(s & kSsOwner)) return false;
  if (act.wr == kWrAcc) return true;
  return !(s & kSsWrite) && ((s & kSsMulti) || act.rd == kRdSlot);
}

// Queues the row moves of entry e (batch index i) that apply_key_in decided
// without running them (defer_conflict(Q, act) is false).
__device__ __forceinline__ void defer_note(uint32_t l, DeferQ& Q, uint32_t e, uint32_t i,
                                           const RowAct& act) {
  if (act.rd == kRdNone && act.wr == kWrNone) return;  // uniform in the group
  const bool on_slot = act.rd == kRdSlot || act.wr != kWrNone;
  uint32_t s = on_slot ? ss_get(Q, act.pos) : 0u;
  uint32_t own = s & kSsOwner;
  uint32_t ek = act.pos << 8, ex = 0;
  if (act.rd == kRdSelf) {
    ek |= kRdFwd;
    ex = i;
  } else if (act.rd == kRdSlot) {
    if (s & kSsWrite) {
      // The slot holds the owner's queued input row: forward that row.
      ek |= kRdFwd;
      ex = dq_get(Q.ex, own - 1);
    } else {
      ek |= kRdSlot;
      if (own) {
        s |= kSsMulti;
      } else {
        own = e + 1;
        s = own;
      }
    }
  }
  if (act.wr != kWrNone) {
    if (own && own != e + 1) {
      // The owner's entry carries the slot's write: this key's input row
      // replaces whatever it queued for the slot.
      const uint32_t o = own - 1;
      const uint32_t oek = dq_get(Q.ek, o);
      dq_set(Q.ek, l, o, (oek & ~0xCu) | (kWrCopy << 2));
      dq_set(Q.ex, l, o, i);
      s |= kSsWrite;
    } else {
      ek |= act.wr << 2;
      ex = i;
      s = (e + 1) | kSsWrite;
    }
  }
  dq_set(Q.ek, l, e, ek);
  dq_set(Q.ex, l, e, ex);
  dq_set(Q.ei, l, e, i);
  if (on_slot) ss_set(Q, l, act.pos, s);
}

// One 16-lane group per bucket handed over by k_apply_fast, which applied
// (and copied the rows of) the bucket's earlier keys: the keys left go
// through the eviction path, in batch order, each key's row moves in place.
template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_apply_deferred(TableView t, ApplyArgs a,
                                                           PartScratch ps) {
  const uint32_t nrec = *(volatile uint32_t*)ps.dctr;
  const uint32_t gl = threadIdx.x & 15;
  const uint64_t ngroups = (uint64_t)gridDim.x * (kBlock / 16);
  gptr<const u64x2> pool = G(reinterpret_cast<const u64x2*>(ps.dpool));
  for (uint64_t r = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) >> 4; r < nrec;
       r += ngroups) {
    gptr<const uint32_t> rec = G(ps.drec) + 4 * r;
    const uint64_t b = rec[0];
    const uint32_t c = rec[1], po = rec[3];
    // The first 16 keys, one per lane, and their input scores, load beside
    // the bucket instead of one dependent pair per step.
    u64x2 mine;
    mine.x = 0;
    mine.y = 0;
    if (gl < c) mine = pool[po + gl];
    Bucket16 S;
    bucket_load(t, S, b, gl);
    const uint64_t mine_in = (gl < c && a.in_scores) ? G(a.in_scores)[mine.y] : 0;
    for (uint32_t q = 0; q < c; q++) {  // uniform in the group
      if (q < 16) {
        const uint64_t k = shfl_u64(mine.x, (int)q, 16);
        const uint64_t i = shfl_u64(mine.y, (int)q, 16);
        apply_key_in<OP, U>(t, S, a, i, k, shfl_u64(mine_in, (int)q, 16));
      } else {
        const u64x2 v = pool[po + q];
        apply_key<OP, U>(t, S, a, v.y, v.x);
      }
    }
    bucket_finish(t, S);
  }
}

// k_apply_deferred for insert_and_evict and accum_or_assign, whose
// handed-over buckets carry the most row traffic: the row moves are queued
// and run after the bucket's last key (defer_run; in segments of at most
// kDefKeys keys, cut early where a move cannot join the queue), and the next
// record and its keys load while a bucket is applied, so a bucket costs
// about two memory round trips instead of one per key.
template <int OP, int U>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4, 4))) void
k_apply_deferred_q(TableView t, ApplyArgs a, PartScratch ps) {
  const uint32_t nrec = *(volatile uint32_t*)ps.dctr;
  const uint32_t gl = threadIdx.x & 15;
  const uint64_t ngroups = (uint64_t)gridDim.x * (kBlock / 16);
  uint64_t r = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) >> 4;
  if (r >= nrec) return;  // uniform in the group
  const bool has_in = a.in_scores != nullptr;
  gptr<const u64x2> pool = G(reinterpret_cast<const u64x2*>(ps.dpool));
  gptr<const uint32_t> drec = G(ps.drec);
  uint64_t b = drec[4 * r];
  uint32_t c = drec[4 * r + 1], po = drec[4 * r + 3];
  gptr<const uint64_t> pw = G(reinterpret_cast<const uint64_t*>(ps.dpool));
  uint64_t mine_k = 0;  // key and batch index of the bucket's key gl
  uint32_t mine_i = 0;
  if (gl < c) {
    mine_k = pw[2 * (uint64_t)(po + gl)];
    mine_i = (uint32_t)pw[2 * (uint64_t)(po + gl) + 1];
  }
  uint64_t mine_in = (gl < c && has_in) ? G(a.in_scores)[mine_i] : 0;
  while (true) {
    Bucket16 S;
    bucket_load(t, S, b, gl);
    const uint64_t rn = r + ngroups;
    uint64_t nb = 0;
    uint32_t nc = 0, npo = 0;
    if (rn < nrec) {
      nb = drec[4 * rn];
      nc = drec[4 * rn + 1];
      npo = drec[4 * rn + 3];
    }
    uint64_t nmine_k = 0;
    uint32_t nmine_i = 0;
    if (gl < nc) {
      nmine_k = pw[2 * (uint64_t)(npo + gl)];
      nmine_i = (uint32_t)pw[2 * (uint64_t)(npo + gl) + 1];
    }
    uint64_t nin = 0;
    {
      DeferQ Q;
      Q.ek = Q.ex = Q.ei = Q.ss0 = Q.ss1 = 0;
      uint32_t seg0 = 0;  // first key of the queue's segment
      for (uint32_t q = 0; q < c; q++) {  // uniform in the group
        uint64_t k, i, in;
        if (q < 16) {
          k = shfl_u64(mine_k, (int)q, 16);
          i = (uint32_t)__shfl((int)mine_i, (int)q, 16);
          in = shfl_u64(mine_in, (int)q, 16);
        } else {
          const u64x2 v = pool[po + q];
          k = v.x;
          i = v.y;
          in = has_in ? G(a.in_scores)[i] : 0;
        }
        const RowAct act = apply_key_in<OP, U, false>(t, S, a, i, k, in);
        if (q - seg0 == kDefKeys || defer_conflict(Q, act)) {
          defer_run_narrow<OP, U>(t, a, b, gl, Q, q - seg0);
          seg0 = q;
        }
        defer_note(gl, Q, q - seg0, (uint32_t)i, act);
      }
      nin = (gl < nc && has_in) ? G(a.in_scores)[nmine_i] : 0;
      defer_run<OP, U>(t, a, b, gl, Q, c - seg0);
    }
    bucket_finish(t, S);
    if (rn >= nrec) break;
    r = rn;
    b = nb;
    c = nc;
    po = npo;
    mine_k = nmine_k;
    mine_i = nmine_i;
    mine_in = nin;
  }
}

/* ------------------------------------------------------------------------ */
/* pointer APIs: find*, find_and_update, find_or_insert*, lock / unlock      */
/* ------------------------------------------------------------------------ */

// Placement of the pointer find_or_insert for the partitions k_apply_fast
// lists (more entries than one LDS load, or a bucket with more than kLaneMax
// keys): each bucket's keys in batch order through apply_key, one 16-lane
// group per bucket.  A
// partition's entries load in runs that end at a chunk boundary (one chunk's
// entries of a partition are contiguous but unordered), so that a bucket's
// keys in one run all precede its keys in the next.
constexpr uint32_t kSeqCap = 2 * kPartChunk;  // entries per run

template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_apply_seq(TableView t, ApplyArgs a, PartScratch ps) {
  __shared__ uint64_t s_key[kSeqCap];
  __shared__ uint32_t s_idx[kSeqCap];
  __shared__ uint8_t s_bk[kSeqCap];
  __shared__ uint16_t s_ord[kSeqCap];  // run positions grouped by bucket
  __shared__ uint16_t s_srt[kSeqCap];  // ... in batch order within each bucket
  __shared__ uint32_t s_cnt[kPartBuckets], s_off[kPartBuckets], s_fill[kPartBuckets];
  __shared__ uint32_t s_bl[kPartBuckets];  // buckets with keys in the run
  __shared__ uint32_t s_w[kBlock / 64];
  __shared__ uint32_t s_li, s_r1, s_nb;
  const uint32_t tid = threadIdx.x, gl = tid & 15;
  gptr<const u64x2> ent = G(reinterpret_cast<const u64x2*>(ps.ent));
  int32_t added = 0;  // keys this lane's buckets gained
  const uint32_t nlist = *(volatile uint32_t*)&ps.dctr[2];
  if (nlist == 0) return;
  for (;;) {
    if (tid == 0) s_li = atomicAdd(&ps.dctr[3], 1u);
    __syncthreads();
    const uint32_t li = s_li;
    if (li >= nlist) break;  // block-uniform
    const uint32_t p = ps.plist[li];
    const uint32_t base_e = ps.pinfo[2 * p], m = ps.pinfo[2 * p + 1];
    const uint64_t part_b0 = (uint64_t)p * kPartBuckets;
    for (uint32_t r0 = 0; r0 < m;) {
      uint32_t r1 = m;
      if (m - r0 > kSeqCap) {
        // The chunk segment holding entry r0 + kSeqCap has at most
        // kPartChunk entries, so it starts after r0 + kPartChunk.
        const uint32_t cg = (uint32_t)(ent[base_e + r0 + kSeqCap].y / kPartChunk);
        if (tid == 0) s_r1 = r0 + kSeqCap;
        __syncthreads();
        for (uint32_t x = r0 + kPartChunk + tid; x < r0 + kSeqCap; x += kBlock)
          if ((uint32_t)(ent[base_e + x].y / kPartChunk) == cg) atomicMin(&s_r1, x);
        __syncthreads();
        r1 = s_r1;
      }
      const uint32_t mr = r1 - r0;
      s_cnt[tid] = 0;
      if (tid == 0) s_nb = 0;
      __syncthreads();
      for (uint32_t x = tid; x < mr; x += kBlock) {
        const u64x2 e = ent[base_e + r0 + x];
        const uint32_t bk = (uint32_t)(bucket_of(t, e.x) - part_b0);
        s_key[x] = e.x;
        s_idx[x] = (uint32_t)e.y;
        s_bk[x] = (uint8_t)bk;
        atomicAdd(&s_cnt[bk], 1u);
      }
      __syncthreads();
      uint32_t tot;
      const uint32_t c = s_cnt[tid];
      const uint32_t off = block_excl_scan256(c, s_w, &tot);
      s_off[tid] = off;
      s_fill[tid] = off;
      if (c) s_bl[atomicAdd(&s_nb, 1u)] = tid;
      __syncthreads();
      for (uint32_t x = tid; x < mr; x += kBlock)
        s_ord[atomicAdd(&s_fill[s_bk[x]], 1u)] = (uint16_t)x;
      __syncthreads();
      const uint32_t nbk = s_nb;
      for (uint32_t q = tid >> 4; q < nbk; q += kBlock / 16) {
        const uint32_t bk = s_bl[q];
        const uint32_t cc = s_cnt[bk], o = s_off[bk];
        // Rank of each key by batch index (indices are distinct).
        for (uint32_t x = gl; x < cc; x += 16) {
          const uint32_t me = s_ord[o + x];
          const uint32_t iv = s_idx[me];
          uint32_t r = 0;
          for (uint32_t y = 0; y < cc; y++) r += s_idx[s_ord[o + y]] < iv ? 1u : 0u;
          s_srt[o + r] = (uint16_t)me;
        }
        group_sync();
        Bucket16 S;
        bucket_load(t, S, part_b0 + bk, gl);
        for (uint32_t step = 0; step < cc; step++) {
          const uint32_t x = s_srt[o + step];
          apply_key<OP, U>(t, S, a, s_idx[x], s_key[x]);
        }
        // Bucket size now, the live count once per wave at the end.
        if (gl == 0 && S.bsz != S.bsz0) {
          G(t.bsize)[S.b] = S.bsz;
          added += S.bsz - S.bsz0;
        }
      }
      __syncthreads();
      r0 = r1;
    }
    __syncthreads();  // every thread has read s_li before it is rewritten
  }
  int64_t w = added;
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) w += shfl_xor_u64((uint64_t)w, m, 64);
  if ((tid & 63) == 0 && w) atomicAdd(t.live, (unsigned long long)w);
}

// Slot words -> value and key addresses and founds; with `restore`, the key
// goes back over LOCKED (find_or_insert_ptr_kernel_unlock_key_vf,
// find_or_insert_ptr_kernel_v2.h:287-303).  Clears the slot words.
__global__ __launch_bounds__(kBlock) void k_ptr_finish(TableView t,
                                                       const uint64_t* __restrict__ keys,
                                                       uint64_t n, uint64_t* __restrict__ slot_w,
                                                       uint64_t* __restrict__ vptrs,
                                                       uint8_t* __restrict__ founds,
                                                       uint64_t* __restrict__ kptrs, int restore) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const uint64_t v = slot_w[i];
  uint64_t vp = 0, kp = 0;
  if (v) {
    slot_w[i] = 0;
    const uint64_t g = (v & ~kSlotFound) - 1;
    vp = (uint64_t)(uintptr_t)row_ptr(t, g >> t.bshift, (uint32_t)(g & (t.B - 1)));
    kp = (uint64_t)(uintptr_t)(t.slots + 2 * g);
    if (restore) slot_key(t, g) = keys[i];
  }
  vptrs[i] = vp;
  if (founds) founds[i] = (v & kSlotFound) ? 1 : 0;
  if (kptrs) kptrs[i] = kp;
}

// find (pointer overload), find_ptr_with_digest_kernel.h:30-148, and
// find_and_update (UPDATE), find_and_update_kernel_with_filter.h:35-165: the
// row address of each present key, null otherwise; find_and_update first
// applies the hit score functor and returns the score it leaves.
template <bool UPDATE>
__global__ __launch_bounds__(kBlock) void k_find_ptr(TableView t, const uint64_t* __restrict__ keys,
                                                     uint64_t n, uint64_t* __restrict__ vptrs,
                                                     uint8_t* __restrict__ founds,
                                                     uint64_t* __restrict__ scores, ScoreCtx sc) {
  __shared__ ProbeLds s_probe[kBlock / 64];
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const uint64_t k = i < n ? keys[i] : 0;
  uint64_t b = 0;
  const int p = wave_probe(t, k, i < n && !is_reserved(k), use_key_first(t),
                           s_probe[threadIdx.x >> 6], &b);
  if (i >= n) return;
  if (p < 0) {
    vptrs[i] = 0;
    if (founds) founds[i] = 0;
    return;
  }
  const uint64_t g = b * t.B + (uint32_t)p;
  if (UPDATE) {
    const bool has_in = scores != nullptr;
    const uint64_t in = has_in ? scores[i] : 0;
    const uint64_t old = slot_score(t, g);
    bool w;
    const uint64_t ns = score_hit(sc, has_in, in, score_desired(sc, has_in, in), old, &w);
    if (w) slot_score(t, g) = ns;
    if (scores) scores[i] = w ? ns : old;
  } else if (scores) {
    scores[i] = slot_score(t, g);
  }
  vptrs[i] = (uint64_t)(uintptr_t)row_ptr(t, b, (uint32_t)p);
  if (founds) founds[i] = 1;
}

// lock_keys (lock_keys_kernel.h:31-141): a present key's slot goes from the
// key to LOCKED with a CAS, so one occurrence of a repeated key wins; the
// winner applies the hit score functor and returns the slot's key address.
__global__ __launch_bounds__(kBlock) void k_lock_keys(TableView t, const uint64_t* __restrict__ keys,
                                                      uint64_t n, uint64_t* __restrict__ kptrs,
                                                      uint8_t* __restrict__ success,
                                                      const uint64_t* __restrict__ scores,
                                                      ScoreCtx sc) {
  __shared__ ProbeLds s_probe[kBlock / 64];
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const uint64_t k = i < n ? keys[i] : 0;
  uint64_t b = 0;
  const int p = wave_probe(t, k, i < n && !is_reserved(k), use_key_first(t),
                           s_probe[threadIdx.x >> 6], &b);
  if (i >= n) return;
  uint64_t kp = 0;
  if (p >= 0) {
    const uint64_t g = b * t.B + (uint32_t)p;
    unsigned long long* ka = reinterpret_cast<unsigned long long*>(t.slots + 2 * g);
    if (atomicCAS(ka, (unsigned long long)k, (unsigned long long)kLockedKey) ==
        (unsigned long long)k) {
      const bool has_in = scores != nullptr;
      const uint64_t in = has_in ? scores[i] : 0;
      bool w;
      const uint64_t ns =
          score_hit(sc, has_in, in, score_desired(sc, has_in, in), slot_score(t, g), &w);
      if (w) slot_score(t, g) = ns;
      kp = (uint64_t)(uintptr_t)ka;
    }
  }
  kptrs[i] = kp;
  if (success) success[i] = kp ? 1 : 0;
}

// unlock_keys (unlock_keys_kernel.h:40-79): LOCKED -> the caller's key.  An
// address outside the table's key records, or a slot not holding LOCKED,
// reports failure and writes nothing.
__global__ __launch_bounds__(kBlock) void k_unlock_keys(TableView t, uint64_t n,
                                                        const uint64_t* __restrict__ kptrs,
                                                        const uint64_t* __restrict__ keys,
                                                        uint8_t* __restrict__ success) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const uint64_t p = kptrs[i];
  const uint64_t lo = (uint64_t)(uintptr_t)t.slots, hi = lo + 16 * t.capacity;
  bool ok = false;
  if (p >= lo && p < hi && ((p - lo) & 15) == 0) {
    unsigned long long* ka = reinterpret_cast<unsigned long long*>((uintptr_t)p);
    ok = atomicCAS(ka, (unsigned long long)kLockedKey, (unsigned long long)keys[i]) ==
         (unsigned long long)kLockedKey;
  }
  if (success) success[i] = ok ? 1 : 0;
}

/* ------------------------------------------------------------------------ */
/* contains, assign, assign_values                                          */
/* ------------------------------------------------------------------------ */

// contains (contains_kernel.h:31-69): founds only.
__global__ __launch_bounds__(kBlock) void k_contains(TableView t, const uint64_t* __restrict__ keys,
                                                     uint64_t n, uint8_t* __restrict__ founds) {
  __shared__ ProbeLds s_probe[kBlock / 64];
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const uint64_t k = i < n ? keys[i] : 0;
  uint64_t b = 0;
  const int p = wave_probe(t, k, i < n && !is_reserved(k), use_key_first(t),
                           s_probe[threadIdx.x >> 6], &b);
  if (i < n) founds[i] = p >= 0 ? 1 : 0;
}

// assign (assign_kernel.h:31-243) and assign_values
// (assign_values_kernel.h:32-233): a present key's row is overwritten with
// the input row, and with SCORES its score takes update_without_missed.
// Absent keys are no-ops.  One key per lane; the wave copies the rows.
template <bool SCORES, int U>
__global__ __launch_bounds__(kBlock) void k_assign(TableView t, const uint64_t* __restrict__ keys,
                                                   uint64_t n, const uint8_t* __restrict__ in_values,
                                                   const uint64_t* __restrict__ scores,
                                                   ScoreCtx sc) {
  __shared__ uint32_t s_rows[kBlock / 64][64];
  __shared__ ProbeLds s_probe[kBlock / 64];
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const uint32_t wv = threadIdx.x >> 6;
  const uint64_t k = i < n ? keys[i] : 0;
  uint64_t b = 0;
  const int p = wave_probe(t, k, i < n && !is_reserved(k), use_key_first(t), s_probe[wv], &b);
  uint64_t src = 0, dst = 0;
  if (p >= 0) {
    if (SCORES) {
      const uint64_t g = b * t.B + (uint32_t)p;
      const bool has_in = scores != nullptr;
      bool w;
      const uint64_t ns =
          score_wo_missed(sc, has_in, has_in ? scores[i] : 0, slot_score(t, g), &w);
      if (w) slot_score(t, g) = ns;
    }
    if (in_values) {
      src = (uint64_t)(uintptr_t)(in_values + i * (uint64_t)t.row_bytes);
      dst = (uint64_t)(uintptr_t)row_ptr(t, b, (uint32_t)p);
    }
  }
  wave_copy_pairs<U>(src, dst, t.row_bytes, s_rows[wv]);  // every lane of the wave
}

/* ------------------------------------------------------------------------ */
/* export_batch                                                              */
/* ------------------------------------------------------------------------ */

// dump_kernel (include/kernels/dump_kernel/dump_kernel.h:36-122) selects
// slots whose key is not reserved.  Here the output is compacted in slot
// order: count per block, scan, write.
__global__ __launch_bounds__(kBlock) void k_export_count(TableView t, uint64_t offset, uint64_t n,
                                                         uint32_t* __restrict__ block_cnt) {
  const uint64_t s = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const bool live = s < n && !is_reserved(slot_key(t, offset + s));
  const uint64_t m = __ballot(live);
  __shared__ uint32_t w[kBlock / 64];
  if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = __popcll(m);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t c = 0;
    for (int q = 0; q < kBlock / 64; q++) c += w[q];
    block_cnt[blockIdx.x] = c;
  }
}

// Exclusive scan of the block counts in one block; total to *d_counter.
__global__ __launch_bounds__(1024) void k_export_scan(uint32_t* __restrict__ block_cnt,
                                                      uint64_t nblocks,
                                                      uint64_t* __restrict__ d_counter) {
  __shared__ uint64_t part[1024];
  const uint64_t per = cdiv(nblocks, 1024);
  const uint64_t lo = threadIdx.x * per;
  const uint64_t hi = lo + per < nblocks ? lo + per : nblocks;
  uint64_t sum = 0;
  for (uint64_t q = lo; q < hi; q++) sum += block_cnt[q];
  part[threadIdx.x] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const uint64_t v = threadIdx.x >= (uint32_t)off ? part[threadIdx.x - off] : 0;
    __syncthreads();
    part[threadIdx.x] += v;
    __syncthreads();
  }
  uint64_t run = part[threadIdx.x] - sum;
  for (uint64_t q = lo; q < hi; q++) {
    const uint32_t c = block_cnt[q];
    block_cnt[q] = (uint32_t)run;
    run += c;
  }
  if (threadIdx.x == 1023) *d_counter = part[1023];
}

template <int U>
__global__ __launch_bounds__(kBlock) void k_export_write(TableView t, uint64_t offset, uint64_t n,
                                                         const uint32_t* __restrict__ block_off,
                                                         uint64_t* __restrict__ out_keys,
                                                         uint8_t* __restrict__ out_vals,
                                                         uint64_t* __restrict__ out_scores) {
  __shared__ uint32_t w[kBlock / 64];
  __shared__ uint32_t s_rows[kBlock / 64][64];
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint64_t s = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  uint64_t k = kEmptyKey;
  if (s < n) k = slot_key(t, offset + s);
  const bool live = s < n && !is_reserved(k);
  const uint64_t m = __ballot(live);
  if (lane == 0) w[wv] = __popcll(m);
  __syncthreads();
  uint32_t wbase = block_off[blockIdx.x];
  for (uint32_t q = 0; q < wv; q++) wbase += w[q];
  const uint32_t r = __popcll(m & ((1ull << lane) - 1));
  gptr<const uint8_t> src = nullptr;
  if (live) {
    const uint64_t g = offset + s;
    const uint64_t b = g >> t.bshift;
    const uint32_t slot = (uint32_t)(g & (t.B - 1));
    out_keys[wbase + r] = k;
    if (out_scores) out_scores[wbase + r] = slot_score(t, g);
    src = row_ptr(t, b, slot);
    s_rows[wv][r] = lane;
  }
  __syncthreads();
  const uint32_t rows = __popcll(m);
  // Rows go to consecutive outputs: output row of lane L = wbase + rank(L).
  // wave_copy_rows addresses destinations by lane index, so pass the rank
  // through the lane table instead.
  if (rows) {
    using T = typename UnitT<U>::T;
    const uint32_t units = t.row_bytes / U;
    uint32_t lpr = 64;
    while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;
    const uint32_t rpi = 64 / lpr;
    const uint32_t sub = lane % lpr;
    for (uint32_t r0 = 0; r0 < rows; r0 += rpi) {
      const uint32_t rr = r0 + lane / lpr;
      const bool ok = rr < rows;
      const uint32_t srcl = ok ? s_rows[wv][rr] : lane;
      const uint64_t sp = shfl_u64((uint64_t)(uintptr_t)src, (int)srcl, 64);
      if (ok) {
        gptr<const T> sr = G<const T>((uintptr_t)sp);
        gptr<T> dr = G(reinterpret_cast<T*>(out_vals + (uint64_t)(wbase + rr) * t.row_bytes));
        for (uint32_t u = sub; u < units; u += lpr) dr[u] = sr[u];
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* size, rehash, fill                                                        */
/* ------------------------------------------------------------------------ */

__global__ __launch_bounds__(kBlock) void k_size(const int32_t* __restrict__ bsize, uint64_t nb,
                                                 unsigned long long* __restrict__ out) {
  int64_t v = 0;
  for (uint64_t b = (uint64_t)blockIdx.x * kBlock + threadIdx.x; b < nb;
       b += (uint64_t)gridDim.x * kBlock)
    v += bsize[b];
  __shared__ int64_t part[kBlock];
  part[threadIdx.x] = v;
  __syncthreads();
  for (int off = kBlock / 2; off > 0; off >>= 1) {
    if (threadIdx.x < (uint32_t)off) part[threadIdx.x] += part[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0 && part[0]) atomicAdd(out, (unsigned long long)part[0]);
}

__global__ void k_fill_u64(uint64_t* p, uint64_t v, uint64_t n) {
  for (uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; q < n;
       q += (uint64_t)gridDim.x * blockDim.x)
    p[q] = v;
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, uint64_t n) {
  for (uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; q < n;
       q += (uint64_t)gridDim.x * blockDim.x)
    p[q] = v;
}

/* ------------------------------------------------------------------------ */
/* rehash (include/kernels/rehash_kernel/rehash_kernel.h:29-207)             */
/* ------------------------------------------------------------------------ */
//
// k_rehash_plan: one 16-lane group per old bucket b replays the reference's
// one-thread-per-bucket algorithm on the bucket held in registers (lane l
// owns slots l + 16 j): scan from slot 0 for the first key whose bucket
// under the doubled capacity is b + old_buckets, place it at the first
// EMPTY slot of that bucket from its start, backward-shift defragment b
// from the hole, and scan again from slot 0.  Each step is a few ballots
// over per-slot flags instead of a chain of global loads.  Rows do not move
// here: every slot tracks the slot its row started in, and the bucket's row
// moves are recorded, as (first slot, destination) pairs, for
// k_rehash_rows.
//
// Record of a row move: origin slot << 8 | (destination in b + old_buckets)
// << 7 | destination slot, at rec[b * 128 + j]; cnt[b] = moves to the new
// bucket | moves within b << 8 (new-bucket moves first).

// Facts of the key a slot holds, moved with the key: start slot under the
// old capacity (bits 0-6), start slot under the doubled capacity (8-14),
// digest (16-23), whether it moves to the new bucket (24), whether the slot
// holds a key (25).
constexpr uint32_t kRhMove = 1u << 24, kRhLive = 1u << 25;

__device__ __forceinline__ uint32_t rh_info(uint64_t k, uint64_t b, uint64_t old_cap,
                                            uint64_t new_cap, uint32_t B) {
  if (k == kEmptyKey) return 0;
  const uint64_t h = murmur3(k);
  const uint64_t ngi = h % new_cap;
  const bool mv = k != kReclaimKey && ngi / B != b;  // RECLAIM slots are skipped by the scan
  return (uint32_t)((h % old_cap) % B) | ((uint32_t)(ngi % B) << 8) | (key_digest(h) << 16) |
         (mv ? kRhMove : 0u) | kRhLive;
}

__device__ __forceinline__ uint32_t sel8(const uint32_t (&v)[8], uint32_t j) {
  uint32_t r = 0;
#pragma unroll
  for (uint32_t q = 0; q < 8; q++) r |= v[q] & (0u - (uint32_t)(j == q));
  return r;
}

__device__ __forceinline__ void set8(uint32_t (&v)[8], uint32_t j, uint32_t x) {
#pragma unroll
  for (uint32_t q = 0; q < 8; q++) v[q] = j == q ? x : v[q];
}

// 128-bit mask (lo, hi) of a 16-lane group's slots from per-lane flags
// (bit j of f: slot l + 16 j).  Lanes of other groups that are not active
// contribute nothing to this group's bits.
__device__ __forceinline__ void group_mask128(uint32_t f, uint32_t gs, uint64_t& lo,
                                              uint64_t& hi) {
  lo = hi = 0;
#pragma unroll
  for (uint32_t j = 0; j < 8; j++) {
    const uint64_t m = (__ballot((f >> j) & 1u) >> (16 * gs)) & 0xFFFFull;
    if (j < 4) lo |= m << (16 * j);
    else hi |= m << (16 * (j - 4));
  }
}

__device__ __forceinline__ uint32_t ctz128(uint64_t lo, uint64_t hi) {
  return lo ? (uint32_t)__builtin_ctzll(lo) : 64u + (uint32_t)__builtin_ctzll(hi);
}

__global__ __launch_bounds__(kBlock) void k_rehash_plan(TableView t, uint64_t old_nb,
                                                        uint16_t* __restrict__ rec,
                                                        uint16_t* __restrict__ cnt,
                                                        uint32_t* __restrict__ tbase,
                                                        uint32_t* __restrict__ tcount) {
  const uint32_t lane = threadIdx.x & 63, l = lane & 15, gs = lane >> 4;
  const uint64_t b = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) >> 4;
  if (b >= old_nb) return;  // group-uniform
  const uint32_t B = t.B;
  const uint64_t base = b * B, nbase = (b + old_nb) * B;
  const uint64_t old_cap = old_nb * B, new_cap = t.capacity;
  uint64_t key[8], score[8];
  uint32_t info[8], org[8];
#pragma unroll
  for (uint32_t j = 0; j < 8; j++) {
    const u64x2 r = slot_load(t, base + l + 16 * j);
    key[j] = r.x;
    score[j] = r.y;
  }
#pragma unroll
  for (uint32_t j = 0; j < 8; j++) {
    info[j] = rh_info(key[j], b, old_cap, new_cap, B);
    org[j] = l + 16 * j;
  }
  uint64_t occ_lo = 0, occ_hi = 0;  // slots of the new bucket taken so far
  uint32_t n_new = 0;
  for (;;) {
    uint32_t f = 0;
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) f |= ((info[j] & kRhMove) ? 1u : 0u) << j;
    uint64_t mlo, mhi;
    group_mask128(f, gs, mlo, mhi);
    if (!(mlo | mhi)) break;
    // The first key to move, placed at the first free slot of the new
    // bucket from its start there.
    const uint32_t kp = ctz128(mlo, mhi);
    const uint32_t ko = kp & 15, kj = kp >> 4;
    const uint64_t mk = shfl_u64(rec_get(key, kj), (int)ko, 16);
    const uint64_t ms = shfl_u64(rec_get(score, kj), (int)ko, 16);
    const uint32_t mi = __shfl(sel8(info, kj), (int)ko, 16);
    const uint32_t mo = __shfl(sel8(org, kj), (int)ko, 16);
    const uint32_t nkp = (mi >> 8) & 127u;
    uint64_t flo = ~occ_lo, fhi = ~occ_hi;
    rot128(flo, fhi, nkp);
    const uint32_t cp = (nkp + ctz128(flo, fhi)) & 127u;
    if (cp < 64) occ_lo |= 1ull << cp;
    else occ_hi |= 1ull << (cp - 64);
    if (l == (cp & 15)) {
      slot_store(t, nbase + cp, mk, ms);
      G(t.digests)[nbase + cp] = (uint8_t)(mi >> 16);
    }
    if (l == 0) rec[b * B + n_new] = (uint16_t)((mo << 8) | 0x80u | cp);
    n_new++;
    if (l == ko) {
      rec_set(key, kj, kEmptyKey);
      set8(info, kj, 0u);
    }
    // Backward-shift defragmentation from the hole at rp: the first slot
    // after rp (circularly) that is EMPTY ends it; the first key before that
    // whose old start slot lies cyclically outside (rp, cur] fills the hole.
    uint32_t rp = kp;
    for (;;) {
      uint32_t fe = 0, fc = 0;
#pragma unroll
      for (uint32_t j = 0; j < 8; j++) {
        const uint32_t cur = l + 16 * j;
        const bool live = (info[j] & kRhLive) != 0;
        const uint32_t sp = info[j] & 127u;
        const bool c = (sp <= rp && rp < cur) || (cur < sp && sp <= rp) || (rp < cur && cur < sp);
        fe |= (live ? 0u : 1u) << j;
        fc |= (live && c ? 1u : 0u) << j;
      }
      uint64_t elo, ehi, clo, chi;
      group_mask128(fe, gs, elo, ehi);
      group_mask128(fc, gs, clo, chi);
      uint64_t xlo = elo | clo, xhi = ehi | chi;
      const uint32_t sh = (rp + 1) & 127u;
      rot128(xlo, xhi, sh);
      xhi &= ~(1ull << 63);  // rp itself
      if (!(xlo | xhi)) break;
      const uint32_t q = (sh + ctz128(xlo, xhi)) & 127u;
      const bool q_empty = q < 64 ? ((elo >> q) & 1) : ((ehi >> (q - 64)) & 1);
      if (q_empty) break;
      const uint32_t qo = q & 15, qj = q >> 4, ro = rp & 15, rj = rp >> 4;
      const uint64_t vk = shfl_u64(rec_get(key, qj), (int)qo, 16);
      const uint64_t vs = shfl_u64(rec_get(score, qj), (int)qo, 16);
      const uint32_t vi = __shfl(sel8(info, qj), (int)qo, 16);
      const uint32_t vo = __shfl(sel8(org, qj), (int)qo, 16);
      if (l == ro) {
        rec_set(key, rj, vk);
        rec_set(score, rj, vs);
        set8(info, rj, vi);
        set8(org, rj, vo);
      }
      if (l == qo) {
        rec_set(key, qj, kEmptyKey);
        set8(info, qj, 0u);
      }
      rp = q;
    }
  }
  // Write the bucket back; record the rows that end in another slot of b.
  uint32_t fm = 0;
#pragma unroll
  for (uint32_t j = 0; j < 8; j++) {
    const uint32_t s = l + 16 * j;
    slot_store(t, base + s, key[j], score[j]);
    G(t.digests)[base + s] = (info[j] & kRhLive) ? (uint8_t)(info[j] >> 16) : kEmptyDigest;
    fm |= ((info[j] & kRhLive) && org[j] != s ? 1u : 0u) << j;
  }
  uint64_t ilo, ihi;
  group_mask128(fm, gs, ilo, ihi);
  const uint32_t n_int = __popcll(ilo) + __popcll(ihi);
#pragma unroll
  for (uint32_t j = 0; j < 8; j++) {
    if ((fm >> j) & 1u) {
      const uint32_t s = l + 16 * j;
      const uint32_t below = s < 64 ? __popcll(ilo & ((1ull << s) - 1))
                                    : __popcll(ilo) + __popcll(ihi & ((1ull << (s - 64)) - 1));
      rec[b * B + n_new + below] = (uint16_t)((org[j] << 8) | s);
    }
  }
  if (l == 0) {
    cnt[b] = (uint16_t)(n_new | (n_int << 8));
    if (n_new) {
      G(t.bsize)[b] -= (int32_t)n_new;
      G(t.bsize)[b + old_nb] = (int32_t)n_new;
    }
    tbase[b] = n_int ? atomicAdd(tcount, n_int) : 0u;
  }
}

// Executes the recorded row moves, one lane per record, rows copied by the
// wave together.  Phase 0 reads only rows in their first slots: it writes
// the rows that go to new buckets and stages the rows that stay in their
// bucket in `stage`; phase 1 writes the staged rows to their slots.
template <int U>
__global__ __launch_bounds__(kBlock) void k_rehash_rows(TableView t, uint64_t old_nb,
                                                        const uint16_t* __restrict__ rec,
                                                        const uint16_t* __restrict__ cnt,
                                                        const uint32_t* __restrict__ tbase,
                                                        uint8_t* __restrict__ stage, int phase) {
  __shared__ uint32_t s_rows[kBlock / 64][64];
  const uint32_t B = t.B, R = t.row_bytes;
  const uint64_t x = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  uint64_t src = 0, dst = 0;
  if (x < old_nb * B) {
    const uint64_t b = x / B;
    const uint32_t j = (uint32_t)(x % B);
    const uint32_t c = cnt[b], nn = c & 0xFFu, ni = c >> 8;
    if (j < nn + ni) {
      const uint32_t r = rec[x], o = r >> 8, d = r & 127u;
      const bool to_new = (r & 0x80u) != 0;
      const uint64_t st = (uint64_t)(tbase[b] + (j - nn)) * R;
      if (phase == 0) {
        src = (uint64_t)(uintptr_t)row_ptr(t, b, o);
        dst = to_new ? (uint64_t)(uintptr_t)row_ptr(t, b + old_nb, d)
                     : (uint64_t)(uintptr_t)(stage + st);
      } else if (!to_new) {
        src = (uint64_t)(uintptr_t)(stage + st);
        dst = (uint64_t)(uintptr_t)row_ptr(t, b, d);
      }
    }
  }
  wave_copy_pairs<U>(src, dst, R, s_rows[threadIdx.x >> 6]);
}

}  // namespace

/* ------------------------------------------------------------------------ */
/* launchers                                                                 */
/* ------------------------------------------------------------------------ */

static inline unsigned grid_for(uint64_t work, uint64_t per_block, uint64_t cap = 1u << 20) {
  uint64_t g = cdiv(work, per_block);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

void launch_init_slots(const TableView& t, uint64_t b0, uint64_t b1, hipStream_t s) {
  const uint64_t slots = (b1 - b0) * t.B;
  hipLaunchKernelGGL(k_init_slots, dim3(grid_for(slots, kBlock * 4, 65536)), dim3(kBlock), 0,
                     s, t, b0 * t.B, b1 * t.B, b0, b1, 1);
}

void launch_clear(const TableView& t, hipStream_t s) {
  const uint64_t slots = t.buckets * t.B;
  hipLaunchKernelGGL(k_init_slots, dim3(grid_for(slots, kBlock * 4, 65536)), dim3(kBlock), 0,
                     s, t, (uint64_t)0, slots, (uint64_t)0, t.buckets, 0);
  launch_fill_u64(reinterpret_cast<uint64_t*>(t.live), 0, 1, s);
}

void launch_fill_u64(uint64_t* p, uint64_t v, uint64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_fill_u64, dim3(grid_for(n, kBlock, 4096)), dim3(kBlock), 0, s, p, v, n);
}

void launch_fill_u32(uint32_t* p, uint32_t v, uint64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(n, kBlock, 4096)), dim3(kBlock), 0, s, p, v, n);
}

template <bool MISSED>
static void find_dispatch(const TableView& t, const uint64_t* keys, uint64_t n, uint8_t* values,
                          uint8_t* founds, uint64_t* scores, uint64_t* mk, int32_t* mi,
                          int32_t* ms, int unit, hipStream_t s) {
  // 1024-thread blocks: half as many blocks as 512-thread ones and a quarter
  // of 256-thread ones for the same waves (2^20 keys: 1024 blocks), which
  // drains the second round of blocks faster (in-step find 0.1455 ms at 256
  // threads, 0.1434 at 512, 0.1428 at 1024).
  constexpr int BLK = 1024;
  const dim3 g(grid_for(n, BLK, 1ull << 31)), b(BLK);
#define HKV_FIND_U(UU)                                                                      \
  hipLaunchKernelGGL((k_find<UU, MISSED, BLK>), g, b, 0, s, t, keys, n, values, founds, scores, \
                     mk, mi, ms)
  switch (unit) {
    case 16: HKV_FIND_U(16); break;
    case 8: HKV_FIND_U(8); break;
    case 4: HKV_FIND_U(4); break;
    case 2: HKV_FIND_U(2); break;
    default: HKV_FIND_U(1); break;
  }
#undef HKV_FIND_U
}

void launch_find(const TableView& t, const uint64_t* keys, uint64_t n, uint8_t* values,
                 uint8_t* founds, uint64_t* scores, int unit, hipStream_t s) {
  find_dispatch<false>(t, keys, n, values, founds, scores, nullptr, nullptr, nullptr, unit, s);
}

void launch_find_missed(const TableView& t, const uint64_t* keys, uint64_t n, uint8_t* values,
                        uint64_t* mk, int32_t* mi, int32_t* ms, uint64_t* scores, int unit,
                        hipStream_t s) {
  find_dispatch<true>(t, keys, n, values, nullptr, scores, mk, mi, ms, unit, s);
}

void launch_erase(const TableView& t, const uint64_t* keys, uint64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_erase, dim3(grid_for(n, kBlock, 1ull << 31)), dim3(kBlock), 0, s, t,
                     keys, n);
}

template <int OP>
static void apply_part_op(const TableView& t, const ApplyArgs& a, const PartScratch& ps,
                          hipStream_t s) {
  const size_t lds = (size_t)(ps.np < ps.prange ? ps.np : ps.prange) * sizeof(uint32_t);
  hipLaunchKernelGGL(k_pcount, dim3(ps.chunks), dim3(kBlock), lds, s, t, a.keys, a.n, ps);
  hipLaunchKernelGGL(k_pscan, dim3((ps.np + kScanCols - 1) / kScanCols), dim3(1024), 0, s, ps);
  hipLaunchKernelGGL(k_pscatter, dim3(ps.chunks), dim3(kBlock), lds, s, t, a.keys, a.n, ps);
  const dim3 g(ps.np), b(kBlock);
  // After the single-run kernel, the eviction path and the multi-run kernel
  // walk device-side lists that are usually empty: small grids.  Batches
  // with repeated keys list many partitions (every bucket with more than 32
  // keys lists its partition); two blocks of the multi-run kernel fit a CU
  // (LDS and registers), so for them 512 blocks take the list two per CU.
  // The eviction kernels hold four waves per SIMD: 1024 blocks of 256
  // threads fill 256 CUs in one round (a second round would double the cost
  // of the usual empty launch).
  const dim3 gd(grid_for(a.n * 16, kBlock, 1024));
  const uint32_t gpn = a.rule == RULE_TILE32 ? 512u : 256u;
  const dim3 gp(ps.np < gpn ? ps.np : gpn);
  const uint32_t nw = (uint32_t)((a.n + 31) / 32);
  const uint32_t nbw = (nw + kEvBlkWords - 1) / kEvBlkWords;
  // Big partitions: at most n / kBigPart of them, kBigTile entries per tile.
  const dim3 gb(grid_for(a.n / kBigTile + kBigMax, 1, 1024));
#define HKV_PART_U(UU)                                                                       \
  hipLaunchKernelGGL((k_apply_fast<OP, UU>), g, b, 0, s, t, a, ps);                          \
  if ((OP == OP_INSERT_AND_EVICT && a.ev_bits) ||                                            \
      (OP == OP_ACCUM_OR_ASSIGN && UU >= acc_elem(a.value_type)))                            \
    hipLaunchKernelGGL((k_apply_deferred_q<OP == OP_ACCUM_OR_ASSIGN ? OP : OP_INSERT_AND_EVICT, UU>), \
                       gd, b, 0, s, t, a, ps);                                               \
  else                                                                                       \
    hipLaunchKernelGGL((k_apply_deferred<OP, UU>), gd, b, 0, s, t, a, ps);                     \
  if (ps.big) {                                                                              \
    hipLaunchKernelGGL(k_big_count, gb, b, 0, s, t, ps);                                     \
    hipLaunchKernelGGL((k_big_fold<OP>), gb, b, 0, s, t, a, ps);                             \
  }                                                                                          \
  hipLaunchKernelGGL((k_apply_part<OP, UU>), gp, b, 0, s, t, a, ps);                         \
  if (ps.big && OP != OP_ASSIGN_SCORES)                                                      \
    hipLaunchKernelGGL((k_big_tasks<OP, UU>), gb, b, 0, s, t, a, ps);                        \
  if (OP == OP_FIND_OR_INSERT)                                                               \
    hipLaunchKernelGGL((k_rowtasks<UU>), dim3(grid_for(a.n, kBlock, 2048)), b, 0, s, t, a, ps); \
  if (OP == OP_INSERT_AND_EVICT && a.ev_bits) {                                              \
    hipLaunchKernelGGL(k_evc_count, dim3(nbw), b, 0, s, ps.ev_bits, nw, ps.ev_wpre, ps.ev_blk); \
    hipLaunchKernelGGL(k_evc_scan, dim3(1), b, 0, s, ps.ev_blk, nbw, ps.ev_bits, ps.ev_wpre,   \
                       nw, a.ev_counter);                                                    \
    hipLaunchKernelGGL((k_evc_move<UU>), dim3(grid_for(a.n, kBlock, 2048)), b, 0, s,         \
                       ps.ev_bits, nw, ps.ev_wpre, ps.ev_blk, nbw, a.n, a.ev_keys,          \
                       a.ev_values, a.ev_scores, t.row_bytes);                               \
  }
  switch (a.unit) {
    case 16: HKV_PART_U(16); break;
    case 8: HKV_PART_U(8); break;
    case 4: HKV_PART_U(4); break;
    case 2: HKV_PART_U(2); break;
    default: HKV_PART_U(1); break;
  }
#undef HKV_PART_U
}

void launch_apply_part(const TableView& t, int op, const ApplyArgs& a, const PartScratch& ps,
                       hipStream_t s) {
  switch (op) {
    case OP_INSERT_OR_ASSIGN: apply_part_op<OP_INSERT_OR_ASSIGN>(t, a, ps, s); break;
    case OP_FIND_OR_INSERT: apply_part_op<OP_FIND_OR_INSERT>(t, a, ps, s); break;
    case OP_INSERT_AND_EVICT: apply_part_op<OP_INSERT_AND_EVICT>(t, a, ps, s); break;
    case OP_ACCUM_OR_ASSIGN: apply_part_op<OP_ACCUM_OR_ASSIGN>(t, a, ps, s); break;
    default: apply_part_op<OP_ASSIGN_SCORES>(t, a, ps, s); break;
  }
}

void launch_find_or_insert_ptr(const TableView& t, const ApplyArgs& a0, const PartScratch& ps,
                               uint64_t* vptrs, uint8_t* founds, uint64_t* kptrs,
                               bool keep_locked, hipStream_t s) {
  ApplyArgs a = a0;
  a.slot_out = ps.trow;
  const size_t lds = (size_t)(ps.np < ps.prange ? ps.np : ps.prange) * sizeof(uint32_t);
  hipLaunchKernelGGL(k_pcount, dim3(ps.chunks), dim3(kBlock), lds, s, t, a.keys, a.n, ps);
  hipLaunchKernelGGL(k_pscan, dim3((ps.np + kScanCols - 1) / kScanCols), dim3(1024), 0, s, ps);
  hipLaunchKernelGGL(k_pscatter, dim3(ps.chunks), dim3(kBlock), lds, s, t, a.keys, a.n, ps);
  const dim3 g(ps.np), b(kBlock);
  hipLaunchKernelGGL((k_apply_fast<OP_FIND_OR_INSERT_PTR, 16>), g, b, 0, s, t, a, ps);
  hipLaunchKernelGGL((k_apply_deferred<OP_FIND_OR_INSERT_PTR, 16>),
                     dim3(grid_for(a.n * 16, kBlock, 1024)), b, 0, s, t, a, ps);
  const dim3 gp(ps.np < 256 ? ps.np : 256);
  hipLaunchKernelGGL((k_apply_seq<OP_FIND_OR_INSERT_PTR, 16>), gp, b, 0, s, t, a, ps);
  hipLaunchKernelGGL(k_ptr_finish, dim3(grid_for(a.n, kBlock, 1ull << 31)), b, 0, s, t, a.keys,
                     a.n, ps.trow, vptrs, founds, kptrs, (a.lock && !keep_locked) ? 1 : 0);
}

void launch_contains(const TableView& t, const uint64_t* keys, uint64_t n, uint8_t* founds,
                     hipStream_t s) {
  hipLaunchKernelGGL(k_contains, dim3(grid_for(n, kBlock, 1ull << 31)), dim3(kBlock), 0, s, t,
                     keys, n, founds);
}

void launch_assign(const TableView& t, const uint64_t* keys, uint64_t n, const uint8_t* values,
                   const uint64_t* scores, bool with_scores, const ScoreCtx& sc, int unit,
                   hipStream_t s) {
  const dim3 g(grid_for(n, kBlock, 1ull << 31)), b(kBlock);
#define HKV_ASSIGN_U(UU)                                                                    \
  if (with_scores)                                                                         \
    hipLaunchKernelGGL((k_assign<true, UU>), g, b, 0, s, t, keys, n, values, scores, sc);  \
  else                                                                                     \
    hipLaunchKernelGGL((k_assign<false, UU>), g, b, 0, s, t, keys, n, values, scores, sc);
  switch (unit) {
    case 16: HKV_ASSIGN_U(16); break;
    case 8: HKV_ASSIGN_U(8); break;
    case 4: HKV_ASSIGN_U(4); break;
    case 2: HKV_ASSIGN_U(2); break;
    default: HKV_ASSIGN_U(1); break;
  }
#undef HKV_ASSIGN_U
}

void launch_find_ptr(const TableView& t, const uint64_t* keys, uint64_t n, uint64_t* vptrs,
                     uint8_t* founds, uint64_t* scores, bool update, const ScoreCtx& sc,
                     hipStream_t s) {
  const dim3 g(grid_for(n, kBlock, 1ull << 31)), b(kBlock);
  if (update)
    hipLaunchKernelGGL(k_find_ptr<true>, g, b, 0, s, t, keys, n, vptrs, founds, scores, sc);
  else
    hipLaunchKernelGGL(k_find_ptr<false>, g, b, 0, s, t, keys, n, vptrs, founds, scores, sc);
}

void launch_lock_keys(const TableView& t, const uint64_t* keys, uint64_t n, uint64_t* kptrs,
                      uint8_t* success, const uint64_t* scores, const ScoreCtx& sc,
                      hipStream_t s) {
  hipLaunchKernelGGL(k_lock_keys, dim3(grid_for(n, kBlock, 1ull << 31)), dim3(kBlock), 0, s, t,
                     keys, n, kptrs, success, scores, sc);
}

void launch_unlock_keys(const TableView& t, uint64_t n, const uint64_t* kptrs,
                        const uint64_t* keys, uint8_t* success, hipStream_t s) {
  hipLaunchKernelGGL(k_unlock_keys, dim3(grid_for(n, kBlock, 1ull << 31)), dim3(kBlock), 0, s, t,
                     n, kptrs, keys, success);
}

void launch_export(const TableView& t, uint64_t offset, uint64_t n, uint64_t* d_counter,
                   uint64_t* keys, uint8_t* values, uint64_t* scores, uint32_t* block_scratch,
                   int unit, hipStream_t s) {
  const uint64_t nblocks = cdiv(n, kBlock);
  hipLaunchKernelGGL(k_export_count, dim3((unsigned)nblocks), dim3(kBlock), 0, s, t, offset, n,
                     block_scratch);
  hipLaunchKernelGGL(k_export_scan, dim3(1), dim3(1024), 0, s, block_scratch, nblocks, d_counter);
  const dim3 g((unsigned)nblocks), b(kBlock);
  switch (unit) {
    case 16: hipLaunchKernelGGL(k_export_write<16>, g, b, 0, s, t, offset, n, block_scratch, keys, values, scores); break;
    case 8: hipLaunchKernelGGL(k_export_write<8>, g, b, 0, s, t, offset, n, block_scratch, keys, values, scores); break;
    case 4: hipLaunchKernelGGL(k_export_write<4>, g, b, 0, s, t, offset, n, block_scratch, keys, values, scores); break;
    case 2: hipLaunchKernelGGL(k_export_write<2>, g, b, 0, s, t, offset, n, block_scratch, keys, values, scores); break;
    default: hipLaunchKernelGGL(k_export_write<1>, g, b, 0, s, t, offset, n, block_scratch, keys, values, scores); break;
  }
}

void launch_size(const TableView& t, uint64_t nb, uint64_t* out, hipStream_t s) {
  hipLaunchKernelGGL(k_size, dim3(grid_for(nb, kBlock * 8, 1024)), dim3(kBlock), 0, s,
                     t.bsize, nb, reinterpret_cast<unsigned long long*>(out));
}

void launch_rehash_plan(const TableView& t, uint64_t old_nb, const RehashScratch& rs,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_rehash_plan, dim3(grid_for(old_nb * 16, kBlock, 1ull << 31)),
                     dim3(kBlock), 0, s, t, old_nb, rs.rec, rs.cnt, rs.tbase, rs.tcount);
}

void launch_rehash_rows(const TableView& t, uint64_t old_nb, const RehashScratch& rs,
                        uint8_t* stage, int phase, int unit, hipStream_t s) {
  const dim3 g(grid_for(old_nb * t.B, kBlock, 1ull << 31)), b(kBlock);
#define HKV_RH_U(UU)                                                                        \
  hipLaunchKernelGGL((k_rehash_rows<UU>), g, b, 0, s, t, old_nb, rs.rec, rs.cnt, rs.tbase, \
                     stage, phase)
  switch (unit) {
    case 16: HKV_RH_U(16); break;
    case 8: HKV_RH_U(8); break;
    case 4: HKV_RH_U(4); break;
    case 2: HKV_RH_U(2); break;
    default: HKV_RH_U(1); break;
  }
#undef HKV_RH_U
}

}  // namespace hkv
