// hkv_kernels.hip -- gfx950 (wave64) kernels of the HierarchicalKV table.
//
// Read-only and idempotent operations (find, find missed, erase, export,
// size, clear) run one thread per key or per slot.  Every mutating batch
// operation (insert_or_assign, find_or_insert, insert_and_evict,
// accum_or_assign, assign_scores) runs in two steps:
//   1. route: every key atomically appends its batch index to its bucket's
//      pending list (arrival order);
//   2. apply: one 16-lane group owns one bucket, sorts the bucket's pending
//      indices and applies the keys one at a time in increasing batch index.
// A bucket is therefore only ever written by one group, with no atomics on
// table memory, and the outcome equals the reference kernel run key by key
// in batch order (including slot placement and eviction tie-breaks).
// Buckets that receive more keys than the pending list holds are applied by
// a second kernel that walks the whole batch in index order.
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
    t.digests[s] = kEmptyDigest;
    t.keys[s] = kEmptyKey;
    if (reset_scores) t.scores[s] = 0;
  }
  for (uint64_t b = b0 + blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < b1;
       b += stride)
    t.bsize[b] = 0;
}

/* ------------------------------------------------------------------------ */
/* find                                                                      */
/* ------------------------------------------------------------------------ */

// find_without_lock (include/find_utils.h:31-86): 4-digest groups from
// align4(start) with wrap; digest matches are confirmed by the key; the first
// EMPTY slot at or after `start` ends the search.  Digests are fetched 16
// bytes at a time.
__device__ __forceinline__ int probe_find(const TableView& t, uint64_t b,
                                          uint32_t start, uint32_t d, uint64_t k) {
  const uint32_t B = t.B;
  const uint8_t* dg = t.digests + b * B;
  const uint64_t* ks = t.keys + b * B;
  const uint32_t a = start & ~3u;
  const uint32_t rep = d * 0x01010101u;
  const uint32_t erep = (uint32_t)kEmptyDigest * 0x01010101u;
  uint32_t cur = kNone;
  uint4 chunk = make_uint4(0, 0, 0, 0);
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t c = g >> 4;
    if (c != cur) {
      chunk = *reinterpret_cast<const uint4*>(dg + (c << 4));
      cur = c;
    }
    const uint32_t wi = (g >> 2) & 3;
    const uint32_t w = wi == 0 ? chunk.x : wi == 1 ? chunk.y : wi == 2 ? chunk.z : chunk.w;
    uint32_t m = eq_bytes4(w, rep);
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      if (ks[g + j] == k) return (int)(g + j);
    }
    uint32_t e = eq_bytes4(w, erep);
    while (e) {
      const uint32_t j = __builtin_ctz(e);
      e &= e - 1;
      const uint32_t p = g + j;
      if (off == 0 && p < start) continue;
      return -1;  // the empty digest marks an EMPTY slot
    }
  }
  return -1;
}

// Wave-cooperative copy of up to 64 rows.  `rows` lane ids are listed in
// lds_rows; row r's source is `src` of lane lds_rows[r], its destination is
// dst_base + (lane_base + lds_rows[r]) * row_bytes.
template <int U>
__device__ __forceinline__ void wave_copy_rows(uint32_t rows, const uint32_t* lds_rows,
                                               const uint8_t* src,
                                               uint8_t* dst_base, uint64_t lane_base,
                                               uint32_t row_bytes, bool src_is_out) {
  using T = typename UnitT<U>::T;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t units = row_bytes / U;
  uint32_t lpr = 64;
  while (lpr > 1 && lpr / 2 >= units) lpr >>= 1;  // lanes per row
  const uint32_t rpi = 64 / lpr;                    // rows per iteration
  const uint32_t sub = lane % lpr;
  for (uint32_t r0 = 0; r0 < rows; r0 += 4 * rpi) {
    const T* s[4];
    T* d[4];
    bool ok[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t r = r0 + q * rpi + lane / lpr;
      ok[q] = r < rows;
      const uint32_t src_lane = ok[q] ? lds_rows[r] : lane;
      const uint64_t sp = shfl_u64((uint64_t)(uintptr_t)src, (int)src_lane, 64);
      const uint64_t row_index = lane_base + src_lane;
      if (src_is_out) {
        s[q] = reinterpret_cast<const T*>(dst_base + row_index * row_bytes);
        d[q] = reinterpret_cast<T*>((uintptr_t)sp);
      } else {
        s[q] = reinterpret_cast<const T*>((uintptr_t)sp);
        d[q] = reinterpret_cast<T*>(dst_base + row_index * row_bytes);
      }
    }
    for (uint32_t u = sub; u < units; u += lpr) {
      T v[4];
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (ok[q]) v[q] = s[q][u];
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (ok[q]) d[q][u] = v[q];
    }
  }
}

template <int U, bool MISSED>
__global__ __launch_bounds__(kBlock) void k_find(TableView t, const uint64_t* __restrict__ keys,
                                                 uint64_t n, uint8_t* __restrict__ values,
                                                 uint8_t* __restrict__ founds,
                                                 uint64_t* __restrict__ scores,
                                                 uint64_t* __restrict__ missed_keys,
                                                 int32_t* __restrict__ missed_idx,
                                                 int32_t* __restrict__ missed_size) {
  __shared__ uint32_t s_rows[kBlock / 64][64];
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wv = threadIdx.x >> 6;
  const uint64_t wave_base = (uint64_t)blockIdx.x * kBlock + wv * 64;
  const uint64_t i = wave_base + lane;
  bool found = false;
  const uint8_t* src = nullptr;
  uint64_t k = 0;
  if (i < n) {
    k = keys[i];
    if (!is_reserved(k)) {
      const uint64_t h = murmur3(k);
      const uint64_t gi = global_idx(t, h);
      const uint64_t b = gi >> t.bshift;
      const uint32_t start = (uint32_t)(gi & (t.B - 1));
      const int p = probe_find(t, b, start, key_digest(h), k);
      if (p >= 0) {
        found = true;
        src = row_ptr(t, b, (uint32_t)p);
        if (scores) scores[i] = t.scores[b * t.B + p];
      }
    }
    if (!MISSED && founds) founds[i] = found ? 1 : 0;
  }
  if (MISSED) {
    const bool miss = (i < n) && !found;
    const uint64_t m = __ballot(miss);
    const uint32_t cnt = __popcll(m);
    uint32_t base = 0;
    if (lane == 0 && cnt) base = atomicAdd(reinterpret_cast<uint32_t*>(missed_size), cnt);
    base = __shfl(base, 0);
    if (miss) {
      const uint32_t r = __popcll(m & ((1ull << lane) - 1));
      missed_keys[base + r] = k;
      missed_idx[base + r] = (int32_t)i;
    }
  }
  const uint64_t hm = __ballot(found);
  if (found) s_rows[wv][__popcll(hm & ((1ull << lane) - 1))] = lane;
  __syncthreads();
  const uint32_t rows = __popcll(hm);
  if (rows) wave_copy_rows<U>(rows, s_rows[wv], src, values, wave_base, t.row_bytes, false);
}

/* ------------------------------------------------------------------------ */
/* erase                                                                     */
/* ------------------------------------------------------------------------ */

// include/kernels/remove_kernel/remove_kernel.h:31-113: every digest group
// is scanned (no early stop); a matching key becomes RECLAIM with score 0
// and the reclaim digest.  The slot is claimed with a CAS so that a key
// repeated in one batch is erased once, as if applied in batch order.
__global__ __launch_bounds__(kBlock) void k_erase(TableView t, const uint64_t* __restrict__ keys,
                                                  uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const uint64_t k = keys[i];
  if (is_reserved(k)) return;
  const uint32_t B = t.B;
  const uint64_t h = murmur3(k);
  const uint64_t gi = global_idx(t, h);
  const uint64_t b = gi >> t.bshift;
  const uint32_t start = (uint32_t)(gi & (B - 1));
  const uint32_t rep = key_digest(h) * 0x01010101u;
  uint8_t* dg = t.digests + b * B;
  uint64_t* ks = t.keys + b * B;
  const uint32_t a = start & ~3u;
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t w = *reinterpret_cast<const uint32_t*>(dg + g);
    uint32_t m = eq_bytes4(w, rep);
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      if (ks[g + j] == k) {
        if (atomicCAS(reinterpret_cast<unsigned long long*>(ks + g + j),
                      (unsigned long long)k, (unsigned long long)kReclaimKey) ==
            (unsigned long long)k) {
          t.scores[b * B + g + j] = 0;
          dg[g + j] = kReclaimDigest;
          atomicSub(t.bsize + b, 1);
        }
        break;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* route + apply (all mutating batch operations)                            */
/* ------------------------------------------------------------------------ */

__global__ __launch_bounds__(kBlock) void k_route(TableView t, const uint64_t* __restrict__ keys,
                                                  uint64_t n, uint32_t* __restrict__ cnt,
                                                  uint32_t* __restrict__ pend, uint32_t P,
                                                  uint32_t* __restrict__ heavy,
                                                  uint32_t* __restrict__ ctrl,
                                                  uint32_t* __restrict__ ctrl_next) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i == 0) ctrl_next[0] = 0;
  if (i >= n) return;
  const uint64_t k = keys[i];
  if (is_reserved(k)) return;
  const uint64_t gi = global_idx(t, murmur3(k));
  const uint64_t b = gi >> t.bshift;
  const uint32_t r = atomicAdd(cnt + b, 1u);
  if (r < P) pend[b * P + r] = (uint32_t)i;
  if (r == P) heavy[atomicAdd(ctrl, 1u)] = (uint32_t)b;
}

enum Outcome : uint32_t { R_DUP = 1, R_EMPTY = 2, R_RECLAIMED = 3, R_EVICT = 4, R_REFUSED = 5 };

// State of one bucket held by a 16-lane group: lane l owns slots l + 16*j
// (j = 0..7).  Only the owner lane ever reads or writes a slot's key, score
// and digest, so the slots need no register cache: the owner re-reads them
// (same-thread ordering makes its own earlier writes visible).  The eight
// digests of a lane are kept packed in two words.
struct Bucket16 {
  uint64_t b;
  uint64_t base;  // b * B
  uint32_t l;
  uint32_t dg0, dg1;  // digest of slot l+16j in byte j (dg0: j<4, dg1: j>=4)
  int32_t bsz, bsz0;
};

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
  S.b = b;
  S.base = b * (uint64_t)t.B;
  S.l = l;
  const uint8_t* dg = t.digests + S.base + l;
  S.dg0 = (uint32_t)dg[0] | ((uint32_t)dg[16] << 8) | ((uint32_t)dg[32] << 16) |
          ((uint32_t)dg[48] << 24);
  S.dg1 = (uint32_t)dg[64] | ((uint32_t)dg[80] << 8) | ((uint32_t)dg[96] << 16) |
          ((uint32_t)dg[112] << 24);
  S.bsz = S.bsz0 = t.bsize[b];
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
__device__ __forceinline__ void accum_units(uint8_t* dst, const uint8_t* delta, uint32_t bytes,
                                            uint32_t r, uint32_t nl) {
  V* d = reinterpret_cast<V*>(dst);
  const V* s = reinterpret_cast<const V*>(delta);
  const uint32_t cntv = bytes / sizeof(V);
  for (uint32_t u = r; u < cntv; u += nl) {
    V v = s[u];
    v += d[u];  // `val = delta; val += dst` (accum_or_assign_kernel.h:41-49)
    d[u] = v;
  }
}

__device__ __forceinline__ void accum_row(uint8_t* dst, const uint8_t* delta, uint32_t bytes,
                                          int vt, uint32_t r, uint32_t nl) {
  switch (vt) {
    case 0: accum_units<float>(dst, delta, bytes, r, nl); break;           // f32
    case 8: accum_units<int32_t>(dst, delta, bytes, r, nl); break;         // i32
    case 10: case 11: accum_units<uint64_t>(dst, delta, bytes, r, nl); break;  // i64/u64
    default: break;
  }
}

// Applies batch key `i` to the bucket held by the group (all 16 lanes call
// this with the same i).  Restates, for one key, the reference kernels
// insert_or_assign_kernel.h:76-303 (unique keys) and find_and_lock
// (find_utils.h:94-227) with its callers (non-unique keys and accum).
template <int OP, int U>
__device__ __forceinline__ void apply_key(const TableView& t, Bucket16& S, const ApplyArgs& a,
                                          uint64_t i) {
  constexpr int SPL = 8;
  const uint32_t B = t.B;
  const uint32_t l = S.l;
  const uint64_t k = a.keys[i];
  const bool has_in = a.in_scores != nullptr;
  const uint64_t in = has_in ? a.in_scores[i] : 0;
  const uint64_t h = murmur3(k);
  const uint64_t gi = global_idx(t, h);
  const uint32_t start = (uint32_t)(gi & (B - 1));
  const uint32_t d = key_digest(h);
  const uint64_t des = score_desired(a.sc, has_in, in);
  const uint64_t* kp = t.keys + S.base + l;

  // 1. Is the key present?  Candidates are digest matches.
  const uint32_t a4 = start & ~3u;
  uint32_t best = kNone;
#pragma unroll
  for (int j = 0; j < SPL; j++) {
    if (dg_of(S, j) == d && kp[16 * j] == k) {
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
    return;  // absent keys are a no-op
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
      const uint64_t* sp = t.scores + S.base + l;
      uint64_t ms = kMaxScore, mk = 0;
      uint32_t mr = kNone, mp = start;
#pragma unroll
      for (int j = 0; j < SPL; j++) {
        const uint32_t p = l + 16 * j;
        const uint64_t kj = kp[16 * j];
        const uint64_t sj = sp[16 * j];
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
        if (l == (start & 15u)) kk = t.keys[S.base + start];
        mk = shfl_u64(kk, (int)(start & 15u), 16);
      }
      if (des < ms) {
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
  const uint8_t* in_row = a.in_values ? a.in_values + i * (uint64_t)R : nullptr;
  if (OP == OP_ACCUM_OR_ASSIGN) {
    if (res == R_REFUSED) return;
    const bool is_accum = a.accum_flags[i] != 0;
    if ((is_accum && res != R_DUP) || (!is_accum && res == R_DUP)) return;
  }
  if (res == R_REFUSED) {
    if (OP == OP_INSERT_AND_EVICT) {
      uint64_t j = 0;
      if (l == 0) j = atomicAdd(reinterpret_cast<unsigned long long*>(a.ev_counter), 1ull);
      j = shfl_u64(j, 0, 16);
      if (l == 0) {
        a.ev_keys[j] = k;
        if (a.ev_scores) a.ev_scores[j] = des;
      }
      copy_units<U>(a.ev_values + j * R, in_row, R, l, 16);
    }
    return;
  }
  uint8_t* trow = row_ptr(t, S.b, pos);
  if (OP == OP_INSERT_AND_EVICT && res == R_EVICT) {
    uint64_t j = 0;
    if (l == 0) j = atomicAdd(reinterpret_cast<unsigned long long*>(a.ev_counter), 1ull);
    j = shfl_u64(j, 0, 16);
    if (l == 0) {
      a.ev_keys[j] = victim_key;
      if (a.ev_scores) a.ev_scores[j] = victim_score;
    }
    copy_units<U>(a.ev_values + j * R, trow, R, l, 16);
  }
  if (res == R_EMPTY || res == R_RECLAIMED) S.bsz++;

  if (res == R_DUP) {
    if (OP == OP_FIND_OR_INSERT) {
      copy_units<U>(a.io_values + i * (uint64_t)R, trow, R, l, 16);
    } else if (OP == OP_ACCUM_OR_ASSIGN) {
      accum_row(trow, in_row, R, a.value_type, l, 16);
    } else if (OP != OP_ASSIGN_SCORES) {
      copy_units<U>(trow, in_row, R, l, 16);
    }
  } else {
    copy_units<U>(trow, in_row, R, l, 16);
  }

  const uint32_t owner = pos & 15u, jj = pos >> 4;
  if (l == owner) {
    uint64_t old = 0;
    if (res == R_DUP && (a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu))
      old = t.scores[S.base + pos];
    bool w;
    uint64_t ns;
    if (OP == OP_ASSIGN_SCORES) {
      ns = score_wo_missed(a.sc, has_in, in, old, &w);
    } else if (res == R_DUP) {
      ns = score_hit(a.sc, has_in, in, des, old, &w);
    } else {
      ns = score_new(a.sc, has_in, in, des, old, &w);
    }
    if (w) {
      t.scores[S.base + pos] = ns;
      if (res != R_DUP) {
        t.digests[S.base + pos] = (uint8_t)d;
        dg_set(S, jj, d);
      }
    }
    if (res != R_DUP) t.keys[S.base + pos] = k;
  }
}

__device__ __forceinline__ void bucket_finish(const TableView& t, Bucket16& S) {
  if (S.l == 0 && S.bsz != S.bsz0) t.bsize[S.b] = S.bsz;
}

// Pending-count word after the lane-per-bucket pass: bits 0-15 hold the
// number of routed keys, bit 31 marks a bucket handed to the 16-lane pass
// and bits 16-30 the sorted position it resumes from.
constexpr uint32_t kDefer = 0x80000000u;
constexpr uint32_t kLightMax = 16;  // keys per bucket the lane pass holds

// Row tasks queued by a wave of the lane pass, executed cooperatively.  The
// destination pointer's top bit marks an accumulate task.
constexpr uint32_t kTaskCap = 256;
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
    const T* s[Q];
    T* d[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
      const uint32_t r = r0 + q * rpi + lane / lpr;
      const bool ok = r < ntask;
      uint64_t dp = ok ? s_dst[r] : 0;
      const uint64_t sp = ok ? s_src[r] : any_src;
      if (dp & kAccumBit) {
        accum_row(reinterpret_cast<uint8_t*>((uintptr_t)(dp & ~kAccumBit)),
                  reinterpret_cast<const uint8_t*>((uintptr_t)sp), row_bytes, vt, sub, lpr);
        dp = 0;
      }
      s[q] = reinterpret_cast<const T*>((uintptr_t)(dp ? sp : any_src));
      d[q] = reinterpret_cast<T*>((uintptr_t)dp);
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
  const uint8_t* dg = t.digests + base;
  const uint64_t* ks = t.keys + base;
  const uint32_t a = start & ~3u;
  const uint32_t rep = d * 0x01010101u;
  const uint32_t erep = (uint32_t)kEmptyDigest * 0x01010101u;
  uint32_t cur = kNone;
  uint4 chunk = make_uint4(0, 0, 0, 0);
  for (uint32_t off = 0; off < B + 4; off += 4) {
    const uint32_t g = (a + off) & (B - 1);
    const uint32_t c = g >> 4;
    if (c != cur) {
      chunk = *reinterpret_cast<const uint4*>(dg + (c << 4));
      cur = c;
    }
    const uint32_t wi = (g >> 2) & 3;
    const uint32_t w = wi == 0 ? chunk.x : wi == 1 ? chunk.y : wi == 2 ? chunk.z : chunk.w;
    uint32_t m = eq_bytes4(w, rep);
    while (m) {
      const uint32_t j = __builtin_ctz(m);
      m &= m - 1;
      if (ks[g + j] == k) {
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

// Lane-per-bucket pass: each lane owns one bucket with 1..16 routed keys and
// applies them in batch order as long as no eviction is needed (the key is
// present, or an EMPTY slot exists).  At the first key that would evict or be
// refused the lane stops and hands the rest of the bucket to the 16-lane
// pass.  Metadata is updated in place by the owning lane; row movements are
// queued in LDS and executed cooperatively by the wave: at the end for
// insert_or_assign / insert_and_evict, after every step for operations that
// read table rows (find_or_insert, accum_or_assign) so that a later key of
// the same batch sees an earlier key's row.
template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_apply_lpb(TableView t, ApplyArgs a,
                                                      uint32_t* __restrict__ cnt,
                                                      const uint32_t* __restrict__ pend,
                                                      uint32_t P) {
  __shared__ uint64_t s_src[kBlock / 64][kTaskCap];
  __shared__ uint64_t s_dst[kBlock / 64][kTaskCap];
  constexpr bool kStepFlush = OP == OP_FIND_OR_INSERT || OP == OP_ACCUM_OR_ASSIGN;
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint64_t b = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const uint32_t B = t.B;
  const uint32_t R = t.row_bytes;
  uint32_t c = 0;
  if (b < t.buckets) c = cnt[b];
  const bool light = c > 0 && c <= P && c <= kLightMax;
  uint32_t e[kLightMax];
#pragma unroll
  for (uint32_t q = 0; q < kLightMax; q++) e[q] = (light && q < c) ? pend[b * P + q] + 1u : 0u;
  const uint64_t base = b * (uint64_t)B;
  int32_t bsz = light ? t.bsize[b] : 0;
  const int32_t bsz0 = bsz;
  uint32_t maxc = light ? c : 0;
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint32_t o = __shfl_xor(maxc, m, 64);
    maxc = o > maxc ? o : maxc;
  }
  // Slots whose row is already queued for writing in this call; a second
  // write to one of them flushes the queue first so that the later key wins.
  uint32_t wr0 = 0, wr1 = 0, wr2 = 0, wr3 = 0;
  bool active = light;
  uint32_t stop = c;
  uint32_t ntask = 0;
  const bool has_in = a.in_scores != nullptr;
  // One-step-ahead prefetch of the next key (batch order).
  uint32_t m_next = kNone;
#pragma unroll
  for (uint32_t q = 0; q < kLightMax; q++)
    if (e[q] > 0 && e[q] < m_next) m_next = e[q];
  uint64_t k_next = 0, in_next = 0;
  if (light) {
    k_next = a.keys[m_next - 1];
    if (has_in) in_next = a.in_scores[m_next - 1];
  }
  for (uint32_t step = 0; step < maxc; step++) {
    uint64_t src = 0, dst = 0;
    bool conflict = false;
    if (active && step < c) {
      const uint32_t m = m_next;
      const uint64_t i = m - 1;
      const uint64_t k = k_next;
      const uint64_t in = in_next;
      m_next = kNone;
#pragma unroll
      for (uint32_t q = 0; q < kLightMax; q++)
        if (e[q] > m && e[q] < m_next) m_next = e[q];
      if (m_next != kNone) {
        k_next = a.keys[m_next - 1];
        if (has_in) in_next = a.in_scores[m_next - 1];
      }
      const uint64_t h = murmur3(k);
      const uint64_t gi = global_idx(t, h);
      const uint32_t start = (uint32_t)(gi & (B - 1));
      const uint32_t d = key_digest(h);
      int dup = 0;
      const bool may_insert = OP != OP_ASSIGN_SCORES;
      const int p = probe_upsert(t, base, start, d, k, may_insert && bsz < (int32_t)B, &dup);
      if (p < 0 && may_insert) {
        active = false;  // eviction path: hand over from this key on
        stop = step;
      } else if (p >= 0) {
        const uint64_t des = score_desired(a.sc, has_in, in);
        bool apply = true;
        if (OP == OP_ACCUM_OR_ASSIGN) {
          const bool is_accum = a.accum_flags[i] != 0;
          apply = is_accum == (dup != 0);
        }
        if (apply) {
          uint8_t* trow = row_ptr(t, b, (uint32_t)p);
          const uint8_t* in_row = a.in_values ? a.in_values + i * (uint64_t)R : nullptr;
          bool w;
          if (dup) {
            uint64_t old = 0;
            if (a.sc.strategy == kLfu || a.sc.strategy == kEpochLfu) old = t.scores[base + p];
            const uint64_t ns = OP == OP_ASSIGN_SCORES
                                    ? score_wo_missed(a.sc, has_in, in, old, &w)
                                    : score_hit(a.sc, has_in, in, des, old, &w);
            if (w) t.scores[base + p] = ns;
            if (OP == OP_FIND_OR_INSERT) {
              src = (uint64_t)(uintptr_t)trow;
              dst = (uint64_t)(uintptr_t)(a.io_values + i * (uint64_t)R);
            } else if (OP == OP_ACCUM_OR_ASSIGN) {
              src = (uint64_t)(uintptr_t)in_row;
              dst = (uint64_t)(uintptr_t)trow | kAccumBit;
            } else if (OP != OP_ASSIGN_SCORES) {
              src = (uint64_t)(uintptr_t)in_row;
              dst = (uint64_t)(uintptr_t)trow;
            }
          } else {
            const uint64_t ns = score_new(a.sc, has_in, in, des, t.scores[base + p], &w);
            if (w) {
              t.scores[base + p] = ns;
              t.digests[base + p] = (uint8_t)d;
            }
            t.keys[base + p] = k;
            bsz++;
            src = (uint64_t)(uintptr_t)in_row;
            dst = (uint64_t)(uintptr_t)trow;
          }
          if (!kStepFlush && dst) {
            const uint32_t bit = 1u << (p & 31);
            const uint32_t wq = (uint32_t)p >> 5;
            const uint32_t cur = wq == 0 ? wr0 : wq == 1 ? wr1 : wq == 2 ? wr2 : wr3;
            conflict = (cur & bit) != 0;
            wr0 |= wq == 0 ? bit : 0u;
            wr1 |= wq == 1 ? bit : 0u;
            wr2 |= wq == 2 ? bit : 0u;
            wr3 |= wq == 3 ? bit : 0u;
          }
        }
      }
    }
    // Queue this step's row tasks; flush first when full or when a slot is
    // written twice.
    const uint64_t tm = __ballot(dst != 0);
    const uint32_t nnew = __popcll(tm);
    if (kStepFlush || __ballot(conflict) != 0 || ntask + nnew > kTaskCap) {
      __builtin_amdgcn_wave_barrier();
      if (ntask) flush_tasks<U, 2>(ntask, s_src[wv], s_dst[wv], R, a.value_type);
      ntask = 0;
      if (kStepFlush) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      __builtin_amdgcn_wave_barrier();
    }
    if (dst) {
      const uint32_t r = ntask + __popcll(tm & ((1ull << lane) - 1));
      s_src[wv][r] = src;
      s_dst[wv][r] = dst;
    }
    ntask += nnew;
    if (kStepFlush) {
      __builtin_amdgcn_wave_barrier();
      if (ntask) flush_tasks<U, 2>(ntask, s_src[wv], s_dst[wv], R, a.value_type);
      ntask = 0;
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      __builtin_amdgcn_wave_barrier();
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (ntask) flush_tasks<U, 8>(ntask, s_src[wv], s_dst[wv], R, a.value_type);
  if (light) {
    if (bsz != bsz0) t.bsize[b] = bsz;
    cnt[b] = stop == c ? 0u : (kDefer | (stop << 16) | c);
  }
}

// One 16-lane group per bucket the lane pass did not finish: buckets with
// more than 16 (and at most P) routed keys, and buckets handed over at their
// first eviction.
template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_apply(TableView t, ApplyArgs a,
                                                  uint32_t* __restrict__ cnt,
                                                  const uint32_t* __restrict__ pend, uint32_t P) {
  const uint64_t gid = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) >> 4;
  const uint32_t l = threadIdx.x & 15;
  if (gid >= t.buckets) return;
  const uint32_t raw = cnt[gid];
  if (raw == 0) return;
  const uint32_t c = raw & 0xFFFFu;
  if (c > P) return;
  const uint32_t first = (raw & kDefer) ? (raw >> 16) & 0x7FFFu : 0u;
  // Pending indices of this bucket, up to 4 per lane, stored as index + 1.
  uint32_t e[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t s = l + 16 * q;
    e[q] = s < c ? pend[gid * P + s] + 1u : 0u;
  }
  Bucket16 S;
  bucket_load(t, S, gid, l);
  uint32_t last = 0;
  for (uint32_t step = 0; step < c; step++) {
    uint32_t m = kNone;
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (e[q] > last && e[q] < m) m = e[q];
    m = group_min_u32(m);
    last = m;
    if (step >= first) apply_key<OP, U>(t, S, a, (uint64_t)(m - 1));
  }
  bucket_finish(t, S);
  if (l == 0) cnt[gid] = 0;
}

// Buckets with more than P routed keys: one group per bucket walks the batch
// in index order.
template <int OP, int U>
__global__ __launch_bounds__(kBlock) void k_apply_heavy(TableView t, ApplyArgs a,
                                                        uint32_t* __restrict__ cnt,
                                                        const uint32_t* __restrict__ heavy,
                                                        const uint32_t* __restrict__ ctrl) {
  const uint32_t nheavy = ctrl[0];
  const uint64_t groups = ((uint64_t)gridDim.x * kBlock) >> 4;
  const uint32_t l = threadIdx.x & 15;
  const uint32_t gslot = (threadIdx.x >> 4) & 3;  // group within the wave
  for (uint64_t g = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) >> 4; g < nheavy;
       g += groups) {
    const uint64_t b = heavy[g];
    Bucket16 S;
    bucket_load(t, S, b, l);
    for (uint64_t base = 0; base < a.n; base += 16) {
      const uint64_t i = base + l;
      bool mine = false;
      if (i < a.n) {
        const uint64_t k = a.keys[i];
        mine = !is_reserved(k) && (global_idx(t, murmur3(k)) >> t.bshift) == b;
      }
      uint32_t mask = (uint32_t)(__ballot(mine) >> (16 * gslot)) & 0xFFFFu;
      while (mask) {
        const uint32_t q = __builtin_ctz(mask);
        mask &= mask - 1;
        apply_key<OP, U>(t, S, a, base + q);
      }
    }
    bucket_finish(t, S);
    if (l == 0) cnt[b] = 0;
  }
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
  const bool live = s < n && !is_reserved(t.keys[offset + s]);
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
  if (s < n) k = t.keys[offset + s];
  const bool live = s < n && !is_reserved(k);
  const uint64_t m = __ballot(live);
  if (lane == 0) w[wv] = __popcll(m);
  __syncthreads();
  uint32_t wbase = block_off[blockIdx.x];
  for (uint32_t q = 0; q < wv; q++) wbase += w[q];
  const uint32_t r = __popcll(m & ((1ull << lane) - 1));
  const uint8_t* src = nullptr;
  if (live) {
    const uint64_t g = offset + s;
    const uint64_t b = g >> t.bshift;
    const uint32_t slot = (uint32_t)(g & (t.B - 1));
    out_keys[wbase + r] = k;
    if (out_scores) out_scores[wbase + r] = t.scores[g];
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
        const T* sr = reinterpret_cast<const T*>((uintptr_t)sp);
        T* dr = reinterpret_cast<T*>(out_vals + (uint64_t)(wbase + rr) * t.row_bytes);
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

__device__ __forceinline__ void thread_copy(uint8_t* dst, const uint8_t* src, uint32_t bytes,
                                            int unit) {
  copy_row(dst, src, bytes, unit, 0, 1);
}

// include/kernels/rehash_kernel/rehash_kernel.h:69-135 (backward-shift
// defragmentation after a key leaves bucket b).
__device__ void rehash_defrag(const TableView& t, uint64_t b, uint32_t remove_pos,
                              uint64_t old_cap, int unit) {
  const uint32_t B = t.B;
  const uint64_t base = b * B;
  uint32_t offset = 1;
  while (offset < B) {
    const uint32_t cur = (remove_pos + offset) % B;
    const uint64_t ck = t.keys[base + cur];
    if (ck == kEmptyKey) break;
    const uint64_t h = murmur3(ck);
    const uint64_t sp = (h % old_cap) % B;
    if ((sp <= remove_pos && remove_pos < cur) || (cur < sp && sp <= remove_pos) ||
        (remove_pos < cur && cur < sp)) {
      t.keys[base + remove_pos] = ck;
      t.scores[base + remove_pos] = t.scores[base + cur];
      t.digests[base + remove_pos] = (uint8_t)key_digest(h);
      thread_copy(row_ptr(t, b, remove_pos), row_ptr(t, b, cur), t.row_bytes, unit);
      t.keys[base + cur] = kEmptyKey;
      t.digests[base + cur] = kEmptyDigest;
      remove_pos = cur;
      offset = 1;
    } else {
      offset++;
    }
  }
}

// include/kernels/rehash_kernel/rehash_kernel.h:137-207: one thread per old
// bucket; keys whose bucket under the doubled capacity differs move to the
// first EMPTY slot (circular from their start) of bucket b + old_buckets.
__global__ __launch_bounds__(kBlock) void k_rehash(TableView t, uint64_t old_nb, int unit) {
  const uint64_t b = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (b >= old_nb) return;
  const uint32_t B = t.B;
  const uint64_t base = b * B;
  const uint64_t new_cap = t.capacity;
  uint32_t kp = 0;
  while (kp < B) {
    const uint64_t ck = t.keys[base + kp];
    if (ck == kEmptyKey || ck == kReclaimKey) {
      kp++;
      continue;
    }
    const uint64_t cs = t.scores[base + kp];
    const uint64_t h = murmur3(ck);
    const uint64_t ngi = h % new_cap;
    const uint64_t nbk = ngi / B;
    if (nbk == b) {
      kp++;
      continue;
    }
    const uint32_t nkp = (uint32_t)(ngi % B);
    const uint64_t nbase = nbk * B;
    for (uint32_t o = 0; o < B; o++) {
      const uint32_t cp = (nkp + o) % B;
      if (t.keys[nbase + cp] == kEmptyKey) {
        t.keys[nbase + cp] = ck;
        t.scores[nbase + cp] = cs;
        t.digests[nbase + cp] = (uint8_t)key_digest(h);
        t.bsize[nbk]++;
        thread_copy(row_ptr(t, nbk, cp), row_ptr(t, b, kp), t.row_bytes, unit);
        break;
      }
    }
    t.keys[base + kp] = kEmptyKey;
    t.digests[base + kp] = kEmptyDigest;
    t.bsize[b]--;
    rehash_defrag(t, b, kp, old_nb * B, unit);
    kp = 0;
  }
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
  const dim3 g(grid_for(n, kBlock, 1ull << 31)), b(kBlock);
  switch (unit) {
    case 16: hipLaunchKernelGGL((k_find<16, MISSED>), g, b, 0, s, t, keys, n, values, founds, scores, mk, mi, ms); break;
    case 8: hipLaunchKernelGGL((k_find<8, MISSED>), g, b, 0, s, t, keys, n, values, founds, scores, mk, mi, ms); break;
    case 4: hipLaunchKernelGGL((k_find<4, MISSED>), g, b, 0, s, t, keys, n, values, founds, scores, mk, mi, ms); break;
    case 2: hipLaunchKernelGGL((k_find<2, MISSED>), g, b, 0, s, t, keys, n, values, founds, scores, mk, mi, ms); break;
    default: hipLaunchKernelGGL((k_find<1, MISSED>), g, b, 0, s, t, keys, n, values, founds, scores, mk, mi, ms); break;
  }
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
static void apply_op(const TableView& t, const ApplyArgs& a, RouteScratch& rs, int parity,
                     hipStream_t s) {
  uint32_t* ctrl = rs.ctrl + 16 * parity;
  uint32_t* ctrl_next = rs.ctrl + 16 * (1 - parity);
  hipLaunchKernelGGL(k_route, dim3(grid_for(a.n, kBlock, 1ull << 31)), dim3(kBlock), 0, s, t,
                     a.keys, a.n, rs.cnt, rs.pend, rs.P, rs.heavy, ctrl, ctrl_next);
  const dim3 gl(grid_for(t.buckets, kBlock, 1ull << 31)), bl(kBlock);
  const dim3 gg(grid_for(t.buckets * 16, kBlock, 1ull << 31));
  const uint64_t max_heavy = a.n / (rs.P + 1) + 1;
  const dim3 gh(grid_for(max_heavy * 16, kBlock, 2048));
  const bool heavy = a.n > rs.P;
#define HKV_APPLY_U(UU)                                                                  \
  hipLaunchKernelGGL((k_apply_lpb<OP, UU>), gl, bl, 0, s, t, a, rs.cnt, rs.pend, rs.P);  \
  hipLaunchKernelGGL((k_apply<OP, UU>), gg, bl, 0, s, t, a, rs.cnt, rs.pend, rs.P);      \
  if (heavy)                                                                             \
    hipLaunchKernelGGL((k_apply_heavy<OP, UU>), gh, bl, 0, s, t, a, rs.cnt, rs.heavy, ctrl);
  switch (a.unit) {
    case 16: HKV_APPLY_U(16); break;
    case 8: HKV_APPLY_U(8); break;
    case 4: HKV_APPLY_U(4); break;
    case 2: HKV_APPLY_U(2); break;
    default: HKV_APPLY_U(1); break;
  }
#undef HKV_APPLY_U
}

void launch_apply(const TableView& t, int op, const ApplyArgs& a, RouteScratch& rs, int parity,
                  hipStream_t s) {
  switch (op) {
    case OP_INSERT_OR_ASSIGN: apply_op<OP_INSERT_OR_ASSIGN>(t, a, rs, parity, s); break;
    case OP_FIND_OR_INSERT: apply_op<OP_FIND_OR_INSERT>(t, a, rs, parity, s); break;
    case OP_INSERT_AND_EVICT: apply_op<OP_INSERT_AND_EVICT>(t, a, rs, parity, s); break;
    case OP_ACCUM_OR_ASSIGN: apply_op<OP_ACCUM_OR_ASSIGN>(t, a, rs, parity, s); break;
    default: apply_op<OP_ASSIGN_SCORES>(t, a, rs, parity, s); break;
  }
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

void launch_rehash(const TableView& t, uint64_t old_nb, int unit, hipStream_t s) {
  hipLaunchKernelGGL(k_rehash, dim3(grid_for(old_nb, kBlock, 1ull << 31)), dim3(kBlock), 0, s, t,
                     old_nb, unit);
}

}  // namespace hkv
