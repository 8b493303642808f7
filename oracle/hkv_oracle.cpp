/*
 * hkv_oracle.cpp -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Host C++ restatement of the HierarchicalKV-ascend table algorithm.  Each
 * routine restates one reference kernel for a single key, literally (same
 * probe order, same lane tournaments, same score functor arithmetic), and the
 * API routines apply a batch as if its keys ran one at a time in increasing
 * batch index.  Buckets are independent, so the optional multi-threaded mode
 * gives each host thread a contiguous bucket range; every thread still walks
 * the batch in index order, so results are identical to one thread.
 *
 * All citations are paths relative to the reference repository root.
 */
#include "hkv_oracle.h"

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t EMPTY_KEY = 0xFFFFFFFFFFFFFFFFull;    // include/types.h:63
constexpr uint64_t RECLAIM_KEY = 0xFFFFFFFFFFFFFFFEull;  // include/types.h:64
constexpr uint64_t LOCKED_KEY = 0xFFFFFFFFFFFFFFFDull;   // include/types.h:65
constexpr uint64_t RESERVED_MASK = 0xFFFFFFFFFFFFFFFCull;  // include/types.h:67
constexpr uint64_t MAX_SCORE = 0xFFFFFFFFFFFFFFFFull;    // include/types.h:70
constexpr uint64_t EMPTY_SCORE = 0;                      // include/types.h:71
constexpr uint64_t IGNORED_EPOCH = 0xFFFFFFFFFFFFFFFFull;  // include/types.h:72
constexpr uint64_t SCORE_MASK = 0xFFFFFFFFull;  // include/score_functor.h:31
constexpr uint64_t EPOCH_MASK = 0xFFFFFFFF00000000ull;  // score_functor.h:30
constexpr uint64_t SCORE32_MAX = 0xFFFFFFFFull;  // score_functor.h:32

enum { kLru = 0, kLfu = 1, kEpochLru = 2, kEpochLfu = 3, kCustomized = 4 };

// include/types.h:153-156
inline bool is_reserved(uint64_t k) { return (k & RESERVED_MASK) == RESERVED_MASK; }

// include/utils.h:52-60 (MurmurHash3 fmix64)
inline uint64_t murmur3(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

inline uint8_t digest_of(uint64_t k) { return (uint8_t)(murmur3(k) >> 32); }

// include/table.h:106-127 (magic-number divisor precomputation)
struct QuickDiv {
  uint64_t cap = 1, magic = 0, shift = 0;
  void init(uint64_t c) {
    cap = c;
    unsigned __int128 one = 1;
    uint64_t s = 0;
    for (s = 0; s < 64; s++)
      if ((one << s) >= c) break;
    unsigned __int128 m = ((one << 64) * ((one << s) - c)) / c + 1;
    magic = (uint64_t)m;
    shift = s - 1;
  }
  // include/utils.h:86-97
  uint64_t mod(uint64_t h) const {
    uint64_t q = (uint64_t)(((unsigned __int128)h * magic) >> 64);
    q = ((h - q) >> 1) + q;
    uint64_t d = q >> shift;
    return h - d * cap;
  }
};

inline int value_size(int vt) {
  switch (vt) {
    case HKVO_F32: case HKVO_I32: case HKVO_U32: return 4;
    case HKVO_F64: case HKVO_I64: case HKVO_U64: return 8;
    case HKVO_F16: case HKVO_BF16: case HKVO_I16: case HKVO_U16: return 2;
    case HKVO_I8: case HKVO_U8: return 1;
    default: return 0;
  }
}

/* ---- score functors: include/score_functor.h ----------------------------- */

// desired_when_missed: Lru :51-55, Lfu :117-121, EpochLru :216-224,
// EpochLfu :287-294, Customized :411-415.
uint64_t desired(int st, bool has_in, uint64_t in, uint64_t epoch, uint64_t clk) {
  switch (st) {
    case kLru: return clk;
    case kLfu: return MAX_SCORE;
    case kEpochLru:
      if (epoch == IGNORED_EPOCH && has_in) return in;
      return (epoch << 32) | ((clk >> 20) & SCORE_MASK);
    case kEpochLfu:
      if (epoch == IGNORED_EPOCH) return in;
      return (epoch << 32) | (in & SCORE_MASK);
    default: return in;
  }
}

// Saturating low-word add used by EpochLfu hits (score_functor.h:361-372).
inline uint64_t epochlfu_add(uint64_t old, uint64_t desired_v) {
  uint64_t lo = old & SCORE_MASK;
  if (SCORE32_MAX - lo > (desired_v & SCORE_MASK)) return lo + desired_v;
  return (desired_v & EPOCH_MASK) | SCORE32_MAX;
}

// Score written for a newly placed key: update_with_digest(new_insert=true)
// (Lru :67-82, Lfu :136-160, EpochLru :233-246, EpochLfu :308-333,
// Customized :424-437).  `written` is false when the functor writes nothing.
uint64_t score_new(int st, bool has_in, uint64_t in, uint64_t des, uint64_t old,
                   bool* written) {
  *written = true;
  if (st == kLfu) {
    if (!has_in) { *written = false; return old; }
    return in;
  }
  return des;
}

// Score written for a key already present: update_score_only(new=false) /
// update_with_digest(new=false) (Lfu :162-183 adds the input, EpochLfu
// :335-355 saturates, the others store `desired`).
uint64_t score_hit(int st, bool has_in, uint64_t in, uint64_t des, uint64_t old,
                   bool* written) {
  *written = true;
  switch (st) {
    case kLfu:
      if (!has_in) { *written = false; return old; }
      return in + old;
    case kEpochLfu: return epochlfu_add(old, des);
    default: return des;
  }
}

// update_without_missed (assign_scores): Lru :96-111, Lfu :185-210,
// EpochLru :266-281, EpochLfu :374-405, Customized :462-477.
uint64_t score_wo_missed(int st, bool has_in, uint64_t in, uint64_t epoch,
                         uint64_t clk, uint64_t old, bool* written) {
  *written = true;
  switch (st) {
    case kLru: return clk;
    case kLfu:
      if (!has_in) { *written = false; return old; }
      return in + old;
    case kEpochLru: return (epoch << 32) | ((clk >> 20) & SCORE_MASK);
    case kEpochLfu: {
      if (!has_in) { *written = false; return old; }
      uint64_t lo = old & SCORE_MASK;
      if (SCORE32_MAX - lo > (in & SCORE_MASK))
        return lo + ((epoch << 32) | (in & SCORE_MASK));
      return (epoch << 32) | SCORE32_MAX;
    }
    default:
      if (!has_in) { *written = false; return old; }
      return in;
  }
}

enum Res { R_ILLEGAL, R_DUP, R_EMPTY, R_RECLAIMED, R_EVICT, R_REFUSED };

struct Loc {
  Res res = R_ILLEGAL;
  uint32_t pos = 0;
  uint64_t victim_key = 0;    // key that occupied `pos` before an eviction
  uint64_t victim_score = 0;  // the tournament's minimum score
};

// Which reference kernel family resolves a key: the 16-lane digest kernels
// (unique keys) or the 32-lane find_and_lock tiles (non-unique keys and
// accum_or_assign).
enum Rule { RULE_DIGEST16 = 0, RULE_TILE32 = 1 };

enum Op {
  OP_INSERT_OR_ASSIGN, OP_FIND_OR_INSERT, OP_INSERT_AND_EVICT, OP_ACCUM,
  OP_FIND_OR_INSERT_PTR,  // pointer overload: slots recorded, no row moves
};
constexpr uint64_t SLOT_FOUND = 1ull << 63;

struct Record {
  uint64_t idx;
  uint64_t key, score;
  std::vector<uint8_t> row;
};

}  // namespace

struct hkvo_table {
  uint64_t init_cap = 0, max_cap = 0, B = 128, dim = 0, nb = 0, C = 0;
  int vtype = HKVO_F32, esize = 4, strategy = kLru;
  float max_lf = 0.5f;
  uint32_t bshift = 7;
  QuickDiv qd;
  bool reach_max = false;
  uint64_t epoch = IGNORED_EPOCH;
  int threads = 1;
  // Pointer find_or_insert: slot word per batch index (global slot + 1, with
  // SLOT_FOUND), and whether claimed / found slots stay LOCKED for the rest
  // of the batch (the unique-key kernel holds its locks until the batch ends,
  // find_or_insert_ptr_kernel_v2.h:38-303).
  uint64_t* slot_out = nullptr;
  bool lock_batch = false;
  uint8_t empty_d = 0, reclaim_d = 0;
  size_t row = 0;
  std::vector<uint8_t> dg;
  std::vector<uint64_t> keys, scores;
  std::vector<int32_t> bsize;
  std::vector<uint8_t> vals;

  uint8_t* rowp(uint64_t b, uint32_t s) { return vals.data() + (b * B + s) * row; }

  void init_buckets(uint64_t from, uint64_t to) {
    // include/kernels/init_table_kernel/init_table_kernel.h:77-106
    for (uint64_t b = from; b < to; b++) {
      for (uint64_t s = 0; s < B; s++) {
        dg[b * B + s] = empty_d;
        keys[b * B + s] = EMPTY_KEY;
        scores[b * B + s] = EMPTY_SCORE;
      }
      bsize[b] = 0;
    }
  }

  void resize_storage() {
    dg.resize(C);
    keys.resize(C);
    scores.resize(C);
    bsize.resize(nb);
    vals.resize(C * row, 0);
  }

  /* ---- per-key probes ---------------------------------------------------- */

  // Digest probe of the unique-key kernels: 4-digest groups from align4(start)
  // with wrap, key match first, then the first EMPTY slot in circular order
  // (include/kernels/insert_or_assign_kernel/insert_or_assign_kernel.h:105-183).
  bool digest_probe(uint64_t b, uint32_t start, uint8_t d, uint64_t k, Loc& L) {
    const uint64_t base = b * B;
    const int32_t bs = bsize[b];
    const uint32_t a = start & ~3u;
    for (uint32_t off = 0; off < B + 4; off += 4) {
      const uint32_t g = (a + off) & (uint32_t)(B - 1);
      for (uint32_t j = 0; j < 4; j++) {
        const uint32_t p = g + j;
        if (dg[base + p] == d && keys[base + p] == k) {
          L.res = R_DUP;
          L.pos = p;
          return true;
        }
      }
      if ((uint64_t)bs == B) continue;
      for (uint32_t j = 0; j < 4; j++) {
        const uint32_t p = g + j;
        if (dg[base + p] != empty_d) continue;
        if (off == 0 && p < start) continue;
        if (keys[base + p] == EMPTY_KEY) {
          L.res = R_EMPTY;
          L.pos = p;
          return true;
        }
      }
    }
    return false;
  }

  // Eviction of the unique-key kernels: 16 lanes each scan slots lane,
  // lane+16, ... keeping the first strictly smaller score among keys that are
  // neither EMPTY nor LOCKED, then an xor butterfly (8,4,2,1) in which a lane
  // keeps its own candidate on ties; lane (batch index mod 16) decides
  // (insert_or_assign_kernel.h:193-271).
  void evict_digest16(uint64_t b, uint32_t start, uint64_t idx, uint64_t des,
                      Loc& L) {
    const uint64_t base = b * B;
    uint64_t ms[16];
    uint32_t mp[16];
    for (uint32_t l = 0; l < 16; l++) {
      ms[l] = MAX_SCORE;
      mp[l] = start;  // min_pos starts at the key's own start slot
      for (uint32_t p = l; p < B; p += 16) {
        const uint64_t s = scores[base + p];
        const uint64_t kk = keys[base + p];
        if (s < ms[l] && kk != LOCKED_KEY && kk != EMPTY_KEY) {
          ms[l] = s;
          mp[l] = p;
        }
      }
    }
    for (uint32_t off = 8; off > 0; off >>= 1) {
      uint64_t ns[16];
      uint32_t np[16];
      for (uint32_t l = 0; l < 16; l++) {
        const uint32_t o = l ^ off;
        if (ms[o] < ms[l]) { ns[l] = ms[o]; np[l] = mp[o]; }
        else { ns[l] = ms[l]; np[l] = mp[l]; }
      }
      std::memcpy(ms, ns, sizeof(ms));
      std::memcpy(mp, np, sizeof(mp));
    }
    const uint32_t me = (uint32_t)(idx & 15);
    if (des < ms[me]) {
      L.res = R_REFUSED;
      return;
    }
    const uint32_t p = mp[me];
    const uint64_t cur = keys[base + p];
    L.pos = p;
    L.victim_key = cur;
    L.victim_score = ms[me];
    L.res = (cur == RECLAIM_KEY) ? R_RECLAIMED : R_EVICT;
  }

  // find_and_lock phase 1: 32-lane tiles from the exact start slot; a tile
  // holding the key wins, else its first EMPTY slot in lane order
  // (include/find_utils.h:94-151).
  bool tile_probe(uint64_t b, uint32_t start, uint64_t k, Loc& L) {
    const uint64_t base = b * B;
    for (uint32_t t = 0; t < B; t += 32) {
      for (uint32_t lane = 0; lane < 32; lane++) {
        const uint32_t p = (uint32_t)((start + t + lane) % B);
        if (keys[base + p] == k) {
          L.res = R_DUP;
          L.pos = p;
          return true;
        }
      }
      for (uint32_t lane = 0; lane < 32; lane++) {
        const uint32_t p = (uint32_t)((start + t + lane) % B);
        if (keys[base + p] == EMPTY_KEY) {
          L.res = R_EMPTY;
          L.pos = p;
          return true;
        }
      }
    }
    return false;
  }

  // find_and_lock phase 2: each of 32 lanes scans start+lane, +32, ... keeping
  // the first strictly smaller score of a non-EMPTY key; the lowest lane whose
  // local minimum equals the global one supplies the victim
  // (include/find_utils.h:153-227).  When every score equals MAX_SCORE and the
  // key's desired score is MAX_SCORE the reference retries forever; this
  // restatement takes the start slot in that case.
  void evict_tile32(uint64_t b, uint32_t start, uint64_t des, Loc& L) {
    const uint64_t base = b * B;
    uint64_t gmin = MAX_SCORE;
    int best_lane = -1;
    uint32_t best_pos = 0;
    uint64_t lmin[32];
    uint32_t lpos[32];
    for (uint32_t lane = 0; lane < 32; lane++) {
      lmin[lane] = MAX_SCORE;
      lpos[lane] = 0;
      for (uint32_t t = 0; t < B; t += 32) {
        const uint32_t p = (uint32_t)((start + t + lane) % B);
        const uint64_t s = scores[base + p];
        if (s < lmin[lane] && keys[base + p] != EMPTY_KEY) {
          lmin[lane] = s;
          lpos[lane] = p;
        }
      }
      if (lmin[lane] < gmin) gmin = lmin[lane];
    }
    if (des < gmin) {
      L.res = R_REFUSED;
      return;
    }
    for (uint32_t lane = 0; lane < 32; lane++) {
      if (lmin[lane] <= gmin && lmin[lane] != MAX_SCORE) {
        best_lane = (int)lane;
        best_pos = lpos[lane];
        break;
      }
    }
    if (best_lane < 0) best_pos = start;
    const uint64_t cur = keys[base + best_pos];
    L.pos = best_pos;
    L.victim_key = cur;
    L.victim_score = gmin;
    L.res = (cur == RECLAIM_KEY) ? R_RECLAIMED : R_EVICT;
  }

  Loc locate(uint64_t b, uint32_t start, uint8_t d, uint64_t k, uint64_t idx,
             uint64_t des, Rule rule) {
    Loc L;
    if (rule == RULE_DIGEST16) {
      if (!digest_probe(b, start, d, k, L)) evict_digest16(b, start, idx, des, L);
    } else {
      if (!tile_probe(b, start, k, L)) evict_tile32(b, start, des, L);
    }
    return L;
  }

  // find_without_lock (include/find_utils.h:31-86): returns the slot or -1.
  int64_t find_slot(uint64_t b, uint32_t start, uint8_t d, uint64_t k) const {
    const uint64_t base = b * B;
    const uint32_t a = start & ~3u;
    for (uint32_t off = 0; off < B + 4; off += 4) {
      const uint32_t g = (a + off) & (uint32_t)(B - 1);
      for (uint32_t j = 0; j < 4; j++) {
        const uint32_t p = g + j;
        if (dg[base + p] == d && keys[base + p] == k) return p;
      }
      for (uint32_t j = 0; j < 4; j++) {
        const uint32_t p = g + j;
        if (dg[base + p] != empty_d) continue;
        if (off == 0 && p < start) continue;
        if (keys[base + p] == EMPTY_KEY) return -1;
      }
    }
    return -1;
  }

  void locate_key(uint64_t k, uint64_t* b, uint32_t* start, uint8_t* d) const {
    const uint64_t h = murmur3(k);
    const uint64_t gi = qd.mod(h);
    *b = gi >> bshift;
    *start = (uint32_t)(gi & (B - 1));
    *d = (uint8_t)(h >> 32);
  }

  /* ---- accumulate (one element), accum_or_assign_kernel.h:37-50 ---------- */
  void accum_row(uint8_t* dst, const uint8_t* delta) const {
    for (uint64_t j = 0; j < dim; j++) {
      switch (vtype) {
        case HKVO_F32: {
          float a, o;
          std::memcpy(&a, delta + 4 * j, 4);
          std::memcpy(&o, dst + 4 * j, 4);
          a += o;  // `val = src; val += dst`
          std::memcpy(dst + 4 * j, &a, 4);
          break;
        }
        case HKVO_I32: {
          int32_t a, o;
          std::memcpy(&a, delta + 4 * j, 4);
          std::memcpy(&o, dst + 4 * j, 4);
          a = (int32_t)((uint32_t)a + (uint32_t)o);
          std::memcpy(dst + 4 * j, &a, 4);
          break;
        }
        case HKVO_I64: case HKVO_U64: {
          uint64_t a, o;
          std::memcpy(&a, delta + 8 * j, 8);
          std::memcpy(&o, dst + 8 * j, 8);
          a += o;
          std::memcpy(dst + 8 * j, &a, 8);
          break;
        }
        default: break;
      }
    }
  }

  /* ---- one key of an insert-like batch ----------------------------------- */
  // Post-location effects follow the kernel family: unique-key kernels
  // (insert_or_assign_kernel.h:76-303, find_or_insert_kernel.h:71-331,
  // insert_and_evict_kernel.h:339-695) and find_and_lock callers
  // (insert_or_assign_kernel.h:1041-1124, find_or_insert_kernel.h:333-411,
  // accum_or_assign_kernel.h:52-155).
  void apply_one(Op op, Rule rule, int st, uint64_t i, const uint64_t* ks,
                 const uint8_t* in_vals, uint8_t* io_vals, const uint64_t* in_sc,
                 const uint8_t* accum, uint64_t clk, std::vector<Record>* recs) {
    const uint64_t k = ks[i];
    if (is_reserved(k)) return;
    const bool has_in = in_sc != nullptr;
    const uint64_t in = has_in ? in_sc[i] : 0;
    const uint64_t des = desired(st, has_in, in, epoch, clk);
    uint64_t b;
    uint32_t start;
    uint8_t d;
    locate_key(k, &b, &start, &d);
    Loc L = locate(b, start, d, k, i, des, rule);
    const uint64_t base = b * B;
    // A LOCKED victim is never taken: the reference kernels wait for it to
    // be unlocked (insert_or_assign_kernel.h:240-268, find_utils.h:160-224).
    if (L.res == R_EVICT && L.victim_key == LOCKED_KEY) L.res = R_REFUSED;

    if (op == OP_ACCUM) {
      if (L.res == R_REFUSED) return;
      const bool is_accum = accum[i] != 0;
      if ((is_accum && L.res != R_DUP) || (!is_accum && L.res == R_DUP)) return;
    }
    if (L.res == R_REFUSED) {
      if (op == OP_INSERT_AND_EVICT) {
        Record r;
        r.idx = i;
        r.key = k;
        r.score = des;
        r.row.assign(in_vals + i * row, in_vals + (i + 1) * row);
        recs->push_back(std::move(r));
      }
      return;
    }
    const uint32_t p = L.pos;
    if (L.res == R_EMPTY || L.res == R_RECLAIMED) bsize[b]++;
    if (op == OP_INSERT_AND_EVICT && L.res == R_EVICT) {
      Record r;
      r.idx = i;
      r.key = L.victim_key;
      r.score = L.victim_score;
      r.row.assign(rowp(b, p), rowp(b, p) + row);
      recs->push_back(std::move(r));
    }
    // Row movement.
    if (op == OP_FIND_OR_INSERT_PTR) {
      // none: the caller goes through the returned row address
    } else if (op == OP_FIND_OR_INSERT && L.res == R_DUP) {
      std::memcpy(io_vals + i * row, rowp(b, p), row);
    } else if (op == OP_ACCUM && L.res == R_DUP) {
      accum_row(rowp(b, p), in_vals + i * row);
    } else {
      std::memcpy(rowp(b, p), in_vals + i * row, row);
    }
    // Score and digest.
    bool w;
    if (L.res == R_DUP) {
      const uint64_t ns = score_hit(st, has_in, in, des, scores[base + p], &w);
      if (w) {
        scores[base + p] = ns;
        if (rule == RULE_TILE32) dg[base + p] = d;
      }
    } else {
      const uint64_t ns = score_new(st, has_in, in, des, scores[base + p], &w);
      if (w) {
        scores[base + p] = ns;
        dg[base + p] = d;
      }
    }
    keys[base + p] = (op == OP_FIND_OR_INSERT_PTR && lock_batch) ? LOCKED_KEY : k;
    if (op == OP_FIND_OR_INSERT_PTR)
      slot_out[i] = (base + p + 1) | (L.res == R_DUP ? SLOT_FOUND : 0);
  }

  /* ---- rehash, include/kernels/rehash_kernel/rehash_kernel.h:29-207 ------- */
  void defrag(uint64_t b, uint32_t remove_pos, uint64_t old_cap) {
    const uint64_t base = b * B;
    uint32_t offset = 1;
    while (offset < B) {
      const uint32_t cur = (uint32_t)((remove_pos + offset) % B);
      const uint64_t ck = keys[base + cur];
      if (ck == EMPTY_KEY) break;
      const uint64_t h = murmur3(ck);
      const uint64_t gi = h % old_cap;
      const uint64_t sp = gi % B;
      if ((sp <= remove_pos && remove_pos < cur) ||
          (cur < sp && sp <= remove_pos) ||
          (remove_pos < cur && cur < sp)) {
        keys[base + remove_pos] = ck;
        scores[base + remove_pos] = scores[base + cur];
        dg[base + remove_pos] = digest_of(ck);
        std::memcpy(rowp(b, remove_pos), rowp(b, cur), row);
        keys[base + cur] = EMPTY_KEY;
        dg[base + cur] = empty_d;
        remove_pos = cur;
        offset = 1;
      } else {
        offset++;
      }
    }
  }

  void rehash_bucket(uint64_t b, uint64_t old_nb) {
    const uint64_t base = b * B;
    const uint64_t new_cap = nb * B;
    uint32_t kp = 0;
    while (kp < B) {
      const uint64_t ck = keys[base + kp];
      const uint64_t cs = scores[base + kp];
      if (ck == EMPTY_KEY || ck == RECLAIM_KEY) { kp++; continue; }
      const uint64_t h = murmur3(ck);
      const uint64_t ngi = h % new_cap;
      const uint64_t nbk = ngi / B;
      if (nbk == b) { kp++; continue; }
      const uint32_t nkp = (uint32_t)(ngi % B);
      const uint64_t nbase = nbk * B;
      for (uint32_t o = 0; o < B; o++) {
        const uint32_t cp = (nkp + o) % B;
        if (keys[nbase + cp] == EMPTY_KEY) {
          keys[nbase + cp] = ck;
          scores[nbase + cp] = cs;
          dg[nbase + cp] = digest_of(ck);
          bsize[nbk]++;
          std::memcpy(rowp(nbk, cp), rowp(b, kp), row);
          break;
        }
      }
      keys[base + kp] = EMPTY_KEY;
      dg[base + kp] = empty_d;
      bsize[b]--;
      defrag(b, kp, old_nb * B);
      kp = 0;
    }
  }

  void double_capacity() {
    // include/table.h:360-377 plus rehash_kernel<FAST> over old buckets.
    const uint64_t old_nb = nb;
    nb *= 2;
    C = nb * B;
    resize_storage();
    init_buckets(old_nb, nb);
    qd.init(C);
    parallel_buckets(0, old_nb, [&](uint64_t lo, uint64_t hi) {
      for (uint64_t b = lo; b < hi; b++) rehash_bucket(b, old_nb);
    });
  }

  template <class F>
  void parallel_buckets(uint64_t lo, uint64_t hi, F&& fn) {
    const int T = std::max(1, threads);
    if (T == 1 || hi - lo < 1024) {
      fn(lo, hi);
      return;
    }
    std::vector<std::thread> th;
    const uint64_t per = (hi - lo + T - 1) / T;
    for (int t = 0; t < T; t++) {
      const uint64_t a = lo + per * t;
      const uint64_t z = std::min(hi, a + per);
      if (a >= z) break;
      th.emplace_back([&fn, a, z] { fn(a, z); });
    }
    for (auto& x : th) x.join();
  }

  // fast_load_factor (include/hkv_hashtable.h:3229-3268).
  float fast_load_factor(uint64_t delta) const {
    const uint64_t N = std::min<uint64_t>(nb, 1024);
    int64_t tot = 0;
    for (uint64_t b = 0; b < N; b++) tot += bsize[b];
    return (float)((delta * 1.0) / (C * 1.0) + (tot * 1.0) / (B * N * 1.0));
  }

  void reserve(uint64_t new_cap) {
    // include/hkv_hashtable.h:2873-2935
    if (reach_max || new_cap > max_cap) {
      reach_max = (C * 2 > max_cap);
      return;
    }
    while (C < new_cap && C * 2 <= max_cap) double_capacity();
    reach_max = (C * 2 > max_cap);
  }

  void maybe_grow(uint64_t n) {
    while (!reach_max && fast_load_factor(n) > max_lf) reserve(C * 2);
  }

  // check_evict_strategy (include/hkv_hashtable.h:3270-3298), plus a check
  // that strategies which read input scores actually receive them.
  int check(int st, const uint64_t* sc, bool ignore) const {
    if (!ignore) {
      if ((st == kLru || st == kEpochLru) && sc) return HKVO_ERR_INVALID;
      if ((st == kLfu || st == kEpochLfu || st == kCustomized) && !sc)
        return HKVO_ERR_INVALID;
      if ((st == kEpochLru || st == kEpochLfu) && epoch == IGNORED_EPOCH)
        return HKVO_ERR_INVALID;
    } else {
      if ((st == kLfu || st == kEpochLfu || st == kCustomized) && !sc)
        return HKVO_ERR_INVALID;
    }
    return HKVO_OK;
  }

  int upsert_batch(Op op, Rule rule, int st, uint64_t n, const uint64_t* ks,
                   const uint8_t* in_vals, uint8_t* io_vals, const uint64_t* sc,
                   const uint8_t* accum, uint64_t clk, std::vector<Record>* recs) {
    std::vector<std::vector<Record>> part(std::max(1, threads));
    std::vector<uint64_t> bk;
    const int T = std::max(1, threads);
    if (T == 1 || nb < 1024) {
      for (uint64_t i = 0; i < n; i++)
        apply_one(op, rule, st, i, ks, in_vals, io_vals, sc, accum, clk, recs);
      return HKVO_OK;
    }
    bk.resize(n);
    for (uint64_t i = 0; i < n; i++) {
      uint64_t b;
      uint32_t s;
      uint8_t d;
      if (is_reserved(ks[i])) { bk[i] = ~0ull; continue; }
      locate_key(ks[i], &b, &s, &d);
      bk[i] = b;
    }
    std::vector<std::thread> th;
    const uint64_t per = (nb + T - 1) / T;
    for (int t = 0; t < T; t++) {
      const uint64_t lo = per * t, hi = std::min(nb, lo + per);
      th.emplace_back([&, t, lo, hi] {
        for (uint64_t i = 0; i < n; i++)
          if (bk[i] >= lo && bk[i] < hi)
            apply_one(op, rule, st, i, ks, in_vals, io_vals, sc, accum, clk,
                      &part[t]);
      });
    }
    for (auto& x : th) x.join();
    if (recs) {
      for (auto& p : part)
        for (auto& r : p) recs->push_back(std::move(r));
      std::stable_sort(recs->begin(), recs->end(),
                       [](const Record& a, const Record& b) { return a.idx < b.idx; });
    }
    return HKVO_OK;
  }
};

extern "C" {

hkvo_table* hkvo_create(uint64_t init_capacity, uint64_t max_capacity,
                        uint64_t max_bucket_size, uint64_t dim, int value_type,
                        int strategy, float max_load_factor, int* status) {
  *status = HKVO_OK;
  const uint64_t B = max_bucket_size;
  // include/hkv_hashtable.h:991-1008 option checks.
  if (B < 16 || (B & (B - 1)) != 0 || dim == 0 || value_size(value_type) == 0 ||
      strategy < 0 || strategy > 4 || init_capacity < B) {
    *status = HKVO_ERR_INVALID;
    return nullptr;
  }
  auto* t = new hkvo_table();
  t->B = B;
  t->dim = dim;
  t->vtype = value_type;
  t->esize = value_size(value_type);
  t->row = (size_t)dim * t->esize;
  t->strategy = strategy;
  t->max_lf = max_load_factor;
  t->init_cap = init_capacity;
  t->max_cap = std::max(init_capacity, max_capacity);
  t->bshift = 0;
  while ((1ull << t->bshift) < B) t->bshift++;
  // create_table bucket-count rule (include/table.h:299-311).
  if (init_capacity * 2 > t->max_cap) {
    t->nb = 1 + (t->max_cap - 1) / B;
  } else {
    t->nb = 1;
    while (t->nb * B < init_capacity) t->nb *= 2;
  }
  t->C = t->nb * B;
  t->qd.init(t->C);
  t->empty_d = digest_of(EMPTY_KEY);
  t->reclaim_d = digest_of(RECLAIM_KEY);
  t->resize_storage();
  t->init_buckets(0, t->nb);
  t->reach_max = (init_capacity * 2 > t->max_cap);
  return t;
}

void hkvo_destroy(hkvo_table* t) { delete t; }
void hkvo_set_threads(hkvo_table* t, int threads) { t->threads = std::max(1, threads); }
void hkvo_set_global_epoch(hkvo_table* t, uint64_t e) { t->epoch = e; }

int hkvo_insert_or_assign(hkvo_table* t, uint64_t n, const uint64_t* keys,
                          const void* values, const uint64_t* scores,
                          int unique_key, int ignore, uint64_t clock) {
  // include/hkv_hashtable.h:1077-1215: ignore_evict_strategy instantiates
  // kCustomized for this call.
  const int st = ignore ? kCustomized : t->strategy;
  if (n == 0) return HKVO_OK;
  t->maybe_grow(n);
  int rc = t->check(st, scores, ignore != 0);
  if (rc) return rc;
  return t->upsert_batch(OP_INSERT_OR_ASSIGN, unique_key ? RULE_DIGEST16 : RULE_TILE32,
                         st, n, keys, (const uint8_t*)values, nullptr, scores,
                         nullptr, clock, nullptr);
}

int hkvo_find_or_insert(hkvo_table* t, uint64_t n, const uint64_t* keys,
                        void* values, const uint64_t* scores, int unique_key,
                        int ignore, uint64_t clock) {
  // include/hkv_hashtable.h:1526-1632 (the table strategy is kept even when
  // ignore_evict_strategy skips the check).
  if (n == 0) return HKVO_OK;
  t->maybe_grow(n);
  int rc = t->check(t->strategy, scores, ignore != 0);
  if (rc) return rc;
  return t->upsert_batch(OP_FIND_OR_INSERT, unique_key ? RULE_DIGEST16 : RULE_TILE32,
                         t->strategy, n, keys, (const uint8_t*)values,
                         (uint8_t*)values, scores, nullptr, clock, nullptr);
}

int hkvo_insert_and_evict(hkvo_table* t, uint64_t n, const uint64_t* keys,
                          const void* values, const uint64_t* scores,
                          uint64_t* ev_keys, void* ev_values, uint64_t* ev_scores,
                          uint64_t* ev_count, int unique_key, int ignore,
                          uint64_t clock) {
  // include/hkv_hashtable.h:1260-1324.  Records are listed in batch order.
  if (n == 0) return HKVO_OK;
  t->maybe_grow(n);
  int rc = t->check(t->strategy, scores, ignore != 0);
  if (rc) return rc;
  std::vector<Record> recs;
  t->upsert_batch(OP_INSERT_AND_EVICT, unique_key ? RULE_DIGEST16 : RULE_TILE32,
                  t->strategy, n, keys, (const uint8_t*)values, nullptr, scores,
                  nullptr, clock, &recs);
  uint64_t c = *ev_count;
  for (auto& r : recs) {
    ev_keys[c] = r.key;
    if (ev_scores) ev_scores[c] = r.score;
    std::memcpy((uint8_t*)ev_values + c * t->row, r.row.data(), t->row);
    c++;
  }
  *ev_count = c;
  return HKVO_OK;
}

int hkvo_accum_or_assign(hkvo_table* t, uint64_t n, const uint64_t* keys,
                         const void* vals, const uint8_t* accum,
                         const uint64_t* scores, int ignore, uint64_t clock) {
  // include/hkv_hashtable.h:1438-1507
  if (t->vtype == HKVO_F64 || t->vtype == HKVO_U16 || t->vtype == HKVO_U32)
    return HKVO_ERR_RUNTIME;
  if (!(t->vtype == HKVO_F32 || t->vtype == HKVO_I32 || t->vtype == HKVO_I64 ||
        t->vtype == HKVO_U64))
    return HKVO_ERR_UNSUPPORTED;
  if (n == 0) return HKVO_OK;
  t->maybe_grow(n);
  int rc = t->check(t->strategy, scores, ignore != 0);
  if (rc) return rc;
  return t->upsert_batch(OP_ACCUM, RULE_TILE32, t->strategy, n, keys,
                         (const uint8_t*)vals, nullptr, scores, accum, clock,
                         nullptr);
}

int hkvo_assign_scores(hkvo_table* t, uint64_t n, const uint64_t* keys,
                       const uint64_t* scores, uint64_t clock) {
  // include/hkv_hashtable.h:1943-1977 and
  // include/kernels/assign_scores_kernel/assign_scores_kernel_with_filter.h:35-143
  if (n == 0) return HKVO_OK;
  int rc = t->check(t->strategy, scores, false);
  if (rc) return rc;
  const bool has_in = scores != nullptr;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    if (is_reserved(k)) continue;
    uint64_t b;
    uint32_t s;
    uint8_t d;
    t->locate_key(k, &b, &s, &d);
    const int64_t p = t->find_slot(b, s, d, k);
    if (p < 0) continue;
    bool w;
    const uint64_t ns = score_wo_missed(t->strategy, has_in, has_in ? scores[i] : 0,
                                        t->epoch, clock, t->scores[b * t->B + p], &w);
    if (w) t->scores[b * t->B + p] = ns;
  }
  return HKVO_OK;
}

int hkvo_find(hkvo_table* t, uint64_t n, const uint64_t* keys, void* values,
              uint8_t* founds, uint64_t* scores) {
  // include/kernels/find_kernel/find_with_digest_kernel.h:30-108; missed rows
  // are left untouched.  Read-only, so in threaded mode each thread takes a
  // contiguous range of the batch.
  auto range = [&](uint64_t i0, uint64_t i1) {
    for (uint64_t i = i0; i < i1; i++) {
      const uint64_t k = keys[i];
      bool found = false;
      if (!is_reserved(k)) {
        uint64_t b;
        uint32_t s;
        uint8_t d;
        t->locate_key(k, &b, &s, &d);
        const int64_t p = t->find_slot(b, s, d, k);
        if (p >= 0) {
          found = true;
          if (scores) scores[i] = t->scores[b * t->B + p];
          std::memcpy((uint8_t*)values + i * t->row, t->rowp(b, (uint32_t)p), t->row);
        }
      }
      if (founds) founds[i] = found ? 1 : 0;
    }
  };
  const uint64_t T = (uint64_t)std::max(1, t->threads);
  if (T == 1 || n < 4096) {
    range(0, n);
    return HKVO_OK;
  }
  std::vector<std::thread> th;
  for (uint64_t j = 0; j < T; j++)
    th.emplace_back(range, n * j / T, n * (j + 1) / T);
  for (auto& x : th) x.join();
  return HKVO_OK;
}

int hkvo_contains(hkvo_table* t, uint64_t n, const uint64_t* keys,
                  uint8_t* founds) {
  // include/kernels/contains_kernel/contains_kernel.h:31-69
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    bool found = false;
    if (!is_reserved(k)) {
      uint64_t b;
      uint32_t s;
      uint8_t d;
      t->locate_key(k, &b, &s, &d);
      found = t->find_slot(b, s, d, k) >= 0;
    }
    founds[i] = found ? 1 : 0;
  }
  return HKVO_OK;
}

int hkvo_assign(hkvo_table* t, uint64_t n, const uint64_t* keys,
                const void* values, const uint64_t* scores, int with_scores,
                uint64_t clock) {
  // assign (include/hkv_hashtable.h:1830-1921, assign_kernel.h:31-243) with
  // with_scores, assign_values (include/hkv_hashtable.h:2003-2093,
  // assign_values_kernel.h:32-233) without: batch order, a present key takes
  // the input row and, for assign, update_without_missed on its score.
  if (n == 0) return HKVO_OK;
  if (with_scores) {
    int rc = t->check(t->strategy, scores, false);
    if (rc) return rc;
  }
  const bool has_in = scores != nullptr;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    if (is_reserved(k)) continue;
    uint64_t b;
    uint32_t s;
    uint8_t d;
    t->locate_key(k, &b, &s, &d);
    const int64_t p = t->find_slot(b, s, d, k);
    if (p < 0) continue;
    if (with_scores) {
      bool w;
      const uint64_t g = b * t->B + (uint64_t)p;
      const uint64_t ns = score_wo_missed(t->strategy, has_in, has_in ? scores[i] : 0,
                                          t->epoch, clock, t->scores[g], &w);
      if (w) t->scores[g] = ns;
    }
    std::memcpy(t->rowp(b, (uint32_t)p), (const uint8_t*)values + i * t->row, t->row);
  }
  return HKVO_OK;
}

int hkvo_find_ptr(hkvo_table* t, uint64_t n, const uint64_t* keys,
                  uint64_t* slots, uint8_t* founds, uint64_t* scores) {
  // include/kernels/find_ptr_kernel/find_ptr_with_digest_kernel.h:30-148
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    slots[i] = HKVO_NO_SLOT;
    if (founds) founds[i] = 0;
    if (is_reserved(k)) continue;
    uint64_t b;
    uint32_t s;
    uint8_t d;
    t->locate_key(k, &b, &s, &d);
    const int64_t p = t->find_slot(b, s, d, k);
    if (p < 0) continue;
    slots[i] = b * t->B + (uint64_t)p;
    if (founds) founds[i] = 1;
    if (scores) scores[i] = t->scores[slots[i]];
  }
  return HKVO_OK;
}

int hkvo_find_and_update(hkvo_table* t, uint64_t n, const uint64_t* keys,
                         uint64_t* slots, uint8_t* founds, uint64_t* scores,
                         int unique_key, uint64_t clock) {
  // include/hkv_hashtable.h:2288-2317 and
  // include/kernels/find_and_update_kernel/find_and_update_kernel_with_filter.h:35-165:
  // a found key takes update_score_only(new_insert=false) with
  // desired_when_missed, and its score after the update is returned.
  if (n == 0) return HKVO_OK;
  int rc = t->check(t->strategy, scores, false);
  if (rc) return rc;
  if (!unique_key) return HKVO_ERR_RUNTIME;
  const bool has_in = scores != nullptr;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    slots[i] = HKVO_NO_SLOT;
    if (founds) founds[i] = 0;
    if (is_reserved(k)) continue;
    uint64_t b;
    uint32_t s;
    uint8_t d;
    t->locate_key(k, &b, &s, &d);
    const int64_t p = t->find_slot(b, s, d, k);
    if (p < 0) continue;
    const uint64_t g = b * t->B + (uint64_t)p;
    const uint64_t in = has_in ? scores[i] : 0;
    const uint64_t des = desired(t->strategy, has_in, in, t->epoch, clock);
    bool w;
    const uint64_t ns = score_hit(t->strategy, has_in, in, des, t->scores[g], &w);
    if (w) t->scores[g] = ns;
    slots[i] = g;
    if (founds) founds[i] = 1;
    if (scores) scores[i] = t->scores[g];
  }
  return HKVO_OK;
}

int hkvo_find_or_insert_ptr(hkvo_table* t, uint64_t n, const uint64_t* keys,
                            uint64_t* slots, uint8_t* founds,
                            const uint64_t* scores, int unique_key, int ignore,
                            int keep_locked, uint64_t clock) {
  // include/hkv_hashtable.h:1658-1728.  unique_key: the lock-key kernel
  // (digest-16 probe and eviction, find_or_insert_ptr_kernel_v2.h:38-285)
  // holds each claimed or found slot LOCKED until the batch ends, then the
  // unlock kernel (:287-303) writes the keys back unless the caller keeps
  // them locked.  Otherwise find_or_insert_ptr_kernel_vf_v2 (:305-386):
  // find_and_lock tiles, each key unlocked right after its own step.
  if (n == 0) return HKVO_OK;
  t->maybe_grow(n);
  int rc = t->check(t->strategy, scores, ignore != 0);
  if (rc) return rc;
  if (keep_locked && !unique_key) return HKVO_ERR_UNSUPPORTED;
  std::vector<uint64_t> w(n, 0);
  t->slot_out = w.data();
  t->lock_batch = unique_key != 0;
  t->upsert_batch(OP_FIND_OR_INSERT_PTR, unique_key ? RULE_DIGEST16 : RULE_TILE32,
                  t->strategy, n, keys, nullptr, nullptr, scores, nullptr, clock,
                  nullptr);
  t->slot_out = nullptr;
  t->lock_batch = false;
  for (uint64_t i = 0; i < n; i++) {
    if (w[i] == 0) {
      slots[i] = HKVO_NO_SLOT;
      founds[i] = 0;
      continue;
    }
    slots[i] = (w[i] & ~SLOT_FOUND) - 1;
    founds[i] = (w[i] & SLOT_FOUND) ? 1 : 0;
    if (unique_key && !keep_locked) t->keys[slots[i]] = keys[i];
  }
  return HKVO_OK;
}

int hkvo_lock_keys(hkvo_table* t, uint64_t n, const uint64_t* keys,
                   uint64_t* slots, uint8_t* success, const uint64_t* scores,
                   uint64_t clock) {
  // include/kernels/lock_keys_kernel/lock_keys_kernel.h:31-141, keys in batch
  // order: a present key's slot becomes LOCKED and takes
  // update_with_digest(new_insert=false); a repeated key is no longer
  // present for its later occurrences.
  if (n == 0) return HKVO_OK;
  const int st = t->strategy;
  if ((st == kEpochLfu || st == kCustomized) && !scores) return HKVO_ERR_INVALID;
  const bool has_in = scores != nullptr;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    slots[i] = HKVO_NO_SLOT;
    if (success) success[i] = 0;
    if (is_reserved(k)) continue;
    uint64_t b;
    uint32_t s;
    uint8_t d;
    t->locate_key(k, &b, &s, &d);
    const int64_t p = t->find_slot(b, s, d, k);
    if (p < 0) continue;
    const uint64_t g = b * t->B + (uint64_t)p;
    t->keys[g] = LOCKED_KEY;
    const uint64_t in = has_in ? scores[i] : 0;
    bool w;
    const uint64_t ns = score_hit(st, has_in, in, desired(st, has_in, in, t->epoch, clock),
                                  t->scores[g], &w);
    if (w) t->scores[g] = ns;
    slots[i] = g;
    if (success) success[i] = 1;
  }
  return HKVO_OK;
}

int hkvo_unlock_keys(hkvo_table* t, uint64_t n, const uint64_t* slots,
                     const uint64_t* keys, uint8_t* success) {
  // include/kernels/unlock_keys_kernel/unlock_keys_kernel.h:40-79
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t g = slots[i];
    const bool ok = g < t->C && t->keys[g] == LOCKED_KEY;
    if (ok) t->keys[g] = keys[i];
    if (success) success[i] = ok ? 1 : 0;
  }
  return HKVO_OK;
}

int hkvo_find_missed(hkvo_table* t, uint64_t n, const uint64_t* keys,
                     void* values, uint64_t* missed_keys, int32_t* missed_idx,
                     int32_t* missed_size, uint64_t* scores) {
  // include/kernels/find_kernel/find_miss_with_digest_kernel.h:30-198.
  // Misses are listed in batch order; reserved keys count as misses.
  int32_t m = 0;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    bool found = false;
    if (!is_reserved(k)) {
      uint64_t b;
      uint32_t s;
      uint8_t d;
      t->locate_key(k, &b, &s, &d);
      const int64_t p = t->find_slot(b, s, d, k);
      if (p >= 0) {
        found = true;
        if (scores) scores[i] = t->scores[b * t->B + p];
        std::memcpy((uint8_t*)values + i * t->row, t->rowp(b, (uint32_t)p), t->row);
      }
    }
    if (!found) {
      missed_keys[m] = k;
      missed_idx[m] = (int32_t)i;
      m++;
    }
  }
  *missed_size = m;
  return HKVO_OK;
}

// Built-in predicates of erase_if / size_if / export_batch_if, in the
// reference's v1 functor form PredFunctor<K, S>(key, score, pattern,
// threshold) (include/hkv_hashtable.h:2380-2398); key_signed selects K =
// int64_t.
static bool pred_eval(int pred, int key_signed, uint64_t k, uint64_t s, uint64_t pat,
                      uint64_t th) {
  switch (pred) {
    case 0: return s < th;
    case 1: return s >= th;
    case 2: return s > th;
    case 3: return (k & pat) == pat;
    case 4:
      if (key_signed) return ((int64_t)(k & 0x7f) > (int64_t)pat) && (s > th);
      return ((k & 0x7f) > pat) && (s > th);
    default: return false;
  }
}

int hkvo_erase_if(hkvo_table* t, int pred, uint64_t pattern, uint64_t threshold,
                  int key_signed, uint64_t* count) {
  // remove_if_kernel (include/kernels/remove_kernel/remove_kernel.h:116-160)
  if (pred < 0 || pred > 4) return HKVO_ERR_INVALID;
  uint64_t c = 0;
  for (uint64_t g = 0; g < t->C; g++) {
    const uint64_t k = t->keys[g];
    if (is_reserved(k)) continue;
    if (!pred_eval(pred, key_signed, k, t->scores[g], pattern, threshold)) continue;
    t->keys[g] = RECLAIM_KEY;
    t->scores[g] = EMPTY_SCORE;
    t->dg[g] = t->reclaim_d;
    t->bsize[g / t->B]--;
    c++;
  }
  *count = c;
  return HKVO_OK;
}

int hkvo_size_if(hkvo_table* t, int pred, uint64_t pattern, uint64_t threshold,
                 int key_signed, uint64_t* count) {
  // size_if_kernel (include/kernels/size_if_kernel/size_if_kernel.h)
  if (pred < 0 || pred > 4) return HKVO_ERR_INVALID;
  uint64_t c = 0;
  for (uint64_t g = 0; g < t->C; g++) {
    const uint64_t k = t->keys[g];
    if (!is_reserved(k) && pred_eval(pred, key_signed, k, t->scores[g], pattern, threshold)) c++;
  }
  *count = c;
  return HKVO_OK;
}

uint64_t hkvo_export_batch_if(hkvo_table* t, int pred, uint64_t pattern,
                              uint64_t threshold, int key_signed, uint64_t n,
                              uint64_t offset, uint64_t* keys, void* values,
                              uint64_t* scores) {
  // dump_kernel_if (include/kernels/dump_kernel/dump_kernel_if.h), listed in
  // slot order (the device order is unspecified).
  if (offset >= t->C) return 0;
  n = std::min(n, t->C - offset);
  uint64_t c = 0;
  for (uint64_t g = offset; g < offset + n; g++) {
    const uint64_t k = t->keys[g];
    if (is_reserved(k) || !pred_eval(pred, key_signed, k, t->scores[g], pattern, threshold))
      continue;
    keys[c] = k;
    if (scores) scores[c] = t->scores[g];
    std::memcpy((uint8_t*)values + c * t->row, t->rowp(g / t->B, (uint32_t)(g % t->B)), t->row);
    c++;
  }
  return c;
}

int hkvo_set_max_capacity(hkvo_table* t, uint64_t new_max) {
  // include/hkv_hashtable.h:2955-2977
  if (new_max == 0 || (new_max & (new_max - 1))) return HKVO_ERR_UNSUPPORTED;
  if (new_max < t->C) return HKVO_OK;
  t->reach_max = false;
  t->max_cap = new_max;
  return HKVO_OK;
}

int hkvo_erase(hkvo_table* t, uint64_t n, const uint64_t* keys) {
  // include/kernels/remove_kernel/remove_kernel.h:31-113: every digest group
  // is scanned (no early stop); a match becomes RECLAIM with score 0 and the
  // reclaim digest.
  const uint64_t B = t->B;
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t k = keys[i];
    if (is_reserved(k)) continue;
    uint64_t b;
    uint32_t s;
    uint8_t d;
    t->locate_key(k, &b, &s, &d);
    const uint64_t base = b * B;
    const uint32_t a = s & ~3u;
    for (uint32_t off = 0; off < B + 4; off += 4) {
      const uint32_t g = (a + off) & (uint32_t)(B - 1);
      for (uint32_t j = 0; j < 4; j++) {
        const uint32_t p = g + j;
        if (t->dg[base + p] == d && t->keys[base + p] == k) {
          t->keys[base + p] = RECLAIM_KEY;
          t->scores[base + p] = EMPTY_SCORE;
          t->dg[base + p] = t->reclaim_d;
          t->bsize[b]--;
          break;
        }
      }
    }
  }
  return HKVO_OK;
}

void hkvo_clear(hkvo_table* t) {
  // include/kernels/clear_kernel/clear_kernel.h:27-59 (scores untouched)
  for (uint64_t i = 0; i < t->C; i++) {
    t->dg[i] = t->empty_d;
    t->keys[i] = EMPTY_KEY;
  }
  std::fill(t->bsize.begin(), t->bsize.end(), 0);
}

uint64_t hkvo_export_batch(hkvo_table* t, uint64_t n, uint64_t offset,
                           uint64_t* keys, void* values, uint64_t* scores) {
  // include/hkv_hashtable.h:2519-2555 and dump_kernel.h:36-122; records are
  // listed in slot order.
  if (offset >= t->C) return 0;
  n = std::min(t->C - offset, n);
  uint64_t c = 0;
  for (uint64_t g = offset; g < offset + n; g++) {
    const uint64_t k = t->keys[g];
    if (is_reserved(k)) continue;
    keys[c] = k;
    if (scores) scores[c] = t->scores[g];
    std::memcpy((uint8_t*)values + c * t->row, t->vals.data() + g * t->row, t->row);
    c++;
  }
  return c;
}

int hkvo_reserve(hkvo_table* t, uint64_t new_capacity) {
  t->reserve(new_capacity);
  return HKVO_OK;
}

uint64_t hkvo_size(hkvo_table* t) {
  int64_t s = 0;
  for (auto v : t->bsize) s += v;
  return (uint64_t)s;
}
uint64_t hkvo_capacity(hkvo_table* t) { return t->C; }
uint64_t hkvo_bucket_count(hkvo_table* t) { return t->nb; }

void hkvo_raw(hkvo_table* t, const uint8_t** digests, const uint64_t** keys,
              const uint64_t** scores, const int32_t** bucket_sizes,
              const uint8_t** values) {
  if (digests) *digests = t->dg.data();
  if (keys) *keys = t->keys.data();
  if (scores) *scores = t->scores.data();
  if (bucket_sizes) *bucket_sizes = t->bsize.data();
  if (values) *values = t->vals.data();
}

uint64_t hkvo_murmur3(uint64_t key) { return murmur3(key); }
uint64_t hkvo_global_idx(uint64_t hashed, uint64_t capacity) {
  QuickDiv q;
  q.init(capacity);
  return q.mod(hashed);
}
uint8_t hkvo_empty_digest(void) { return digest_of(EMPTY_KEY); }
uint8_t hkvo_reclaim_digest(void) { return digest_of(RECLAIM_KEY); }

uint64_t hkvo_score_desired(int st, int has_in, uint64_t in, uint64_t epoch,
                            uint64_t clock) {
  return desired(st, has_in != 0, in, epoch, clock);
}
uint64_t hkvo_score_new(int st, int has_in, uint64_t in, uint64_t des,
                        uint64_t old) {
  bool w;
  return score_new(st, has_in != 0, in, des, old, &w);
}
uint64_t hkvo_score_hit(int st, int has_in, uint64_t in, uint64_t des,
                        uint64_t old) {
  bool w;
  return score_hit(st, has_in != 0, in, des, old, &w);
}
uint64_t hkvo_score_without_missed(int st, int has_in, uint64_t in,
                                   uint64_t epoch, uint64_t clock, uint64_t old) {
  bool w;
  return score_wo_missed(st, has_in != 0, in, epoch, clock, old, &w);
}

}  // extern "C"
