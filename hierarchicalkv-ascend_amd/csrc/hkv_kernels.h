// hkv_kernels.h -- host launchers of the gfx950 table kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hkv_dev.h"

namespace hkv {

// Operations served by the bucket-owner apply path.
enum ApplyOp {
  OP_INSERT_OR_ASSIGN = 0,
  OP_FIND_OR_INSERT = 1,
  OP_INSERT_AND_EVICT = 2,
  OP_ACCUM_OR_ASSIGN = 3,
  OP_ASSIGN_SCORES = 4,
  OP_FIND_OR_INSERT_PTR = 5,  // find_or_insert returning row addresses: no row moves
};

// Slot word of the pointer find_or_insert: global slot index + 1 (0 = no
// slot), with this bit set when the key was found.
constexpr uint64_t kSlotFound = 1ull << 63;

// Eviction tie-break family: the reference's 16-lane digest kernels (unique
// keys) or its 32-lane find_and_lock tiles (non-unique keys, accum_or_assign).
enum EvictRule { RULE_DIGEST16 = 0, RULE_TILE32 = 1 };

struct ApplyArgs {
  const uint64_t* keys;
  const uint8_t* in_values;   // input rows (deltas for accum)
  uint8_t* io_values;         // find_or_insert output rows
  const uint64_t* in_scores;  // may be null
  const uint8_t* accum_flags; // accum_or_assign only
  uint64_t* ev_keys;          // insert_and_evict outputs
  uint8_t* ev_values;
  uint64_t* ev_scores;
  uint64_t* ev_counter;
  uint32_t* ev_bits;          // insert_and_evict: records at their batch index, flagged here
                              // (null: records appended at an atomic counter)
  uint64_t* slot_out;         // pointer find_or_insert: slot word per batch index
  int lock;                   // pointer find_or_insert: claimed and found slots hold
                              // LOCKED until the batch ends
  uint64_t n;
  ScoreCtx sc;
  int rule;
  int unit;        // row copy unit in bytes
  int value_type;  // for accumulation
};

// Listed partitions with more than kBigPart entries of a batch with repeated
// keys (Zipf traffic) are counted, folded and tasked over the whole GPU; one
// slot of per-partition state each, at most kBigMax per call (others take
// the in-block path).
constexpr uint32_t kBigPart = 4096;
constexpr uint32_t kBigMax = 256;
constexpr uint32_t kBigMapCap = 1024;  // distinct keys of a partition's heavy buckets
constexpr uint32_t kBigLight = 1024;   // other entries, run by one LDS run
struct BigSlot {
  uint32_t tot[256];                // entries per bucket of the partition
  uint64_t mkey[kBigMapCap];        // key map: key (EMPTY: free),
  uint64_t msum[kBigMapCap];        // fold of the input scores,
  uint32_t mfirst[kBigMapCap];      // first and last batch index,
  uint32_t mlast[kBigMapCap];
  uint32_t mres[kBigMapCap];        // placement (slot | new / placed flags)
  uint32_t mfull;                   // a key did not fit the map
  uint32_t nlight;                  // entries of the other buckets
  uint32_t fast;                    // k_apply_part left the row tasks to k_big_tasks
  uint32_t pad;
  uint64_t light[2 * kBigLight];    // those entries, {key, batch index}
};

// Per-call scratch of the partitioned apply pipeline (owned by the table).
// A partition is a run of 256 consecutive buckets; the batch is cut into
// chunks of 1024 keys.  Segment (g, p) = the keys of chunk g that fall in
// partition p.
struct PartScratch {
  uint32_t* hist;       // [chunks][partitions]: segment sizes, then offsets
  uint64_t* ent;        // {key, batch index} entries: [partitions * cap + n][2]
  uint32_t* pinfo;      // [partitions][2]: first entry, entry count
  uint32_t* spill_top;  // entries placed past the fixed regions
  uint64_t* trow;       // [n] row task per batch index, zero between calls
  uint32_t* plist;      // [partitions] partitions the single-run kernel left: whole ones
                        // from the front, long-bucket-only ones from the back
  uint32_t* drec;       // [n][4] buckets handed to the 16-lane kernel
  uint64_t* dpool;      // [n][2] their keys, {key, batch index}
  uint32_t* dctr;       // [8] records, pool entries, whole partitions listed, partitions
                        // taken, big partitions listed, long-bucket-only partitions
                        // listed (zeroed by the count kernel)
  uint32_t* ev_bits;    // [n / 32 + 1] insert_and_evict record flags, zero between calls
  uint32_t* ev_wpre;    // [n / 32 + 1] set bits before each word, within its block of 256 words
  uint32_t* ev_blk;     // [n / 8192 + 3] block offsets, then the record count and records below it
  BigSlot* big;         // [kBigMax] big-partition state (null: that path is off)
  uint32_t* big_part;   // [kBigMax] partition of each big slot
  uint32_t np;          // partitions
  uint32_t prange;      // partitions per counting pass (LDS histogram size)
  uint32_t chunks;      // batch chunks
  uint32_t cap;         // fixed region size per partition (entries)
};

// Partitions one pass of the counting and scatter kernels holds in LDS.
constexpr uint32_t kPartRange = 16384;
constexpr uint32_t kPartBuckets = 256;
constexpr uint32_t kPartChunk = 1024;

void launch_init_slots(const TableView& t, uint64_t from_bucket,
                       uint64_t to_bucket, hipStream_t s);
void launch_clear(const TableView& t, hipStream_t s);
void launch_find(const TableView& t, const uint64_t* keys, uint64_t n,
                 uint8_t* values, uint8_t* founds, uint64_t* scores, int unit,
                 hipStream_t s);
void launch_find_missed(const TableView& t, const uint64_t* keys, uint64_t n,
                        uint8_t* values, uint64_t* missed_keys,
                        int32_t* missed_idx, int32_t* missed_size,
                        uint64_t* scores, int unit, hipStream_t s);
void launch_erase(const TableView& t, const uint64_t* keys, uint64_t n,
                  hipStream_t s);
void launch_apply_part(const TableView& t, int op, const ApplyArgs& a,
                       const PartScratch& ps, hipStream_t s);
// Pointer find_or_insert: placement in batch order, slot words in
// ps.trow, then value / key addresses, founds, and (unless keep_locked) the
// keys written back over LOCKED.
void launch_find_or_insert_ptr(const TableView& t, const ApplyArgs& a, const PartScratch& ps,
                               uint64_t* value_ptrs, uint8_t* founds, uint64_t* key_ptrs,
                               bool keep_locked, hipStream_t s);
// Row addresses of present keys; with `update`, the hit score functor runs
// on each found key first (find_and_update).
void launch_find_ptr(const TableView& t, const uint64_t* keys, uint64_t n,
                     uint64_t* value_ptrs, uint8_t* founds, uint64_t* scores, bool update,
                     const ScoreCtx& sc, hipStream_t s);
void launch_contains(const TableView& t, const uint64_t* keys, uint64_t n, uint8_t* founds,
                     hipStream_t s);
// assign (with_scores: update_without_missed on each found key) and
// assign_values: present keys' rows overwritten from `values`.
void launch_assign(const TableView& t, const uint64_t* keys, uint64_t n, const uint8_t* values,
                   const uint64_t* scores, bool with_scores, const ScoreCtx& sc, int unit,
                   hipStream_t s);
void launch_lock_keys(const TableView& t, const uint64_t* keys, uint64_t n,
                      uint64_t* key_ptrs, uint8_t* success, const uint64_t* scores,
                      const ScoreCtx& sc, hipStream_t s);
void launch_unlock_keys(const TableView& t, uint64_t n, const uint64_t* key_ptrs,
                        const uint64_t* keys, uint8_t* success, hipStream_t s);
void launch_export(const TableView& t, uint64_t offset, uint64_t n,
                   uint64_t* d_counter, uint64_t* keys, uint8_t* values,
                   uint64_t* scores, uint32_t* block_scratch, int unit,
                   hipStream_t s);
void launch_size(const TableView& t, uint64_t nbuckets, uint64_t* out,
                 hipStream_t s);
// Growth: the plan kernel rebuilds the old buckets' metadata and the new
// buckets' (include/kernels/rehash_kernel/rehash_kernel.h:29-207) and
// records the row moves; phase 0 of the row kernel moves rows to new buckets
// and stages the ones that stay in their bucket, phase 1 writes the staged
// rows back.
struct RehashScratch {
  uint16_t* rec;     // [old buckets * 128] row-move records
  uint16_t* cnt;     // [old buckets] moves to the new bucket | moves within << 8
  uint32_t* tbase;   // [old buckets] first staging row of the bucket
  uint32_t* tcount;  // staging rows in all (zero before the plan kernel)
};
void launch_rehash_plan(const TableView& t, uint64_t old_buckets, const RehashScratch& rs,
                        hipStream_t s);
void launch_rehash_rows(const TableView& t, uint64_t old_buckets, const RehashScratch& rs,
                        uint8_t* stage, int phase, int unit, hipStream_t s);
void launch_fill_u64(uint64_t* p, uint64_t v, uint64_t n, hipStream_t s);
void launch_fill_u32(uint32_t* p, uint32_t v, uint64_t n, hipStream_t s);

}  // namespace hkv
