// C++ drop-in check of the functor APIs (erase_if, erase_if_v2,
// export_batch_if, export_batch_if_v2, size_if, for_each), built with hipcc
// so that the facade instantiates its kernels with these functors.  The
// functors are written the way the reference's tests write them
// (tests/community/find_or_insert_ptr_test.cpp:49-56,
// tests/test_export_batch_if_v2.cpp:47-69, tests/test_size_if.cpp:38-69) and
// their results are compared with the oracle's built-in predicates.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <random>
#include <tuple>
#include <vector>

#include "hkv_hashtable.hpp"
#include "../../oracle/hkv_oracle.h"

#define REQUIRE(c)                                                  \
  do {                                                              \
    if (!(c)) {                                                     \
      std::printf("FAILED %s at line %d\n", #c, __LINE__);          \
      return 1;                                                     \
    }                                                               \
  } while (0)

using K = uint64_t;
using V = float;
using S = uint64_t;
constexpr size_t kDim = 8;

template <class KT, class ST>
struct ScoreLtPred {
  __forceinline__ __simt_callee__ bool operator()(const KT& key, const ST& score,
                                                  const KT& pattern, const ST& threshold) {
    return score < threshold;
  }
};

template <class KT, class ST>
struct EraseIfPredFunctor {
  __forceinline__ __simt_callee__ bool operator()(const KT& key, ST& score,
                                                  const KT& pattern, const ST& threshold) {
    return (((key & 0x7f) > pattern) && (score > threshold));
  }
};

template <class KT, class VT, class ST>
struct ExportV2Pred {
  KT pattern;
  ST threshold;
  ExportV2Pred(KT p, ST t) : pattern(p), threshold(t) {}
  template <int GroupSize>
  __forceinline__ __simt_callee__ bool operator()(const KT& key, const __gm__ VT* value,
                                                  const ST& score) {
    return ((!npu::hkv::IS_RESERVED_KEY<KT>(key)) && (score < threshold));
  }
};

template <class KT, class VT, class ST>
struct EraseV2Pred {
  KT pattern;
  ST threshold;
  __forceinline__ __simt_callee__ bool operator()(const KT& key, const __gm__ VT* value,
                                                  const ST& score, int group_size) {
    return (key & pattern) == pattern;
  }
};

struct AddOne {
  __device__ void operator()(const K& key, V* value, S* score, int group_size) {
    if (npu::hkv::IS_RESERVED_KEY<K>(key)) return;
    value[0] += 1.0f;
    *score += 1;
  }
};

template <class T>
T* dev(size_t n) {
  T* d = nullptr;
  if (hipMalloc(&d, n * sizeof(T) + 16) != hipSuccess) return nullptr;
  hipMemset(d, 0, n * sizeof(T));
  return d;
}

template <class T>
std::vector<T> host(const T* d, size_t n) {
  std::vector<T> h(n);
  hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost);
  return h;
}

// (key, score, row) tuples sorted by key.
using Rec = std::tuple<uint64_t, uint64_t, std::vector<float>>;
std::vector<Rec> records(const uint64_t* k, const uint64_t* s, const float* v, size_t c) {
  std::vector<Rec> r;
  for (size_t i = 0; i < c; i++)
    r.emplace_back(k[i], s[i], std::vector<float>(v + i * kDim, v + (i + 1) * kDim));
  std::sort(r.begin(), r.end());
  return r;
}

int main() {
  using namespace npu::hkv;
  using Table = HashTable<K, V, S, EvictStrategy::kCustomized>;
  const size_t cap = 1 << 14, n = 10000;
  HashTableOptions opt;
  opt.init_capacity = cap;
  opt.max_capacity = cap;
  opt.max_hbm_for_vectors = 1ull << 30;
  opt.dim = kDim;
  Table table;
  table.init(opt);
  REQUIRE(table.empty());
  int st = 0;
  hkvo_table* o = hkvo_create(cap, cap, 128, kDim, HKVO_F32, 4, 0.5f, &st);
  REQUIRE(st == 0);

  std::mt19937_64 rng(7);
  std::vector<uint64_t> keys(n), scores(n);
  std::vector<float> vals(n * kDim);
  for (size_t i = 0; i < n; i++) {
    keys[i] = rng() >> 1;
    scores[i] = rng() % 1000;
    for (size_t j = 0; j < kDim; j++) vals[i * kDim + j] = (float)(rng() % 100000) * 1e-5f;
  }
  K* dk = dev<K>(n);
  S* ds = dev<S>(n);
  V* dv = dev<V>(n * kDim);
  hipMemcpy(dk, keys.data(), n * 8, hipMemcpyHostToDevice);
  hipMemcpy(ds, scores.data(), n * 8, hipMemcpyHostToDevice);
  hipMemcpy(dv, vals.data(), n * kDim * 4, hipMemcpyHostToDevice);
  table.insert_or_assign(n, dk, dv, ds);
  REQUIRE(hkvo_insert_or_assign(o, n, keys.data(), vals.data(), scores.data(), 1, 0, 0) == 0);
  REQUIRE(table.size() == hkvo_size(o));
  REQUIRE(!table.empty());

  size_t* dcount = dev<size_t>(1);
  K* ek = dev<K>(cap);
  V* ev = dev<V>(cap * kDim);
  S* es = dev<S>(cap);
  std::vector<uint64_t> ok(cap), os(cap);
  std::vector<float> ov(cap * kDim);

  // size_if and export_batch_if with score < 500
  table.size_if<ScoreLtPred>(0, 500, dcount);
  uint64_t oc = 0;
  REQUIRE(hkvo_size_if(o, HKV_PRED_SCORE_LT, 0, 500, 0, &oc) == 0);
  REQUIRE(host(dcount, 1)[0] == oc);
  REQUIRE(oc > 1000 && oc < n);
  table.export_batch_if<ScoreLtPred>(0, 500, cap, 0, dcount, ek, ev, es);
  size_t c = host(dcount, 1)[0];
  oc = hkvo_export_batch_if(o, HKV_PRED_SCORE_LT, 0, 500, 0, cap, 0, ok.data(), ov.data(),
                            os.data());
  REQUIRE(c == oc);
  {
    auto gk = host(ek, c);
    auto gs = host(es, c);
    auto gv = host(ev, c * kDim);
    REQUIRE(records(gk.data(), gs.data(), gv.data(), c) ==
            records(ok.data(), os.data(), ov.data(), oc));
  }
  // a window of slots
  table.export_batch_if<ScoreLtPred>(0, 500, 3000, 5000, dcount, ek, ev, es);
  c = host(dcount, 1)[0];
  oc = hkvo_export_batch_if(o, HKV_PRED_SCORE_LT, 0, 500, 0, 3000, 5000, ok.data(), ov.data(),
                            os.data());
  REQUIRE(c == oc);

  // export_batch_if_v2 with score < 300
  ExportV2Pred<K, V, S> p2(0, 300);
  table.export_batch_if_v2(p2, cap, 0, dcount, ek, ev, es);
  c = host(dcount, 1)[0];
  oc = hkvo_export_batch_if(o, HKV_PRED_SCORE_LT, 0, 300, 0, cap, 0, ok.data(), ov.data(),
                            os.data());
  REQUIRE(c == oc);
  {
    auto gk = host(ek, c);
    auto gs = host(es, c);
    auto gv = host(ev, c * kDim);
    REQUIRE(records(gk.data(), gs.data(), gv.data(), c) ==
            records(ok.data(), os.data(), ov.data(), oc));
  }

  // erase_if: ((key & 0x7f) > 0x3f) && score > 500
  const size_t erased = table.erase_if<EraseIfPredFunctor>(0x3f, 500);
  uint64_t oerased = 0;
  REQUIRE(hkvo_erase_if(o, HKV_PRED_KEY_LOW7_GT_SCORE_GT, 0x3f, 500, 0, &oerased) == 0);
  REQUIRE(erased == oerased && erased > 0);
  REQUIRE(table.size() == hkvo_size(o));

  // erase_if_v2: (key & 3) == 3
  EraseV2Pred<K, V, S> e2{3, 0};
  const size_t erased2 = table.erase_if_v2(e2);
  REQUIRE(hkvo_erase_if(o, HKV_PRED_KEY_MASK_EQ, 3, 0, 0, &oerased) == 0);
  REQUIRE(erased2 == oerased && erased2 > 0);
  REQUIRE(table.size() == hkvo_size(o));

  // slot-order state equal after both erases
  table.export_batch(cap, 0, dcount, ek, ev, es);
  c = host(dcount, 1)[0];
  oc = hkvo_export_batch(o, cap, 0, ok.data(), ov.data(), os.data());
  REQUIRE(c == oc);
  auto gk = host(ek, c);
  auto gs = host(es, c);
  auto gv = host(ev, c * kDim);
  REQUIRE(std::memcmp(gk.data(), ok.data(), c * 8) == 0);
  REQUIRE(std::memcmp(gs.data(), os.data(), c * 8) == 0);
  REQUIRE(std::memcmp(gv.data(), ov.data(), c * kDim * 4) == 0);

  // for_each over every slot: live rows get +1 in column 0 and score + 1
  AddOne f;
  table.for_each(0, cap, f);
  table.export_batch(cap, 0, dcount, ek, ev, es);
  REQUIRE(host(dcount, 1)[0] == oc);
  auto fk = host(ek, c);
  auto fs = host(es, c);
  auto fv = host(ev, c * kDim);
  for (size_t i = 0; i < c; i++) {
    REQUIRE(fk[i] == ok[i]);
    REQUIRE(fs[i] == os[i] + 1);
    REQUIRE(fv[i * kDim] == ov[i * kDim] + 1.0f);
    REQUIRE(std::memcmp(&fv[i * kDim + 1], &ov[i * kDim + 1], (kDim - 1) * 4) == 0);
  }

  // set_max_capacity: a power of 2 only
  bool threw = false;
  try {
    table.set_max_capacity(3 * cap);
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  REQUIRE(threw);
  table.set_max_capacity(4 * cap);
  table.reserve(4 * cap);
  REQUIRE(table.capacity() == 4 * cap);

  hkvo_destroy(o);
  std::printf("facade predicates ok: %zu erased, %zu left\n", erased + erased2, c);
  return 0;
}
