// C++ drop-in check: drives the gfx950 table through the header-only facade
// (npu::hkv::HashTable, include/hkv_hashtable.hpp) exactly as reference code
// would, and compares every result with the oracle (oracle/hkv_oracle.h).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>
#include <string>
#include <unistd.h>

#include "hkv_hashtable.hpp"
#include "../../oracle/hkv_oracle.h"

#define REQUIRE(c)                                                  \
  do {                                                              \
    if (!(c)) {                                                     \
      std::printf("FAILED %s at line %d\n", #c, __LINE__);          \
      return 1;                                                     \
    }                                                               \
  } while (0)

template <class T>
T* dev(const std::vector<T>& h) {
  T* d = nullptr;
  if (hipMalloc(&d, h.size() * sizeof(T) + 16) != hipSuccess) return nullptr;
  hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice);
  return d;
}

template <class T>
std::vector<T> host(const T* d, size_t n) {
  std::vector<T> h(n);
  hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost);
  return h;
}

int main() {
  using namespace npu::hkv;
  using Table = HashTable<uint64_t, float, uint64_t, EvictStrategy::kCustomized>;
  const size_t cap = 1 << 14, dim = 8, n = 12000;
  HashTableOptions opt;
  opt.init_capacity = cap;
  opt.max_capacity = cap;
  opt.max_hbm_for_vectors = 1ull << 30;
  opt.dim = dim;
  Table table;
  table.init(opt);
  REQUIRE(table.capacity() == cap);
  REQUIRE(table.dim() == dim);
  REQUIRE(table.is_pure_hbm_mode());
  int st = 0;
  hkvo_table* o = hkvo_create(cap, cap, 128, dim, HKVO_F32, 4, 0.5f, &st);
  REQUIRE(st == 0);

  std::mt19937_64 rng(42);
  std::vector<uint64_t> keys(n), scores(n);
  std::vector<float> vals(n * dim);
  for (size_t i = 0; i < n; i++) {
    keys[i] = rng() >> 1;
    scores[i] = rng() % 1000;
    for (size_t j = 0; j < dim; j++) vals[i * dim + j] = (float)(rng() % 100000) * 1e-5f;
  }
  uint64_t* dk = dev(keys);
  uint64_t* ds = dev(scores);
  float* dv = dev(vals);
  table.insert_or_assign(n, dk, dv, ds);
  REQUIRE(hkvo_insert_or_assign(o, n, keys.data(), vals.data(), scores.data(), 1, 0, 0) == 0);
  REQUIRE(table.size() == hkvo_size(o));

  // find: founds, rows and scores bit-exact
  std::vector<float> zero(n * dim, 0.f);
  float* dout = dev(zero);
  bool* dfound = nullptr;
  uint64_t* dsc = nullptr;
  hipMalloc(&dfound, n);
  hipMalloc(&dsc, n * 8);
  table.find(n, dk, dout, dfound, dsc);
  hipDeviceSynchronize();
  std::vector<float> ov(n * dim, 0.f);
  std::vector<uint8_t> of(n);
  std::vector<uint64_t> os(n);
  hkvo_find(o, n, keys.data(), ov.data(), of.data(), os.data());
  auto gv = host(dout, n * dim);
  auto gf = host(reinterpret_cast<uint8_t*>(dfound), n);
  auto gs = host(dsc, n);
  REQUIRE(std::memcmp(gv.data(), ov.data(), n * dim * 4) == 0);
  REQUIRE(std::memcmp(gf.data(), of.data(), n) == 0);
  for (size_t i = 0; i < n; i++)
    if (of[i]) REQUIRE(gs[i] == os[i]);

  // erase a third, then export everything (slot order) and compare
  table.erase(n / 3, dk);
  hkvo_erase(o, n / 3, keys.data());
  REQUIRE(table.size() == hkvo_size(o));
  uint64_t* ek = nullptr;
  float* ev = nullptr;
  uint64_t* es = nullptr;
  hipMalloc(&ek, cap * 8);
  hipMalloc(&ev, cap * dim * 4);
  hipMalloc(&es, cap * 8);
  const size_t c = table.export_batch(cap, 0, ek, ev, es);
  std::vector<uint64_t> xk(cap), xs(cap);
  std::vector<float> xv(cap * dim);
  const uint64_t oc = hkvo_export_batch(o, cap, 0, xk.data(), xv.data(), xs.data());
  REQUIRE(c == oc);
  auto hk = host(ek, c);
  auto hv = host(ev, c * dim);
  auto hs = host(es, c);
  REQUIRE(std::memcmp(hk.data(), xk.data(), c * 8) == 0);
  REQUIRE(std::memcmp(hs.data(), xs.data(), c * 8) == 0);
  REQUIRE(std::memcmp(hv.data(), xv.data(), c * dim * 4) == 0);

  // argument check surfaces as HkvException
  bool threw = false;
  try {
    table.insert_or_assign(n, dk, dv, nullptr);
  } catch (const HkvException&) {
    threw = true;
  }
  REQUIRE(threw);
  // save through LocalKVFile: the files hold the slot-order export
  const std::string base = std::string("/tmp/hkv_facade_") + std::to_string((long)getpid());
  const std::string kp = base + ".keys", vp = base + ".values", sp = base + ".scores";
  {
    LocalKVFile<uint64_t, float, uint64_t> f;
    REQUIRE(f.open(kp, vp, sp, "wb"));
    REQUIRE(table.save(&f, 64 * 1024) == c);
  }
  {
    std::vector<uint64_t> fk(c), fs(c);
    std::vector<float> fv(c * dim);
    FILE* a = std::fopen(kp.c_str(), "rb");
    FILE* b = std::fopen(vp.c_str(), "rb");
    FILE* d = std::fopen(sp.c_str(), "rb");
    REQUIRE(a && b && d);
    REQUIRE(std::fread(fk.data(), 8, c, a) == c);
    REQUIRE(std::fread(fv.data(), 4 * dim, c, b) == c);
    REQUIRE(std::fread(fs.data(), 8, c, d) == c);
    std::fclose(a);
    std::fclose(b);
    std::fclose(d);
    REQUIRE(std::memcmp(fk.data(), xk.data(), c * 8) == 0);
    REQUIRE(std::memcmp(fs.data(), xs.data(), c * 8) == 0);
    REQUIRE(std::memcmp(fv.data(), xv.data(), c * dim * 4) == 0);
  }
  // load into a second table: same contents
  {
    Table t2;
    t2.init(opt);
    LocalKVFile<uint64_t, float, uint64_t> f;
    REQUIRE(f.open(kp, vp, sp, "rb"));
    REQUIRE(t2.load(&f, 64 * 1024) == c);
    REQUIRE(t2.size() == c);
    const size_t c2 = t2.export_batch(cap, 0, ek, ev, es);
    REQUIRE(c2 == c);
    // same key set (a probe that wraps around the bucket can place a key
    // elsewhere when the table is rebuilt in slot order)
    auto k2 = host(ek, c2);
    std::vector<uint64_t> a(k2.begin(), k2.end()), b(xk.begin(), xk.begin() + c);
    std::sort(a.begin(), a.end());
    std::sort(b.begin(), b.end());
    REQUIRE(a == b);
  }
  std::remove(kp.c_str());
  std::remove(vp.c_str());
  std::remove(sp.c_str());

  // pointer overloads: find (row addresses), find_or_insert with locked
  // keys, unlock_keys, lock_keys
  {
    float** dptr = nullptr;
    hipMalloc(&dptr, n * sizeof(float*));
    table.find(n, dk, dptr, dfound, dsc);
    hipDeviceSynchronize();
    auto ptrs = host(dptr, n);
    auto pf = host(reinterpret_cast<uint8_t*>(dfound), n);
    std::vector<float> ov2(n * dim, 0.f);
    std::vector<uint8_t> of2(n);
    hkvo_find(o, n, keys.data(), ov2.data(), of2.data(), nullptr);
    REQUIRE(std::memcmp(pf.data(), of2.data(), n) == 0);
    std::vector<float> row(dim);
    for (size_t i = 0; i < n; i += 97) {
      REQUIRE((ptrs[i] != nullptr) == (of2[i] != 0));
      if (!of2[i]) continue;
      hipMemcpy(row.data(), ptrs[i], dim * 4, hipMemcpyDefault);
      REQUIRE(std::memcmp(row.data(), &ov2[i * dim], dim * 4) == 0);
    }
    const size_t m = 256;  // the first half was erased above: misses, then hits
    std::vector<uint64_t> mk(keys.end() - m, keys.end()), msc(m, 7);
    std::copy(keys.begin(), keys.begin() + m / 2, mk.begin());
    uint64_t* dmk = dev(mk);
    uint64_t* dmsc = dev(msc);
    uint64_t** dkp = nullptr;
    hipMalloc(&dkp, m * sizeof(uint64_t*));
    table.find_or_insert(m, dmk, dptr, dfound, dmsc, 0, true, false, dkp);
    hipDeviceSynchronize();
    std::vector<uint64_t> oslot(m);
    std::vector<uint8_t> ofd(m);
    REQUIRE(hkvo_find_or_insert_ptr(o, m, mk.data(), oslot.data(), ofd.data(), msc.data(), 1, 0,
                                    1, 0) == 0);
    auto gfd = host(reinterpret_cast<uint8_t*>(dfound), m);
    REQUIRE(std::memcmp(gfd.data(), ofd.data(), m) == 0);
    auto kps = host(dkp, m);
    for (size_t i = 0; i < m; i++) {
      REQUIRE((kps[i] != nullptr) == (oslot[i] != HKVO_NO_SLOT));
      if (!kps[i]) continue;
      uint64_t w = 0;
      hipMemcpy(&w, kps[i], 8, hipMemcpyDefault);
      REQUIRE(w == 0xFFFFFFFFFFFFFFFDull);
    }
    table.unlock_keys(m, dkp, dmk, dfound);
    hipDeviceSynchronize();
    REQUIRE(hkvo_unlock_keys(o, m, oslot.data(), mk.data(), ofd.data()) == 0);
    gfd = host(reinterpret_cast<uint8_t*>(dfound), m);
    REQUIRE(std::memcmp(gfd.data(), ofd.data(), m) == 0);
    table.lock_keys(m, dmk, dkp, dfound, 0, dmsc);
    table.unlock_keys(m, dkp, dmk);
    hipDeviceSynchronize();
    gfd = host(reinterpret_cast<uint8_t*>(dfound), m);
    REQUIRE(hkvo_lock_keys(o, m, mk.data(), oslot.data(), ofd.data(), msc.data(), 0) == 0);
    REQUIRE(std::memcmp(gfd.data(), ofd.data(), m) == 0);
    REQUIRE(hkvo_unlock_keys(o, m, oslot.data(), mk.data(), nullptr) == 0);
    REQUIRE(table.size() == hkvo_size(o));
  }

  hkvo_destroy(o);
  std::printf("facade parity ok: %zu keys, %zu exported\n", (size_t)table.size(), c);
  return 0;
}
