// hkv_table.hip -- host side of the gfx950 HierarchicalKV table: lifecycle,
// value slices (HBM or pinned host), argument checks and the C ABI declared
// in include/hkv_amd.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/hkv_amd.h"
#include "../../include/hkv_device_ops.hpp"
#include "hkv_kernels.h"

using namespace hkv;

namespace {

thread_local std::string g_last_error;

struct HkvError {
  int code;
  std::string msg;
};

[[noreturn]] void fail(int code, const std::string& msg) { throw HkvError{code, msg}; }

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fail(HKV_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
  }
}

int value_size(int vt) {
  switch (vt) {
    case HKV_F32: case HKV_I32: case HKV_U32: return 4;
    case HKV_F64: case HKV_I64: case HKV_U64: return 8;
    case HKV_F16: case HKV_BF16: case HKV_I16: case HKV_U16: return 2;
    case HKV_I8: case HKV_U8: return 1;
    default: return 0;
  }
}

bool ispow2(uint64_t x) { return x && !(x & (x - 1)); }

uint32_t log2_ceil(uint64_t x) {
  uint32_t s = 0;
  while ((1ull << s) < x) s++;
  return s;
}

// Value slice size (include/table.h:244-268).
uint64_t ref_slice_bytes(uint64_t max_slots, uint64_t B, uint64_t row) {
  const uint64_t GB = 1ull << 30, MB = 1ull << 20;
  const uint64_t min_slice = B * row;
  const uint64_t tbl = max_slots * row;
  uint64_t s;
  if (tbl >= 128 * GB) s = 16 * GB;
  else if (tbl >= 16 * GB) s = 2 * GB;
  else if (tbl >= 2 * GB) s = 128 * MB;
  else if (tbl >= 128 * MB) s = 16 * MB;
  else if (tbl >= 16 * MB) s = MB;
  else s = min_slice;
  return std::max(std::max(min_slice, s), 2 * MB);
}

// Allocation flags of pinned-host value slices.  HKV_HOST_ROWS=coherent or
// noncoherent selects hipHostMallocCoherent / hipHostMallocNonCoherent; the
// default is hipHostMallocDefault.  Only kernels of this library touch the
// rows between calls, and a kernel's completion makes its writes visible
// either way.
unsigned host_row_flags() {
  const char* e = std::getenv("HKV_HOST_ROWS");
  if (e && std::strcmp(e, "coherent") == 0) return hipHostMallocCoherent;
  if (e && std::strcmp(e, "noncoherent") == 0) return hipHostMallocNonCoherent;
  return hipHostMallocDefault;
}

struct Slice {
  uint8_t* host_ptr;  // non-null for pinned host slices
  uint8_t* dev_ptr;
  bool hbm;
};

}  // namespace

// Partition scratch of hkv_insert_or_assign_noalloc: one file-scope array,
// a copy per GPU that each GPU holds until the process ends.  On the host
// the name `scratch` only identifies the symbol; host code uses the device
// address that hipGetSymbolAddress returned for the GPU (noalloc_base).
constexpr uint64_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_base[kMaxDevices] = {};

// Looks up the scratch array's address on `device`, which must be the
// current device, once per device.
void resolve_noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) fail(HKV_ERR_DEVICE, "device id out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_base[device]) return;
  void* p = nullptr;
  hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (!p) fail(HKV_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned null");
  g_scratch_base[device] = static_cast<uint8_t*>(p);
}

uint8_t* noalloc_base(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  uint8_t* p = (device >= 0 && device < kMaxDevices) ? g_scratch_base[device] : nullptr;
  if (!p) fail(HKV_ERR_DEVICE, "the static scratch array was not resolved on this device");
  return p;
}

}  // namespace

struct hkv_table {
  hkv_options opt{};
  int key_type = HKV_KEY_U64;
  int value_type = HKV_F32;
  int strategy = HKV_LRU;
  int device = 0;
  uint64_t B = 128, nb = 0, C = 0, row = 0;
  uint64_t qd_magic = 0, qd_shift = 0;
  bool reach_max = false;
  // Upper bound on the occupancy sum that fast_load_factor reads (the first
  // min(buckets, 1024) bucket sizes), kept on the host so that a call whose
  // bound cannot exceed max_load_factor skips the stream synchronisation of
  // the exact sum; the growth decision is the same either way, since the
  // load factor rises with the sum.  The bound starts from an exact sum and
  // grows by each insert-like call's batch size (a call raises the sum by at
  // most that); erase only lowers the true sum; growth and clear drop it.
  // It is used only while every insert-like call comes on one stream: work
  // queued on another stream before an exact sum would escape the bound.
  uint64_t samp_hi = 0;
  bool samp_ok = false;
  bool samp_off = false;
  bool samp_has_stream = false;
  hipStream_t samp_stream = nullptr;
  uint64_t epoch = kIgnoredEpoch;
  bool clock_override = false;
  uint64_t clock_value = 0;

  uint8_t* digests = nullptr;
  uint64_t* slots = nullptr;  // {key, score} records, 16 bytes per slot
  int32_t* bsize = nullptr;
  uint64_t* live = nullptr;   // live keys, maintained by the kernels

  uint64_t slice_shift = 0;  // buckets per slice = 1 << slice_shift
  uint64_t remaining_hbm = 0;
  std::vector<Slice> slices;
  uint8_t** d_slices = nullptr;
  size_t d_slices_cap = 0;
  bool pure_hbm = true;

  // partitioned apply scratch
  uint32_t part_range = kPartRange;  // partitions per counting pass
  uint32_t* p_hist = nullptr;
  uint64_t p_hist_cap = 0;
  uint64_t* p_ent = nullptr;
  uint64_t p_ent_cap = 0;  // entries
  uint32_t* p_info = nullptr;
  uint64_t p_info_cap = 0;
  uint32_t* p_spill = nullptr;
  uint64_t* p_trow = nullptr;  // zero between calls
  uint64_t p_trow_cap = 0;
  uint32_t* p_list = nullptr;  // partitions left to the multi-run kernel
  uint64_t p_list_cap = 0;
  uint32_t* p_drec = nullptr;
  uint64_t* p_dpool = nullptr;
  uint64_t p_defer_cap = 0;
  uint32_t* p_dctr = nullptr;
  uint32_t* p_evbits = nullptr;  // insert_and_evict record flags (zero between calls)
  uint32_t* p_evwpre = nullptr;
  uint32_t* p_evblk = nullptr;
  uint64_t p_evw_cap = 0;
  BigSlot* p_big = nullptr;
  uint32_t* p_bigpart = nullptr;
  // export scratch
  uint32_t* blk = nullptr;
  uint64_t blk_cap = 0;
  // size scratch
  uint64_t* d_sum = nullptr;
  uint64_t* h_sum = nullptr;

  TableView view() const {
    TableView v{};
    v.digests = digests;
    v.slots = slots;
    v.bsize = bsize;
    v.live = reinterpret_cast<unsigned long long*>(live);
    v.slices = d_slices;
    v.capacity = C;
    v.buckets = nb;
    v.qd_magic = qd_magic;
    v.qd_shift = qd_shift;
    v.B = (uint32_t)B;
    v.bshift = log2_ceil(B);
    v.slice_shift = (uint32_t)slice_shift;
    v.row_bytes = (uint32_t)row;
    v.pow2 = ispow2(C) ? 1u : 0u;
    return v;
  }

  void set_capacity(uint64_t c) {
    C = c;
    // Divisor precomputation (include/table.h:106-127).
    unsigned __int128 one = 1;
    uint64_t s = 0;
    for (s = 0; s < 64; s++)
      if ((one << s) >= c) break;
    unsigned __int128 m = ((one << 64) * ((one << s) - c)) / c + 1;
    qd_magic = (uint64_t)m;
    qd_shift = s - 1;
  }

  // One slice of `nbk` buckets' rows: HBM while the budget lasts, then
  // pinned host memory (include/table.h:130-242).
  Slice alloc_slice(uint64_t nbk) {
    std::vector<Slice> v = alloc_slices({nbk});
    return v[0];
  }

  // Slices of nbk[j] buckets' rows, in order: HBM while the budget lasts,
  // then pinned host memory.  The host slices are allocated by several host
  // threads at once (pinning a fresh 2 GiB takes tens of milliseconds of one
  // core); on any failure every slice of the call is released again.
  std::vector<Slice> alloc_slices(const std::vector<uint64_t>& nbk) {
    std::vector<Slice> out(nbk.size(), Slice{nullptr, nullptr, true});
    std::vector<uint64_t> bytes(nbk.size());
    std::vector<size_t> host;
    uint64_t budget = remaining_hbm;
    for (size_t j = 0; j < nbk.size(); j++) {
      bytes[j] = std::max<uint64_t>(nbk[j] * B * row, 256);
      if (budget >= bytes[j]) budget -= bytes[j];
      else host.push_back(j);
    }
    std::vector<hipError_t> err(nbk.size(), hipSuccess);
    size_t hi = 0;
    for (size_t j = 0; j < nbk.size(); j++) {
      if (hi < host.size() && host[hi] == j) {
        hi++;
        continue;
      }
      err[j] = hipMalloc(&out[j].dev_ptr, bytes[j]);
    }
    const unsigned nth = (unsigned)std::min<size_t>(host.size(), 8);
    auto pin = [&](unsigned w) {
      if (hipSetDevice(device) != hipSuccess) {
        for (size_t q = w; q < host.size(); q += nth) err[host[q]] = hipErrorInvalidDevice;
        return;
      }
      for (size_t q = w; q < host.size(); q += nth) {
        const size_t j = host[q];
        Slice& sl = out[j];
        sl.hbm = false;
        err[j] = hipHostMalloc(&sl.host_ptr, bytes[j], host_row_flags());
        if (err[j] == hipSuccess)
          err[j] = hipHostGetDevicePointer((void**)&sl.dev_ptr, sl.host_ptr, 0);
      }
    };
    if (nth <= 1) {
      if (nth) pin(0);
    } else {
      std::vector<std::thread> th;
      for (unsigned w = 0; w < nth; w++) th.emplace_back(pin, w);
      for (auto& x : th) x.join();
    }
    for (size_t j = 0; j < nbk.size(); j++) {
      if (err[j] == hipSuccess) continue;
      for (auto& sl : out) {
        if (sl.hbm && sl.dev_ptr) (void)hipFree(sl.dev_ptr);
        if (!sl.hbm && sl.host_ptr) (void)hipHostFree(sl.host_ptr);
      }
      (void)hipGetLastError();
      fail(HKV_ERR_DEVICE, std::string(out[j].hbm ? "hipMalloc(values): "
                                                  : "hipHostMalloc(values): ") +
                               hipGetErrorString(err[j]));
    }
    remaining_hbm = budget;
    if (!host.empty()) pure_hbm = false;
    return out;
  }

  // Allocates value rows for buckets [b0, b1).  Slice j holds buckets
  // [j << slice_shift, (j + 1) << slice_shift), which is what row_ptr
  // assumes.  A bucket count that is not a multiple of the slice size leaves
  // the last slice short; growing past it first replaces that slice with a
  // longer one and copies its rows over.
  void add_slices(uint64_t b0, uint64_t b1, hipStream_t st) {
    const uint64_t bps = 1ull << slice_shift;
    uint64_t b = b0;
    if (b0 % bps != 0) {
      const uint64_t sb0 = b0 - b0 % bps;
      if (slices.size() != (sb0 >> slice_shift) + 1)
        fail(HKV_ERR_DEVICE, "value slices out of step with the bucket count");
      const uint64_t have = b0 - sb0, want = std::min(bps, b1 - sb0);
      const Slice old = slices.back();
      // The replacement may take the budget of the slice it replaces.
      if (old.hbm) remaining_hbm += std::max<uint64_t>(have * B * row, 256);
      const Slice ns = alloc_slice(want);
      hip_check(hipMemcpyAsync(ns.dev_ptr, old.dev_ptr, have * B * row, hipMemcpyDefault, st),
                "hipMemcpyAsync(slice rows)");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
      if (old.hbm) (void)hipFree(old.dev_ptr);
      else (void)hipHostFree(old.host_ptr);
      slices.back() = ns;
      b = sb0 + want;
    } else if (slices.size() != (b0 >> slice_shift)) {
      fail(HKV_ERR_DEVICE, "value slices out of step with the bucket count");
    }
    std::vector<uint64_t> nbk;
    for (; b < b1; b += bps) nbk.push_back(std::min(bps, b1 - b));
    for (const Slice& sl : alloc_slices(nbk)) slices.push_back(sl);
    if (slices.size() > d_slices_cap) {
      if (d_slices) hip_check(hipFree(d_slices), "hipFree");
      d_slices_cap = std::max<size_t>(slices.size() * 2, 16);
      hip_check(hipMalloc(&d_slices, d_slices_cap * sizeof(uint8_t*)), "hipMalloc(slices)");
    }
    std::vector<uint8_t*> ptrs;
    for (auto& s : slices) ptrs.push_back(s.dev_ptr);
    hip_check(hipMemcpy(d_slices, ptrs.data(), ptrs.size() * sizeof(uint8_t*),
                        hipMemcpyHostToDevice),
              "hipMemcpy(slices)");
  }

  void free_all() {
    (void)hipFree(digests);
    (void)hipFree(slots);
    (void)hipFree(bsize);
    (void)hipFree(live);
    for (auto& s : slices) {
      if (s.hbm) (void)hipFree(s.dev_ptr);
      else (void)hipHostFree(s.host_ptr);
    }
    slices.clear();
    (void)hipFree(d_slices);
    (void)hipFree(p_hist);
    (void)hipFree(p_ent);
    (void)hipFree(p_info);
    (void)hipFree(p_spill);
    (void)hipFree(p_trow);
    (void)hipFree(p_list);
    (void)hipFree(p_drec);
    (void)hipFree(p_dpool);
    (void)hipFree(p_dctr);
    (void)hipFree(p_evbits);
    (void)hipFree(p_evwpre);
    (void)hipFree(p_evblk);
    (void)hipFree(p_big);
    (void)hipFree(p_bigpart);
    (void)hipFree(blk);
    (void)hipFree(d_sum);
    if (h_sum) (void)hipHostFree(h_sum);
  }

  uint64_t clock_now() const {
    if (clock_override) return clock_value;
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
  }

  // The same scratch carved out of the static array instead (no allocation).
  // Calls on one GPU share the array, so calls that overlap on a GPU race.
  // The row-task region must start at zero and is cleared with a fill kernel;
  // the kernels write every other region before they read it.
  void noalloc_scratch(uint64_t n, PartScratch* ps, hipStream_t s) const {
    const PartLayout L = part_layout(n);
    uint8_t* base = noalloc_base(device);
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
      uint8_t* p = base + off;
      off += (bytes + 255) & ~255ull;
      return p;
    };
    auto* trow = reinterpret_cast<uint64_t*>(take(n * 8));
    auto* hist = reinterpret_cast<uint32_t*>(take(L.hist * 4));
    auto* ent = reinterpret_cast<uint64_t*>(take(L.ent * 16));
    auto* info = reinterpret_cast<uint32_t*>(take(L.info * 4));
    auto* list = reinterpret_cast<uint32_t*>(take(L.np * 4));
    auto* drec = reinterpret_cast<uint32_t*>(take(n * 16));
    auto* dpool = reinterpret_cast<uint64_t*>(take(n * 16));
    auto* dctr = reinterpret_cast<uint32_t*>(take(32));
    auto* spill = reinterpret_cast<uint32_t*>(take(4));
    if (off > kNoAllocScratchBytes)
      fail(HKV_ERR_INVALID,
           "insert_or_assign_noalloc: this batch needs " + std::to_string(off >> 20) +
               " MiB of scratch on this table; the static scratch array holds " +
               std::to_string(kNoAllocScratchBytes >> 20) + " MiB");
    launch_fill_u64(trow, 0, n, s);
    *ps = PartScratch{};
    ps->hist = hist;
    ps->ent = ent;
    ps->pinfo = info;
    ps->spill_top = spill;
    ps->trow = trow;
    ps->plist = list;
    ps->drec = drec;
    ps->dpool = dpool;
    ps->dctr = dctr;
    ps->np = (uint32_t)L.np;
    ps->prange = part_range;
    ps->chunks = (uint32_t)L.ng;
    ps->cap = (uint32_t)L.cap;
  }

  // Sizes of the partitioned apply path's scratch for a batch of n keys.
  // Entries are addressed with 32-bit offsets, which bounds a batch below
  // 2^32 keys.
  struct PartLayout {
    uint64_t np, ng, cap;            // partitions, chunks, fixed region size
    uint64_t hist, ent, info;        // elements of the histogram, entries, info
  };
  PartLayout part_layout(uint64_t n) const {
    PartLayout L{};
    L.np = (nb + kPartBuckets - 1) / kPartBuckets;
    if (n >= (1ull << 32))
      fail(HKV_ERR_UNSUPPORTED, "batches of 2^32 keys or more are not supported");
    L.ng = (n + kPartChunk - 1) / kPartChunk;
    // Fixed region per partition: the mean plus eight standard deviations;
    // a partition that receives more goes to the spill area, which holds n.
    const double mu = std::ceil((double)n / (double)L.np);
    uint64_t cap = (uint64_t)(mu + 8.0 * std::sqrt(mu) + 64.0);
    cap = (cap + 63) & ~63ull;
    if (L.np * cap + n >= (1ull << 32)) cap = 64;
    if (L.np * cap + n >= (1ull << 32))
      fail(HKV_ERR_UNSUPPORTED, "batch and table too large for 32-bit entry offsets");
    L.cap = cap;
    L.hist = L.ng * L.np;
    L.ent = L.np * cap + n;
    L.info = 2 * L.np;
    return L;
  }

  // Scratch of the partitioned apply path for a batch of n keys, owned by
  // the handle and grown on demand.
  void part_scratch(uint64_t n, PartScratch* ps, hipStream_t s) {
    const PartLayout L = part_layout(n);
    const uint64_t np = L.np, ng = L.ng, cap = L.cap;
    const uint64_t hist = L.hist, ent = L.ent, info = L.info;
    if (hist > p_hist_cap) {
      if (p_hist) hip_check(hipFree(p_hist), "hipFree");
      hip_check(hipMalloc(&p_hist, hist * sizeof(uint32_t)), "hipMalloc(part hist)");
      p_hist_cap = hist;
    }
    if (ent > p_ent_cap) {
      if (p_ent) hip_check(hipFree(p_ent), "hipFree");
      hip_check(hipMalloc(&p_ent, ent * 16), "hipMalloc(part entries)");
      p_ent_cap = ent;
    }
    if (info > p_info_cap) {
      if (p_info) hip_check(hipFree(p_info), "hipFree");
      hip_check(hipMalloc(&p_info, info * sizeof(uint32_t)), "hipMalloc(part info)");
      p_info_cap = info;
    }
    if (!p_spill) hip_check(hipMalloc(&p_spill, sizeof(uint32_t)), "hipMalloc(part spill)");
    if (n > p_trow_cap) {
      if (p_trow) hip_check(hipFree(p_trow), "hipFree");
      hip_check(hipMalloc(&p_trow, n * sizeof(uint64_t)), "hipMalloc(part tasks)");
      launch_fill_u64(p_trow, 0, n, s);
      p_trow_cap = n;
    }
    if (np > p_list_cap) {
      if (p_list) hip_check(hipFree(p_list), "hipFree");
      hip_check(hipMalloc(&p_list, np * sizeof(uint32_t)), "hipMalloc(part list)");
      p_list_cap = np;
    }
    if (n > p_defer_cap) {
      if (p_drec) hip_check(hipFree(p_drec), "hipFree");
      if (p_dpool) hip_check(hipFree(p_dpool), "hipFree");
      hip_check(hipMalloc(&p_drec, n * 4 * sizeof(uint32_t)), "hipMalloc(defer records)");
      hip_check(hipMalloc(&p_dpool, n * 16), "hipMalloc(defer pool)");
      p_defer_cap = n;
    }
    if (!p_dctr) hip_check(hipMalloc(&p_dctr, 8 * sizeof(uint32_t)), "hipMalloc(part counters)");
    const uint64_t nw = n / 32 + 1;
    if (nw > p_evw_cap) {
      if (p_evbits) hip_check(hipFree(p_evbits), "hipFree");
      if (p_evwpre) hip_check(hipFree(p_evwpre), "hipFree");
      if (p_evblk) hip_check(hipFree(p_evblk), "hipFree");
      hip_check(hipMalloc(&p_evbits, nw * sizeof(uint32_t)), "hipMalloc(evict flags)");
      hip_check(hipMalloc(&p_evwpre, nw * sizeof(uint32_t)), "hipMalloc(evict prefix)");
      hip_check(hipMalloc(&p_evblk, (nw / 256 + 4) * sizeof(uint32_t)), "hipMalloc(evict blocks)");
      launch_fill_u32(p_evbits, 0, nw, s);
      p_evw_cap = nw;
    }
    *ps = PartScratch{};
    ps->hist = p_hist;
    ps->ent = p_ent;
    ps->pinfo = p_info;
    ps->spill_top = p_spill;
    ps->trow = p_trow;
    ps->plist = p_list;
    ps->drec = p_drec;
    ps->dpool = p_dpool;
    ps->dctr = p_dctr;
    ps->ev_bits = p_evbits;
    ps->ev_wpre = p_evwpre;
    ps->ev_blk = p_evblk;
    ps->np = (uint32_t)np;
    ps->prange = part_range;
    ps->chunks = (uint32_t)ng;
    ps->cap = (uint32_t)cap;
  }

  // State of the big-partition path (batches with repeated keys).
  void big_scratch(PartScratch* ps) {
    if (!p_big) {
      hip_check(hipMalloc(&p_big, kBigMax * sizeof(BigSlot)), "hipMalloc(big partitions)");
      hip_check(hipMalloc(&p_bigpart, kBigMax * sizeof(uint32_t)), "hipMalloc(big partitions)");
    }
    ps->big = p_big;
    ps->big_part = p_bigpart;
  }

  uint64_t sampled_size(hipStream_t s) {
    const uint64_t N = std::min<uint64_t>(nb, 1024);
    launch_fill_u64(d_sum, 0, 1, s);
    launch_size(view(), N, d_sum, s);
    hip_check(hipMemcpyAsync(h_sum, d_sum, sizeof(uint64_t), hipMemcpyDeviceToHost, s),
              "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    return *h_sum;
  }

  // fast_load_factor (include/hkv_hashtable.h:3229-3268) for a given sum of
  // the first min(buckets, 1024) bucket sizes.
  float fast_load_factor_of(uint64_t delta, uint64_t tot) const {
    const uint64_t N = std::min<uint64_t>(nb, 1024);
    return (float)((delta * 1.0) / (C * 1.0) + (tot * 1.0) / (B * N * 1.0));
  }

  // Every insert-like call passes its stream here; a second stream turns
  // the host-side bound off for the table's lifetime.
  void note_stream(hipStream_t s) {
    if (!samp_has_stream) {
      samp_has_stream = true;
      samp_stream = s;
    } else if (s != samp_stream) {
      samp_off = true;
    }
  }

  // After an insert-like call of n keys has been queued.
  void note_insert(uint64_t n) {
    const uint64_t most = B * std::min<uint64_t>(nb, 1024);
    samp_hi = (n >= most - std::min(samp_hi, most)) ? most : samp_hi + n;
  }

  void double_capacity(hipStream_t s) {
    // include/table.h:360-377 followed by the rehash kernel.
    const uint64_t old_nb = nb, old_C = C;
    uint8_t* nd = nullptr;
    uint64_t* nsl = nullptr;
    int32_t* nbs = nullptr;
    hip_check(hipMalloc(&nd, 2 * old_C), "hipMalloc(digests)");
    hip_check(hipMalloc(&nsl, 2 * old_C * 16), "hipMalloc(slots)");
    hip_check(hipMalloc(&nbs, 2 * old_nb * 4), "hipMalloc(bsize)");
    hip_check(hipMemcpyAsync(nd, digests, old_C, hipMemcpyDeviceToDevice, s), "copy");
    hip_check(hipMemcpyAsync(nsl, slots, old_C * 16, hipMemcpyDeviceToDevice, s), "copy");
    hip_check(hipMemcpyAsync(nbs, bsize, old_nb * 4, hipMemcpyDeviceToDevice, s), "copy");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    (void)hipFree(digests);
    (void)hipFree(slots);
    (void)hipFree(bsize);
    digests = nd;
    slots = nsl;
    bsize = nbs;
    nb = 2 * old_nb;
    samp_ok = false;
    set_capacity(2 * old_C);
    add_slices(old_nb, nb, s);
    launch_init_slots(view(), old_nb, nb, s);
    // Metadata first, with the row moves recorded; then the rows.
    RehashScratch rs{};
    uint8_t* stage = nullptr;
    bool stage_host = false;
    try {
      hip_check(hipMalloc(&rs.rec, old_C * sizeof(uint16_t)), "hipMalloc(rehash records)");
      hip_check(hipMalloc(&rs.cnt, old_nb * sizeof(uint16_t)), "hipMalloc(rehash counts)");
      hip_check(hipMalloc(&rs.tbase, old_nb * sizeof(uint32_t)), "hipMalloc(rehash bases)");
      hip_check(hipMalloc(&rs.tcount, sizeof(uint32_t)), "hipMalloc(rehash counter)");
      launch_fill_u32(rs.tcount, 0, 1, s);
      launch_rehash_plan(view(), old_nb, rs, s);
      hip_check(hipGetLastError(), "rehash launch");
      uint32_t staged = 0;
      hip_check(hipMemcpyAsync(&staged, rs.tcount, sizeof(staged), hipMemcpyDeviceToHost, s),
                "hipMemcpyAsync");
      hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
      if (staged) {
        // Rows that stay in their bucket pass through a staging buffer: HBM
        // when it can be had, else pinned host memory.
        if (hipMalloc(&stage, (uint64_t)staged * row) != hipSuccess) {
          (void)hipGetLastError();
          hip_check(hipHostMalloc(&stage, (uint64_t)staged * row, hipHostMallocDefault),
                    "hipHostMalloc(rehash staging)");
          stage_host = true;
        }
      }
      const int unit = value_unit(nullptr);
      launch_rehash_rows(view(), old_nb, rs, stage, 0, unit, s);
      if (staged) launch_rehash_rows(view(), old_nb, rs, stage, 1, unit, s);
      hip_check(hipGetLastError(), "rehash launch");
      hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    } catch (...) {
      (void)hipFree(rs.rec);
      (void)hipFree(rs.cnt);
      (void)hipFree(rs.tbase);
      (void)hipFree(rs.tcount);
      if (stage) (void)(stage_host ? hipHostFree(stage) : hipFree(stage));
      throw;
    }
    (void)hipFree(rs.rec);
    (void)hipFree(rs.cnt);
    (void)hipFree(rs.tbase);
    (void)hipFree(rs.tcount);
    if (stage) (void)(stage_host ? hipHostFree(stage) : hipFree(stage));
  }

  // include/hkv_hashtable.h:2873-2935
  void reserve(uint64_t new_cap, hipStream_t s) {
    if (reach_max || new_cap > opt.max_capacity) {
      reach_max = (C * 2 > opt.max_capacity);
      return;
    }
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    while (C < new_cap && C * 2 <= opt.max_capacity) double_capacity(s);
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    reach_max = (C * 2 > opt.max_capacity);
  }

  // The auto-grow loop of the insert-like calls (include/hkv_hashtable.h:
  // 1103-1106, 1278-1281, 1456-1459, 1535-1538, 1669-1672), then the bound
  // update.
  void maybe_grow(uint64_t n, hipStream_t s) {
    note_stream(s);
    while (!reach_max) {
      if (samp_ok && !samp_off && fast_load_factor_of(n, samp_hi) <= opt.max_load_factor)
        break;
      const uint64_t tot = sampled_size(s);
      samp_hi = tot;
      samp_ok = true;
      if (fast_load_factor_of(n, tot) <= opt.max_load_factor) break;
      reserve(C * 2, s);
    }
    note_insert(n);
  }

  // check_evict_strategy (include/hkv_hashtable.h:3270-3298), plus a check
  // that strategies which read input scores receive them.
  void check_scores(int st, const uint64_t* sc, bool ignore) const {
    if (!ignore) {
      if ((st == HKV_LRU || st == HKV_EPOCH_LRU) && sc)
        fail(HKV_ERR_INVALID,
             "the scores should not be specified when running on LRU or Epoch LRU mode.");
      if ((st == HKV_LFU || st == HKV_EPOCH_LFU) && !sc)
        fail(HKV_ERR_INVALID,
             "the scores should be specified when running on LFU or Epoch LFU mode.");
      if (st == HKV_CUSTOMIZED && !sc)
        fail(HKV_ERR_INVALID,
             "the scores should be specified when running on customized mode.");
      if ((st == HKV_EPOCH_LRU || st == HKV_EPOCH_LFU) && epoch == kIgnoredEpoch)
        fail(HKV_ERR_INVALID,
             "the global_epoch is invalid and should be assigned by calling "
             "`set_global_epoch` when running on Epoch LRU or Epoch LFU mode.");
    } else if ((st == HKV_LFU || st == HKV_EPOCH_LFU || st == HKV_CUSTOMIZED) && !sc) {
      fail(HKV_ERR_INVALID, "this evict strategy reads input scores; scores is null.");
    }
  }

  // Largest copy unit dividing the row size and the alignment of `p`.
  int value_unit(const void* p) const {
    uint64_t a = (uint64_t)(uintptr_t)p | row;
    if (p == nullptr) a = row;
    for (int u = 16; u > 1; u >>= 1)
      if ((a & (u - 1)) == 0) return u;
    return 1;
  }
};

namespace {

template <class F>
int guarded(F&& f) {
  try {
    f();
    return HKV_OK;
  } catch (const HkvError& e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return HKV_ERR_DEVICE;
  } catch (...) {
    g_last_error = "unknown error";
    return HKV_ERR_DEVICE;
  }
}

void need_table(const hkv_table* t) {
  if (!t) fail(HKV_ERR_INVALID, "null table handle");
}

hipStream_t S(hkv_stream s) { return reinterpret_cast<hipStream_t>(s); }

int min_unit(const hkv_table* t, std::initializer_list<const void*> ps) {
  int u = 16;
  for (const void* p : ps)
    if (p) u = std::min(u, t->value_unit(p));
  return std::min(u, t->value_unit(nullptr));
}

int insert_like(hkv_table* t, int op, uint64_t n, const void* keys, const void* in_values,
                void* io_values, const uint64_t* scores, const uint8_t* accum,
                void* ev_keys, void* ev_values, uint64_t* ev_scores, uint64_t* ev_counter,
                int strategy, int rule, hipStream_t s, const PartScratch* given = nullptr) {
  ApplyArgs a{};
  a.keys = reinterpret_cast<const uint64_t*>(keys);
  a.in_values = reinterpret_cast<const uint8_t*>(in_values);
  a.io_values = reinterpret_cast<uint8_t*>(io_values);
  a.in_scores = scores;
  a.accum_flags = accum;
  a.ev_keys = reinterpret_cast<uint64_t*>(ev_keys);
  a.ev_values = reinterpret_cast<uint8_t*>(ev_values);
  a.ev_scores = ev_scores;
  a.ev_counter = ev_counter;
  a.n = n;
  a.sc.strategy = strategy;
  a.sc.epoch = t->epoch;
  a.sc.clock = t->clock_now();
  a.rule = rule;
  a.unit = min_unit(t, {in_values, io_values, ev_values});
  a.value_type = t->value_type;
  PartScratch ps{};
  if (given) {
    ps = *given;
  } else {
    t->part_scratch(n, &ps, s);
    // Batches with repeated keys may hold hot keys: their big partitions
    // are counted and folded grid-wide (accum_or_assign accumulates in
    // batch order inside one block instead).
    if (rule == RULE_TILE32 && op != OP_ACCUM_OR_ASSIGN) t->big_scratch(&ps);
  }
  if (op == OP_INSERT_AND_EVICT) a.ev_bits = ps.ev_bits;
  launch_apply_part(t->view(), op, a, ps, s);
  hip_check(hipGetLastError(), "kernel launch");
  return HKV_OK;
}

}  // namespace

extern "C" {

void hkv_options_default(hkv_options* o) {
  std::memset(o, 0, sizeof(*o));
  o->max_bucket_size = 128;
  o->dim = 64;
  o->max_load_factor = 0.5f;
  o->block_size = 128;
  o->io_block_size = 1024;
  o->device_id = -1;
  o->num_of_buckets_per_alloc = 1;
}

int hkv_create(const hkv_options* o, int key_type, int value_type, int strategy,
               hkv_table** out) {
  return guarded([&] {
    if (!o || !out) fail(HKV_ERR_INVALID, "null argument");
    *out = nullptr;
    if (key_type != HKV_KEY_U64 && key_type != HKV_KEY_I64)
      fail(HKV_ERR_INVALID, "The key_type must be int64_t or uint64_t.");
    if (value_size(value_type) == 0) fail(HKV_ERR_INVALID, "unknown value type");
    if (strategy < HKV_LRU || strategy > HKV_CUSTOMIZED)
      fail(HKV_ERR_INVALID, "unknown evict strategy");
    // include/hkv_hashtable.h:991-1024
    if (o->reserved_key_start_bit < 0 || o->reserved_key_start_bit > 62)
      fail(HKV_ERR_INVALID, "options.reserved_key_start_bit should >= 0 and <= 62.");
    if (o->max_bucket_size < 16)
      fail(HKV_ERR_INVALID, "Bucket size should be greater than or equal to 16");
    if (!ispow2(o->max_bucket_size)) fail(HKV_ERR_INVALID, "Bucket size should be the pow of 2");
    if (!ispow2(o->num_of_buckets_per_alloc))
      fail(HKV_ERR_INVALID, "Then `num_of_buckets_per_alloc` should be the pow of 2");
    if (o->init_capacity < o->num_of_buckets_per_alloc * o->max_bucket_size)
      fail(HKV_ERR_INVALID,
           "Then `num_of_buckets_per_alloc` must be equal or less than initial required "
           "buckets number");
    if ((o->max_bucket_size * 16) % 128 != 0)
      fail(HKV_ERR_INVALID,
           "Storage size of keys and scores in one bucket should be the mutiple of cache "
           "line size");
    if (o->io_by_cpu && o->max_hbm_for_vectors != 0)
      fail(HKV_ERR_INVALID,
           "[HierarchicalKV] `io_by_cpu` should not be true when `max_hbm_for_vectors` is not 0!");
    if (o->io_by_cpu) fail(HKV_ERR_UNSUPPORTED, "io_by_cpu is not supported by this build");
    if (o->api_lock) fail(HKV_ERR_UNSUPPORTED, "api_lock is not supported by this build");
    if (o->max_bucket_size != 128)
      fail(HKV_ERR_UNSUPPORTED, "this build supports max_bucket_size == 128");
    if (o->dim == 0) fail(HKV_ERR_INVALID, "dim must be positive");

    auto* t = new hkv_table();
    t->opt = *o;
    t->key_type = key_type;
    t->value_type = value_type;
    t->strategy = strategy;
    t->B = o->max_bucket_size;
    t->row = o->dim * (uint64_t)value_size(value_type);
    // Test knob: fewer partitions per counting pass, so that small tables
    // take the multi-pass counting path of very large ones.
    if (const char* r = std::getenv("HKV_PART_RANGE")) {
      const long v = std::strtol(r, nullptr, 10);
      if (v >= 1 && v <= (long)kPartRange) t->part_range = (uint32_t)v;
    }
    try {
      if (o->device_id >= 0) {
        hip_check(hipSetDevice(o->device_id), "hipSetDevice");
        t->device = o->device_id;
      } else {
        hip_check(hipGetDevice(&t->device), "hipGetDevice");
        t->opt.device_id = t->device;
      }
      const uint64_t maxc = std::max(o->init_capacity, o->max_capacity);
      t->opt.max_capacity = maxc;
      // create_table bucket count (include/table.h:299-311).
      if (o->init_capacity * 2 > maxc) {
        t->nb = 1 + (maxc - 1) / t->B;
      } else {
        t->nb = 1;
        while (t->nb * t->B < o->init_capacity) t->nb *= 2;
      }
      t->set_capacity(t->nb * t->B);
      t->reach_max = (o->init_capacity * 2 > maxc);
      // Value slices: one slice for everything when it all fits in HBM,
      // otherwise power-of-two bucket groups of about the reference's slice
      // size.
      t->remaining_hbm = o->max_hbm_for_vectors;
      const uint64_t all_bytes = t->nb * t->B * t->row;
      if (t->remaining_hbm >= all_bytes) {
        t->slice_shift = log2_ceil(t->nb);
      } else {
        const uint64_t sb = ref_slice_bytes(maxc, t->B, t->row);
        uint64_t bps = std::max<uint64_t>(1, sb / (t->B * t->row));
        uint32_t sh = 0;
        while ((2ull << sh) <= bps) sh++;
        t->slice_shift = std::min<uint64_t>(sh, log2_ceil(t->nb));
      }
      hip_check(hipMalloc(&t->digests, t->C), "hipMalloc(digests)");
      hip_check(hipMalloc(&t->slots, t->C * 16), "hipMalloc(slots)");
      hip_check(hipMalloc(&t->bsize, t->nb * 4), "hipMalloc(bsize)");
      hip_check(hipMalloc(&t->live, sizeof(uint64_t)), "hipMalloc(live)");
      hip_check(hipMalloc(&t->d_sum, sizeof(uint64_t)), "hipMalloc(sum)");
      hip_check(hipHostMalloc(&t->h_sum, sizeof(uint64_t), hipHostMallocDefault),
                "hipHostMalloc(sum)");
      resolve_noalloc_scratch(t->device);
      t->add_slices(0, t->nb, 0);
      launch_init_slots(t->view(), 0, t->nb, 0);
      launch_fill_u64(t->live, 0, 1, 0);
      hip_check(hipGetLastError(), "init launch");
      hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    } catch (...) {
      t->free_all();
      delete t;
      throw;
    }
    *out = t;
  });
}

int hkv_destroy(hkv_table* t) {
  return guarded([&] {
    if (!t) return;
    (void)hipDeviceSynchronize();
    t->free_all();
    delete t;
  });
}

int hkv_insert_or_assign(hkv_table* t, uint64_t n, const void* keys, const void* values,
                         const uint64_t* scores, hkv_stream stream, int unique_key,
                         int ignore_evict_strategy) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1077-1215: ignore_evict_strategy instantiates
    // the kCustomized functor for this call.
    const int st = ignore_evict_strategy ? HKV_CUSTOMIZED : t->strategy;
    if (n == 0) return;
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    t->maybe_grow(n, S(stream));
    t->check_scores(st, scores, ignore_evict_strategy != 0);
    insert_like(t, OP_INSERT_OR_ASSIGN, n, keys, values, nullptr, scores, nullptr, nullptr,
                nullptr, nullptr, nullptr, st, unique_key ? RULE_DIGEST16 : RULE_TILE32,
                S(stream));
  });
}

int hkv_insert_or_assign_noalloc(hkv_table* t, uint64_t n, const void* keys,
                                 const void* values, const uint64_t* scores, hkv_stream stream,
                                 int unique_key, int ignore_evict_strategy) {
  return guarded([&] {
    need_table(t);
    const int st = ignore_evict_strategy ? HKV_CUSTOMIZED : t->strategy;
    if (n == 0) return;
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    if (!t->reach_max)
      fail(HKV_ERR_INVALID,
           "insert_or_assign_noalloc needs a table at its maximum capacity "
           "(growing the table allocates)");
    t->check_scores(st, scores, ignore_evict_strategy != 0);
    t->note_stream(S(stream));
    t->note_insert(n);
    PartScratch ps{};
    t->noalloc_scratch(n, &ps, S(stream));
    insert_like(t, OP_INSERT_OR_ASSIGN, n, keys, values, nullptr, scores, nullptr, nullptr,
                nullptr, nullptr, nullptr, st, unique_key ? RULE_DIGEST16 : RULE_TILE32,
                S(stream), &ps);
  });
}

int hkv_insert_and_evict(hkv_table* t, uint64_t n, const void* keys, const void* values,
                         const uint64_t* scores, void* evicted_keys, void* evicted_values,
                         uint64_t* evicted_scores, uint64_t* d_evicted_counter,
                         hkv_stream stream, int unique_key, int ignore_evict_strategy) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1260-1324
    if (n == 0) return;
    if (!keys || !values || !evicted_keys || !evicted_values || !d_evicted_counter) return;
    t->maybe_grow(n, S(stream));
    t->check_scores(t->strategy, scores, ignore_evict_strategy != 0);
    if (!t->pure_hbm) fail(HKV_ERR_RUNTIME, "Only allow insert_and_evict in pure HBM mode.");
    insert_like(t, OP_INSERT_AND_EVICT, n, keys, values, nullptr, scores, nullptr,
                evicted_keys, evicted_values, evicted_scores, d_evicted_counter, t->strategy,
                unique_key ? RULE_DIGEST16 : RULE_TILE32, S(stream));
  });
}

int hkv_accum_or_assign(hkv_table* t, uint64_t n, const void* keys, const void* vals,
                        const uint8_t* accum, const uint64_t* scores, hkv_stream stream,
                        int ignore_evict_strategy) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1438-1507
    if (t->value_type == HKV_F64 || t->value_type == HKV_U16 || t->value_type == HKV_U32)
      fail(HKV_ERR_RUNTIME,
           "[accum_or_assign] Does not support double/uint16_t/uint32_t value_type.");
    if (!(t->value_type == HKV_F32 || t->value_type == HKV_I32 || t->value_type == HKV_I64 ||
          t->value_type == HKV_U64))
      fail(HKV_ERR_UNSUPPORTED, "accum_or_assign supports f32/i32/i64/u64 values in this build");
    if (n == 0) return;
    if (!keys || !vals || !accum) fail(HKV_ERR_INVALID, "null argument");
    t->maybe_grow(n, S(stream));
    t->check_scores(t->strategy, scores, ignore_evict_strategy != 0);
    insert_like(t, OP_ACCUM_OR_ASSIGN, n, keys, vals, nullptr, scores, accum, nullptr, nullptr,
                nullptr, nullptr, t->strategy, RULE_TILE32, S(stream));
  });
}

int hkv_find_or_insert(hkv_table* t, uint64_t n, const void* keys, void* values,
                       const uint64_t* scores, hkv_stream stream, int unique_key,
                       int ignore_evict_strategy) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1526-1632
    if (n == 0) return;
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    t->maybe_grow(n, S(stream));
    t->check_scores(t->strategy, scores, ignore_evict_strategy != 0);
    insert_like(t, OP_FIND_OR_INSERT, n, keys, values, values, scores, nullptr, nullptr,
                nullptr, nullptr, nullptr, t->strategy,
                unique_key ? RULE_DIGEST16 : RULE_TILE32, S(stream));
  });
}

int hkv_assign_scores(hkv_table* t, uint64_t n, const void* keys, const uint64_t* scores,
                      hkv_stream stream, int unique_key) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1943-1977
    (void)unique_key;
    if (n == 0) return;
    t->check_scores(t->strategy, scores, false);
    if (!keys) fail(HKV_ERR_INVALID, "keys must not be null");
    insert_like(t, OP_ASSIGN_SCORES, n, keys, nullptr, nullptr, scores, nullptr, nullptr,
                nullptr, nullptr, nullptr, t->strategy, RULE_DIGEST16, S(stream));
  });
}

int hkv_find(hkv_table* t, uint64_t n, const void* keys, void* values, uint8_t* founds,
             uint64_t* scores, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    if (n == 0) return;
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    launch_find(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                reinterpret_cast<uint8_t*>(values), founds, scores, t->value_unit(values),
                S(stream));
    hip_check(hipGetLastError(), "find launch");
  });
}

int hkv_find_missed(hkv_table* t, uint64_t n, const void* keys, void* values,
                    void* missed_keys, int32_t* missed_indices, int32_t* missed_size,
                    uint64_t* scores, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    if (n == 0) return;
    if (!keys || !values || !missed_keys || !missed_indices || !missed_size)
      fail(HKV_ERR_INVALID, "null argument");
    launch_fill_u32(reinterpret_cast<uint32_t*>(missed_size), 0, 1, S(stream));
    launch_find_missed(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                       reinterpret_cast<uint8_t*>(values),
                       reinterpret_cast<uint64_t*>(missed_keys), missed_indices, missed_size,
                       scores, t->value_unit(values), S(stream));
    hip_check(hipGetLastError(), "find launch");
  });
}

int hkv_erase(hkv_table* t, uint64_t n, const void* keys, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    if (n == 0) return;
    if (!keys) fail(HKV_ERR_INVALID, "keys must not be null");
    launch_erase(t->view(), reinterpret_cast<const uint64_t*>(keys), n, S(stream));
    hip_check(hipGetLastError(), "erase launch");
  });
}

int hkv_clear(hkv_table* t, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    t->samp_ok = false;
    launch_clear(t->view(), S(stream));
    hip_check(hipGetLastError(), "clear launch");
  });
}

int hkv_export_batch(hkv_table* t, uint64_t n, uint64_t offset, uint64_t* d_counter,
                     void* keys, void* values, uint64_t* scores, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    if (!d_counter) fail(HKV_ERR_INVALID, "d_counter must not be null");
    launch_fill_u64(d_counter, 0, 1, S(stream));
    if (offset >= t->C) return;
    n = std::min(t->C - offset, n);
    if (n == 0) return;
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    const uint64_t nblk = (n + 255) / 256;
    if (nblk > t->blk_cap) {
      if (t->blk) hip_check(hipFree(t->blk), "hipFree");
      hip_check(hipMalloc(&t->blk, nblk * sizeof(uint32_t)), "hipMalloc(export)");
      t->blk_cap = nblk;
    }
    launch_export(t->view(), offset, n, d_counter, reinterpret_cast<uint64_t*>(keys),
                  reinterpret_cast<uint8_t*>(values), scores, t->blk, t->value_unit(values),
                  S(stream));
    hip_check(hipGetLastError(), "export launch");
  });
}

int hkv_reserve(hkv_table* t, uint64_t new_capacity, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    t->reserve(new_capacity, S(stream));
  });
}

namespace {

// Host and device buffers of one save/load chunk.
struct KvChunk {
  uint64_t* h_keys = nullptr;
  uint64_t* h_scores = nullptr;
  uint8_t* h_values = nullptr;
  uint64_t* d_keys = nullptr;
  uint64_t* d_scores = nullptr;
  uint8_t* d_values = nullptr;
  uint64_t* d_count = nullptr;
  KvChunk(uint64_t n, uint64_t row) {
    hip_check(hipHostMalloc(&h_keys, n * 8, hipHostMallocDefault), "hipHostMalloc(kv keys)");
    hip_check(hipHostMalloc(&h_scores, n * 8, hipHostMallocDefault), "hipHostMalloc(kv scores)");
    hip_check(hipHostMalloc(&h_values, n * row, hipHostMallocDefault), "hipHostMalloc(kv rows)");
    hip_check(hipMalloc(&d_keys, n * 8), "hipMalloc(kv keys)");
    hip_check(hipMalloc(&d_scores, n * 8), "hipMalloc(kv scores)");
    hip_check(hipMalloc(&d_values, n * row), "hipMalloc(kv rows)");
    hip_check(hipMalloc(&d_count, 8), "hipMalloc(kv count)");
  }
  ~KvChunk() {
    (void)hipHostFree(h_keys);
    (void)hipHostFree(h_scores);
    (void)hipHostFree(h_values);
    (void)hipFree(d_keys);
    (void)hipFree(d_scores);
    (void)hipFree(d_values);
    (void)hipFree(d_count);
  }
};

uint64_t kv_chunk_records(const hkv_table* t, uint64_t max_workspace_size) {
  const uint64_t tuple = 8 + 8 + t->row;  // key + score + row
  if (max_workspace_size < tuple)
    fail(HKV_ERR_INVALID,
         "max_workspace_size is smaller than a single key + score + value tuple");
  return max_workspace_size / tuple;
}

void ok_or_throw(int rc) {
  if (rc != HKV_OK) throw HkvError{rc, g_last_error};
}

}  // namespace

int hkv_save(hkv_table* t, hkv_kv_write_fn write, void* ctx, uint64_t max_workspace_size,
             hkv_stream stream, uint64_t* count) {
  return guarded([&] {
    need_table(t);
    if (!write || !count) fail(HKV_ERR_INVALID, "write and count must not be null");
    const hipStream_t s = S(stream);
    const uint64_t total = t->C;
    const uint64_t n = std::min(kv_chunk_records(t, max_workspace_size), total);
    KvChunk c(n, t->row);
    uint64_t written = 0;
    for (uint64_t i = 0; i < total; i += n) {
      const uint64_t m = std::min(total - i, n);
      ok_or_throw(hkv_export_batch(t, m, i, c.d_count, c.d_keys, c.d_values, c.d_scores, stream));
      uint64_t got = 0;
      hip_check(hipMemcpyAsync(&got, c.d_count, 8, hipMemcpyDeviceToHost, s), "hipMemcpy(count)");
      hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
      if (got == 0) continue;
      hip_check(hipMemcpyAsync(c.h_keys, c.d_keys, got * 8, hipMemcpyDeviceToHost, s), "hipMemcpy");
      hip_check(hipMemcpyAsync(c.h_scores, c.d_scores, got * 8, hipMemcpyDeviceToHost, s),
                "hipMemcpy");
      hip_check(hipMemcpyAsync(c.h_values, c.d_values, got * t->row, hipMemcpyDeviceToHost, s),
                "hipMemcpy");
      hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
      write(ctx, got, t->row, c.h_keys, c.h_values, c.h_scores);
      written += got;
    }
    *count = written;
  });
}

int hkv_load(hkv_table* t, hkv_kv_read_fn read, void* ctx, uint64_t max_workspace_size,
             hkv_stream stream, uint64_t* count) {
  return guarded([&] {
    need_table(t);
    if (!read || !count) fail(HKV_ERR_INVALID, "read and count must not be null");
    const hipStream_t s = S(stream);
    const uint64_t n = kv_chunk_records(t, max_workspace_size);
    KvChunk c(n, t->row);
    uint64_t loaded = 0;
    uint64_t got = read(ctx, n, t->row, c.h_keys, c.h_values, c.h_scores);
    while (got > 0) {
      hip_check(hipMemcpyAsync(c.d_keys, c.h_keys, got * 8, hipMemcpyHostToDevice, s), "hipMemcpy");
      hip_check(hipMemcpyAsync(c.d_scores, c.h_scores, got * 8, hipMemcpyHostToDevice, s),
                "hipMemcpy");
      hip_check(hipMemcpyAsync(c.d_values, c.h_values, got * t->row, hipMemcpyHostToDevice, s),
                "hipMemcpy");
      t->epoch = kIgnoredEpoch;  // include/hkv_hashtable.h:3182
      ok_or_throw(hkv_insert_or_assign(t, got, c.d_keys, c.d_values, c.d_scores, stream, 1, 1));
      loaded += got;
      hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
      got = read(ctx, n, t->row, c.h_keys, c.h_values, c.h_scores);
    }
    *count = loaded;
  });
}

struct hkv_local_kv_file {
  FILE* keys = nullptr;
  FILE* values = nullptr;
  FILE* scores = nullptr;
};

hkv_local_kv_file* hkv_local_kv_file_open(const char* keys_path, const char* values_path,
                                          const char* scores_path, const char* mode) {
  if (!keys_path || !values_path || !scores_path || !mode) return nullptr;
  auto* f = new hkv_local_kv_file();
  f->keys = fopen(keys_path, mode);
  f->values = f->keys ? fopen(values_path, mode) : nullptr;
  f->scores = f->values ? fopen(scores_path, mode) : nullptr;
  if (!f->scores) {
    hkv_local_kv_file_close(f);
    return nullptr;
  }
  return f;
}

void hkv_local_kv_file_close(hkv_local_kv_file* f) {
  if (!f) return;
  if (f->keys) fclose(f->keys);
  if (f->values) fclose(f->values);
  if (f->scores) fclose(f->scores);
  delete f;
}

uint64_t hkv_local_kv_file_write(void* fp, uint64_t n, uint64_t row_bytes, const void* keys,
                                 const void* values, const uint64_t* scores) {
  auto* f = static_cast<hkv_local_kv_file*>(fp);
  const size_t nk = fwrite(keys, 8, n, f->keys);
  const size_t nv = fwrite(values, row_bytes, n, f->values);
  const size_t ns = fwrite(scores, 8, n, f->scores);
  return (nk == nv && nk == ns) ? nk : 0;
}

uint64_t hkv_local_kv_file_read(void* fp, uint64_t n, uint64_t row_bytes, void* keys,
                                void* values, uint64_t* scores) {
  auto* f = static_cast<hkv_local_kv_file*>(fp);
  const size_t nk = fread(keys, 8, n, f->keys);
  const size_t nv = fread(values, row_bytes, n, f->values);
  const size_t ns = fread(scores, 8, n, f->scores);
  return (nk == nv && nk == ns) ? nk : 0;
}

int hkv_set_global_epoch(hkv_table* t, uint64_t epoch) {
  return guarded([&] {
    need_table(t);
    t->epoch = epoch;
  });
}

int hkv_size(hkv_table* t, hkv_stream stream, uint64_t* out) {
  return guarded([&] {
    need_table(t);
    if (!out) fail(HKV_ERR_INVALID, "null output");
    launch_fill_u64(t->d_sum, 0, 1, S(stream));
    launch_size(t->view(), t->nb, t->d_sum, S(stream));
    hip_check(hipMemcpyAsync(t->h_sum, t->d_sum, sizeof(uint64_t), hipMemcpyDeviceToHost,
                             S(stream)),
              "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
    *out = *t->h_sum;
  });
}

int hkv_load_factor(hkv_table* t, hkv_stream stream, float* out) {
  uint64_t sz = 0;
  const int rc = hkv_size(t, stream, &sz);
  if (rc == HKV_OK) *out = (float)((sz * 1.0) / (t->C * 1.0));
  return rc;
}

uint64_t hkv_capacity(const hkv_table* t) { return t ? t->C : 0; }
uint64_t hkv_dim(const hkv_table* t) { return t ? t->opt.dim : 0; }
uint64_t hkv_max_bucket_size(const hkv_table* t) { return t ? t->B : 0; }
uint64_t hkv_bucket_count(const hkv_table* t) { return t ? t->nb : 0; }
int hkv_is_pure_hbm_mode(const hkv_table* t) { return t && t->pure_hbm ? 1 : 0; }
const char* hkv_last_error(void) { return g_last_error.c_str(); }

int hkv_set_lru_clock(hkv_table* t, uint64_t clock, int enable) {
  return guarded([&] {
    need_table(t);
    t->clock_override = enable != 0;
    t->clock_value = clock;
  });
}

}  // extern "C"

namespace {

// Built-in predicates of the C ABI, in the reference's v1 functor form.
template <class K, class S>
struct PredScoreLt {
  __device__ bool operator()(const K&, const S& s, const K&, const S& th) const { return s < th; }
};
template <class K, class S>
struct PredScoreGe {
  __device__ bool operator()(const K&, const S& s, const K&, const S& th) const { return s >= th; }
};
template <class K, class S>
struct PredScoreGt {
  __device__ bool operator()(const K&, const S& s, const K&, const S& th) const { return s > th; }
};
template <class K, class S>
struct PredKeyMaskEq {
  __device__ bool operator()(const K& k, const S&, const K& p, const S&) const {
    return (k & p) == p;
  }
};
template <class K, class S>
struct PredKeyLow7GtScoreGt {
  __device__ bool operator()(const K& k, const S& s, const K& p, const S& th) const {
    return ((k & 0x7f) > p) && (s > th);
  }
};

hkv_device_view device_view(const hkv_table* t) {
  hkv_device_view v{};
  v.digests = t->digests;
  v.slots = t->slots;
  v.bucket_sizes = t->bsize;
  v.live = t->live;
  v.slices = t->d_slices;
  v.capacity = t->C;
  v.buckets = t->nb;
  v.max_bucket_size = (uint32_t)t->B;
  v.bucket_shift = log2_ceil(t->B);
  v.slice_shift = (uint32_t)t->slice_shift;
  v.row_bytes = (uint32_t)t->row;
  v.reclaim_digest = kReclaimDigest;
  return v;
}

// Runs `body.template run<K, V, Pred>()` for the table's key type, a row
// element type the row size allows, and the predicate kind.
template <class Body>
void with_pred(const hkv_table* t, int pred, bool wide_rows, Body&& body) {
  auto by_k = [&](auto kz) {
    using K = decltype(kz);
    auto by_v = [&](auto vz) {
      using V = decltype(vz);
      switch (pred) {
        case HKV_PRED_SCORE_LT: body.template run<K, V, PredScoreLt>(); break;
        case HKV_PRED_SCORE_GE: body.template run<K, V, PredScoreGe>(); break;
        case HKV_PRED_SCORE_GT: body.template run<K, V, PredScoreGt>(); break;
        case HKV_PRED_KEY_MASK_EQ: body.template run<K, V, PredKeyMaskEq>(); break;
        case HKV_PRED_KEY_LOW7_GT_SCORE_GT: body.template run<K, V, PredKeyLow7GtScoreGt>(); break;
        default: fail(HKV_ERR_INVALID, "unknown predicate");
      }
    };
    if (wide_rows) by_v(uint32_t{});
    else by_v(uint8_t{});
  };
  if (t->key_type == HKV_KEY_I64) by_k(int64_t{});
  else by_k(uint64_t{});
}

struct EraseIfBody {
  hkv_device_view v;
  uint64_t pattern, threshold;
  unsigned long long* d;
  hipStream_t s;
  template <class K, class V, template <typename, typename> class P>
  void run() {
    hkv_ops::PatternPred<K, V, uint64_t, P> a{(K)pattern, threshold};
    hip_check(hkv_ops::erase_if<K, V, uint64_t>(v, a, d, s), "erase_if launch");
  }
};

struct SizeIfBody {
  hkv_device_view v;
  uint64_t pattern, threshold;
  unsigned long long* d;
  hipStream_t s;
  template <class K, class V, template <typename, typename> class P>
  void run() {
    hkv_ops::PatternPred<K, V, uint64_t, P> a{(K)pattern, threshold};
    hip_check(hkv_ops::size_if<K, V, uint64_t>(v, a, d, s), "size_if launch");
  }
};

struct ExportIfBody {
  hkv_device_view v;
  uint64_t pattern, threshold, n, offset;
  unsigned long long* d;
  void* keys;
  void* values;
  uint64_t* scores;
  hipStream_t s;
  template <class K, class V, template <typename, typename> class P>
  void run() {
    hkv_ops::PatternPred<K, V, uint64_t, P> a{(K)pattern, threshold};
    hip_check(hkv_ops::export_if<K, V, uint64_t>(v, a, n, offset, d, static_cast<K*>(keys),
                                                 static_cast<V*>(values), scores, s),
              "export_batch_if launch");
  }
};

}  // namespace

extern "C" {

int hkv_set_max_capacity(hkv_table* t, uint64_t new_max_capacity) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2955-2977
    if (!ispow2(new_max_capacity))
      fail(HKV_ERR_UNSUPPORTED, "None power-of-2 new_max_capacity is not supported.");
    if (new_max_capacity < t->C) return;
    t->reach_max = false;
    t->opt.max_capacity = new_max_capacity;
  });
}

int hkv_device_view_get(const hkv_table* t, hkv_device_view* out) {
  return guarded([&] {
    need_table(t);
    if (!out) fail(HKV_ERR_INVALID, "null output");
    *out = device_view(t);
  });
}

int hkv_erase_if(hkv_table* t, int pred, uint64_t pattern, uint64_t threshold, hkv_stream stream,
                 uint64_t* count) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2409-2441
    if (!count) fail(HKV_ERR_INVALID, "null count");
    const hipStream_t s = S(stream);
    const hkv_device_view v = device_view(t);
    unsigned long long* d = reinterpret_cast<unsigned long long*>(t->d_sum);
    launch_fill_u64(t->d_sum, 0, 1, s);
    EraseIfBody body{v, pattern, threshold, d, s};
    with_pred(t, pred, false, body);
    hip_check(hipMemcpyAsync(t->h_sum, t->d_sum, 8, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    *count = *t->h_sum;
  });
}

int hkv_size_if(hkv_table* t, int pred, uint64_t pattern, uint64_t threshold,
                uint64_t* d_counter, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2829-2845
    if (!d_counter) fail(HKV_ERR_INVALID, "null counter");
    const hkv_device_view v = device_view(t);
    SizeIfBody body{v, pattern, threshold, reinterpret_cast<unsigned long long*>(d_counter), S(stream)};
    with_pred(t, pred, false, body);
  });
}

int hkv_export_batch_if(hkv_table* t, int pred, uint64_t pattern, uint64_t threshold, uint64_t n,
                        uint64_t offset, uint64_t* d_counter, void* keys, void* values,
                        uint64_t* scores, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2623-2672: the counter is cleared, and a window
    // of no slots (n == 0, or offset at or past the capacity) returns there.
    if (!d_counter) fail(HKV_ERR_INVALID, "d_counter must not be null");
    const bool window = offset < t->C && n > 0;
    if (window && (!keys || !values)) fail(HKV_ERR_INVALID, "keys and values must not be null");
    const hkv_device_view v = device_view(t);
    const bool wide = (t->row % 4) == 0 && ((uintptr_t)values % 4) == 0;
    ExportIfBody body{v, pattern, threshold, n, offset, reinterpret_cast<unsigned long long*>(d_counter),
           keys, values, scores, S(stream)};
    with_pred(t, pred, wide, body);
  });
}

int hkv_assign(hkv_table* t, uint64_t n, const void* keys, const void* values,
               const uint64_t* scores, hkv_stream stream, int unique_key) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1830-1921
    if (n == 0) return;
    t->check_scores(t->strategy, scores, false);
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    const ScoreCtx sc{t->strategy, t->epoch, t->clock_now()};
    if (!unique_key) {
      // Scores in batch order through the bucket-owner pipeline, then rows.
      insert_like(t, OP_ASSIGN_SCORES, n, keys, nullptr, nullptr, scores, nullptr, nullptr,
                  nullptr, nullptr, nullptr, t->strategy, RULE_DIGEST16, S(stream));
    }
    launch_assign(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                  reinterpret_cast<const uint8_t*>(values), scores, unique_key != 0, sc,
                  t->value_unit(values), S(stream));
    hip_check(hipGetLastError(), "assign launch");
  });
}

int hkv_assign_values(hkv_table* t, uint64_t n, const void* keys, const void* values,
                      hkv_stream stream, int unique_key) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2003-2093
    (void)unique_key;
    if (n == 0) return;
    if (!keys || !values) fail(HKV_ERR_INVALID, "keys and values must not be null");
    launch_assign(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                  reinterpret_cast<const uint8_t*>(values), nullptr, false, ScoreCtx{},
                  t->value_unit(values), S(stream));
    hip_check(hipGetLastError(), "assign_values launch");
  });
}

int hkv_contains(hkv_table* t, uint64_t n, const void* keys, uint8_t* founds,
                 hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2330-2347
    if (n == 0) return;
    if (!keys || !founds) fail(HKV_ERR_INVALID, "keys and founds must not be null");
    launch_contains(t->view(), reinterpret_cast<const uint64_t*>(keys), n, founds, S(stream));
    hip_check(hipGetLastError(), "contains launch");
  });
}

int hkv_find_ptr(hkv_table* t, uint64_t n, const void* keys, void** value_ptrs,
                 uint8_t* founds, uint64_t* scores, hkv_stream stream, int unique_key) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2244-2262
    (void)unique_key;
    if (n == 0) return;
    if (!keys || !value_ptrs) fail(HKV_ERR_INVALID, "keys and values must not be null");
    launch_find_ptr(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                    reinterpret_cast<uint64_t*>(value_ptrs), founds, scores, false, ScoreCtx{},
                    S(stream));
    hip_check(hipGetLastError(), "find launch");
  });
}

int hkv_find_and_update(hkv_table* t, uint64_t n, const void* keys, void** value_ptrs,
                        uint8_t* founds, uint64_t* scores, hkv_stream stream, int unique_key) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:2288-2317
    if (n == 0) return;
    if (!keys || !value_ptrs) fail(HKV_ERR_INVALID, "keys and values must not be null");
    t->check_scores(t->strategy, scores, false);
    if (!unique_key)
      fail(HKV_ERR_RUNTIME,
           "Not support update score when keys are not unique or bucket capacity is small.");
    const ScoreCtx sc{t->strategy, t->epoch, t->clock_now()};
    launch_find_ptr(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                    reinterpret_cast<uint64_t*>(value_ptrs), founds, scores, true, sc,
                    S(stream));
    hip_check(hipGetLastError(), "find_and_update launch");
  });
}

int hkv_find_or_insert_ptr(hkv_table* t, uint64_t n, const void* keys, void** value_ptrs,
                           uint8_t* founds, const uint64_t* scores, hkv_stream stream,
                           int unique_key, int ignore_evict_strategy, void** locked_key_ptrs) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1658-1728
    if (n == 0) return;
    if (!keys || !value_ptrs || !founds)
      fail(HKV_ERR_INVALID, "keys, values and founds must not be null");
    const hipStream_t s = S(stream);
    t->maybe_grow(n, s);
    t->check_scores(t->strategy, scores, ignore_evict_strategy != 0);
    if (locked_key_ptrs && !unique_key)
      fail(HKV_ERR_UNSUPPORTED,
           "unique_key should be true and max_bucket_size should be larger.");
    PartScratch ps{};
    t->part_scratch(n, &ps, s);
    ApplyArgs a{};
    a.keys = reinterpret_cast<const uint64_t*>(keys);
    a.in_scores = scores;
    a.n = n;
    a.sc.strategy = t->strategy;
    a.sc.epoch = t->epoch;
    a.sc.clock = t->clock_now();
    a.rule = unique_key ? RULE_DIGEST16 : RULE_TILE32;
    a.lock = unique_key ? 1 : 0;
    a.unit = 16;
    a.value_type = t->value_type;
    launch_find_or_insert_ptr(t->view(), a, ps, reinterpret_cast<uint64_t*>(value_ptrs), founds,
                              reinterpret_cast<uint64_t*>(locked_key_ptrs),
                              locked_key_ptrs != nullptr, s);
    hip_check(hipGetLastError(), "find_or_insert launch");
  });
}

int hkv_lock_keys(hkv_table* t, uint64_t n, const void* keys, void** locked_key_ptrs,
                  uint8_t* success, hkv_stream stream, const uint64_t* scores) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1744-1771
    if (n == 0) return;
    if (!keys || !locked_key_ptrs) fail(HKV_ERR_INVALID, "keys and locked_key_ptrs must not be null");
    if ((t->strategy == HKV_EPOCH_LFU || t->strategy == HKV_CUSTOMIZED) && !scores)
      fail(HKV_ERR_INVALID, "this evict strategy reads input scores; scores is null.");
    const ScoreCtx sc{t->strategy, t->epoch, t->clock_now()};
    launch_lock_keys(t->view(), reinterpret_cast<const uint64_t*>(keys), n,
                     reinterpret_cast<uint64_t*>(locked_key_ptrs), success, scores, sc,
                     S(stream));
    hip_check(hipGetLastError(), "lock_keys launch");
  });
}

int hkv_unlock_keys(hkv_table* t, uint64_t n, void* const* locked_key_ptrs, const void* keys,
                    uint8_t* success, hkv_stream stream) {
  return guarded([&] {
    need_table(t);
    // include/hkv_hashtable.h:1788-1804
    if (n == 0) return;
    if (!keys || !locked_key_ptrs) fail(HKV_ERR_INVALID, "keys and locked_key_ptrs must not be null");
    launch_unlock_keys(t->view(), n, reinterpret_cast<const uint64_t*>(locked_key_ptrs),
                       reinterpret_cast<const uint64_t*>(keys), success, S(stream));
    hip_check(hipGetLastError(), "unlock_keys launch");
  });
}

int hkv_slot_addresses(const hkv_table* t, uint64_t n, const uint64_t* slots, void** key_ptrs,
                       void** value_ptrs) {
  return guarded([&] {
    need_table(t);
    const uint64_t mask = (1ull << t->slice_shift) - 1;
    for (uint64_t i = 0; i < n; i++) {
      const uint64_t g = slots[i];
      if (g >= t->C) fail(HKV_ERR_INVALID, "slot index out of range");
      const uint64_t b = g / t->B, sl = g % t->B;
      if (key_ptrs) key_ptrs[i] = t->slots + 2 * g;
      if (value_ptrs)
        value_ptrs[i] = t->slices[b >> t->slice_shift].dev_ptr + ((b & mask) * t->B + sl) * t->row;
    }
  });
}

int hkv_live_count(hkv_table* t, hkv_stream stream, uint64_t* out) {
  return guarded([&] {
    need_table(t);
    if (!out) fail(HKV_ERR_INVALID, "null output");
    hip_check(hipMemcpyAsync(t->h_sum, t->live, sizeof(uint64_t), hipMemcpyDeviceToHost,
                             S(stream)),
              "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
    *out = *t->h_sum;
  });
}

}  // extern "C"
