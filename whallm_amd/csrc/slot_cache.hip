// HBM expert slot cache: the reference's expert arena (Native/QwenNative/engine.mm:649-778,
// and ExpertCache, runtime/deepseek_v4_ssd/expert_cache.py:1465-1945), on MI355X.
//
// Policy (host side, as ExpertArena::plan / victim / touch): a plan hands out one
// slot per requested expert; hits bump the slot's use count; misses take a free slot
// in order, else the least-used slot, oldest stamp among equals, never one handed out
// by the same plan; use counts halve (floor 1) every max(8 * slots, 64) touches.
//
// Route mode (ExpertCache with eviction_policy "route", expert_cache.py:1131-1181): the
// caller supplies a retention score per (file, expert) and a slot quota per file (the
// route-history policy's output). The victim is the resident expert with the lowest
// (tier, score, last access), never one handed out by the same plan, where tier 0 holds
// the files over their quota (or the incoming file at its quota) and tier 1 the rest.
//
// Whole-file reads and seeding (engine.mm:1647-1678): a file's blobs are copied in one
// hipMemcpyAsync into a caller buffer (a prefill layer reads its experts from there while
// the next file is read into the other buffer), and a file's most used experts can then
// be seeded into slots from that buffer with device-to-device copies.
//
// Fills: the blobs of a plan's misses are copied from the caller's pinned host pool
// (the stand-in for the reference's SSD expert files: [files][experts][blob]) into
// their HBM slots with hipMemcpyAsync on the cache's own copy stream. The copy
// stream first waits for everything already enqueued on the compute stream (those
// kernels may still read the slots being refilled), and the compute stream then waits
// for the fills, so work enqueued after an acquire sees its experts resident. The
// device expert -> slot map of the plan's file is refreshed on the same stream.
#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "wm_common.h"

namespace wm {

class SlotCache {
 public:
  SlotCache(int slots, int64_t blob, int files, int experts, void* device_slots, int32_t* device_map,
            const void* host_pool)
      : slots_(slots), blob_(blob), files_(files), experts_(experts), dev_(static_cast<uint8_t*>(device_slots)),
        map_(device_map), pool_(static_cast<const uint8_t*>(host_pool)) {
    owner_.assign(slots, -1);
    stamp_.assign(slots, 0);
    uses_.assign(slots, 0);
    access_.assign(slots, 0);
    count_.assign(files, 0);
    host_map_.assign((size_t)files * experts, -1);
    if (dev_) {
      check(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking), "hipStreamCreateWithFlags");
      check(hipEventCreateWithFlags(&compute_done_, hipEventDisableTiming), "hipEventCreate");
      check(hipEventCreateWithFlags(&fills_done_, hipEventDisableTiming), "hipEventCreate");
      staging_.resize(kStaging);
      for (auto& st : staging_) {
        check(hipHostMalloc(reinterpret_cast<void**>(&st.row), (size_t)experts * sizeof(int32_t), hipHostMallocDefault),
              "hipHostMalloc");
        check(hipEventCreateWithFlags(&st.done, hipEventDisableTiming), "hipEventCreate");
      }
    }
  }
  ~SlotCache() {
    if (!dev_) return;
    (void)hipStreamSynchronize(copy_);
    for (auto& kv : layer_done_) (void)hipEventDestroy(kv.second);
    for (auto& st : staging_) {
      (void)hipEventDestroy(st.done);
      (void)hipHostFree(st.row);
    }
    (void)hipEventDestroy(compute_done_);
    (void)hipEventDestroy(fills_done_);
    (void)hipStreamDestroy(copy_);
  }

  // ExpertArena::plan (engine.mm:679-707): slots for `experts` of `file`; missing ones
  // get a slot (flag 1 in `filled`) and must be filled before use.
  void plan(int file, const int32_t* experts, int n, int32_t* out_slots, int32_t* filled) {
    if (file < 0 || file >= files_) throw std::runtime_error("slot cache: file out of range");
    for (int i = 0; i < n; ++i)
      if (experts[i] < 0 || experts[i] >= experts_) throw std::runtime_error("slot cache: expert id out of range");
    ++clock_;
    for (int i = 0; i < n; ++i) {
      const long key = (long)file * experts_ + experts[i];
      touch();
      auto found = where_.find(key);
      if (found != where_.end()) {
        const int s = found->second;
        out_slots[i] = s;
        stamp_[s] = clock_;
        access_[s] = ++seq_;
        ++uses_[s];
        ++hits_;
        if (filled) filled[i] = 0;
        continue;
      }
      const int s = victim(file);
      if (owner_[s] >= 0) {
        where_.erase(owner_[s]);
        host_map_[owner_[s]] = -1;
        --count_[owner_[s] / experts_];
      }
      owner_[s] = key;
      where_[key] = s;
      host_map_[key] = s;
      ++count_[file];
      stamp_[s] = clock_;
      access_[s] = ++seq_;
      uses_[s] = 1;
      out_slots[i] = s;
      if (filled) filled[i] = 1;
      ++misses_;
    }
  }

  void acquire(int file, const int32_t* experts, int n, int32_t* out_slots, hipStream_t compute) {
    fill(file, experts, n, out_slots, compute, nullptr);
  }

  // plan + copies of the misses: from the host pool, or with `layer` (a device copy of the
  // whole file) device to device.
  void fill(int file, const int32_t* experts, int n, int32_t* out_slots, hipStream_t compute, const uint8_t* layer) {
    if (!dev_) throw std::runtime_error("slot cache: opened without device memory (policy only)");
    std::vector<int32_t> filled(n);
    plan(file, experts, n, out_slots, filled.data());
    bool any = false;
    for (int i = 0; i < n; ++i) any |= filled[i] != 0;
    if (!any) return;
    // the slots being refilled may still be read by work already on the compute stream
    check(hipEventRecord(compute_done_, compute), "hipEventRecord");
    check(hipStreamWaitEvent(copy_, compute_done_, 0), "hipStreamWaitEvent");
    for (int i = 0; i < n; ++i) {
      if (!filled[i]) continue;
      if (layer) {
        check(hipMemcpyAsync(dev_ + (size_t)out_slots[i] * blob_, layer + (size_t)experts[i] * blob_, blob_,
                             hipMemcpyDeviceToDevice, copy_),
              "hipMemcpyAsync");
      } else {
        const uint8_t* src = pool_ + ((size_t)file * experts_ + experts[i]) * blob_;
        check(hipMemcpyAsync(dev_ + (size_t)out_slots[i] * blob_, src, blob_, hipMemcpyHostToDevice, copy_),
              "hipMemcpyAsync");
      }
      copied_ += blob_;
      ++fills_;
    }
    if (map_) {  // refresh this file's expert -> slot row through a pinned staging row
      Staging& st = staging_[next_staging_++ % kStaging];
      check(hipEventSynchronize(st.done), "hipEventSynchronize");
      std::memcpy(st.row, &host_map_[(size_t)file * experts_], (size_t)experts_ * sizeof(int32_t));
      check(hipMemcpyAsync(map_ + (size_t)file * experts_, st.row, (size_t)experts_ * sizeof(int32_t),
                           hipMemcpyHostToDevice, copy_),
            "hipMemcpyAsync");
      check(hipEventRecord(st.done, copy_), "hipEventRecord");
    }
    check(hipEventRecord(fills_done_, copy_), "hipEventRecord");
    check(hipStreamWaitEvent(compute, fills_done_, 0), "hipStreamWaitEvent");
  }

  // ExpertArena::seed (engine.mm:1664-1678): plan `experts` of `file` (least valuable
  // first) with their use counts, filling the misses from `layer`, a device copy of the
  // whole file.
  void seed(int file, const int32_t* experts, const int32_t* uses, int n, const uint8_t* layer, int32_t* out_slots,
            hipStream_t compute) {
    fill(file, experts, n, out_slots, compute, layer);
    for (int i = 0; i < n; ++i)
      if (uses) uses_[out_slots[i]] = std::max<long>(1, uses[i]);
  }

  // The whole file's blobs into dst, on the copy stream after the compute stream's
  // earlier work (which may still read dst); wait_layer makes a stream wait for it.
  void read_layer(int file, uint8_t* dst, hipStream_t compute) {
    if (!dev_) throw std::runtime_error("slot cache: opened without device memory (policy only)");
    if (file < 0 || file >= files_) throw std::runtime_error("slot cache: file out of range");
    if (!dst) throw std::runtime_error("slot cache: null layer buffer");
    check(hipEventRecord(compute_done_, compute), "hipEventRecord");
    check(hipStreamWaitEvent(copy_, compute_done_, 0), "hipStreamWaitEvent");
    const size_t bytes = (size_t)experts_ * blob_;
    check(hipMemcpyAsync(dst, pool_ + (size_t)file * bytes, bytes, hipMemcpyHostToDevice, copy_), "hipMemcpyAsync");
    copied_ += (int64_t)bytes;
    hipEvent_t& ev = layer_done_[file];
    if (!ev) check(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate");
    check(hipEventRecord(ev, copy_), "hipEventRecord");
  }
  void wait_layer(int file, hipStream_t compute) {
    auto it = layer_done_.find(file);
    if (it == layer_done_.end()) throw std::runtime_error("slot cache: wait for a file that was never read");
    check(hipStreamWaitEvent(compute, it->second, 0), "hipStreamWaitEvent");
  }

  // Route mode on (scores [files][experts], quotas [files]) or off (scores NULL).
  void set_route(const double* scores, const int32_t* quotas) {
    if (!scores) {
      route_ = false;
      return;
    }
    if (!quotas) throw std::runtime_error("slot cache: route scores need quotas");
    score_.assign(scores, scores + (size_t)files_ * experts_);
    quota_.assign(quotas, quotas + files_);
    route_ = true;
  }

  void stats(int64_t* out) const {
    out[0] = hits_;
    out[1] = misses_;
    out[2] = copied_;
    out[3] = fills_;
  }

  std::string error;

 private:
  static constexpr int kStaging = 8;
  struct Staging {
    int32_t* row = nullptr;
    hipEvent_t done = nullptr;
  };

  static void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("slot cache: ") + what + ": " + hipGetErrorString(e));
  }
  int victim(int incoming) {
    if (used_ < slots_) return used_++;
    if (route_) return route_victim(incoming);
    return lfu_victim();
  }
  // ExpertCache._evict_route_locked (expert_cache.py:1143-1181): lowest (tier, score, last
  // access); the reference's per-layer heaps pick the same entry
  int route_victim(int incoming) {
    int best = -1, best_tier = 0;
    double best_score = 0.0;
    for (int s = 0; s < slots_; ++s) {
      if (stamp_[s] == clock_ || owner_[s] < 0) continue;
      const int f = (int)(owner_[s] / experts_);
      const int tier = count_[f] > quota_[f] || (f == incoming && count_[f] >= quota_[f]) ? 0 : 1;
      const double sc = score_[owner_[s]];
      if (best < 0 || tier < best_tier || (tier == best_tier && (sc < best_score ||
                                                                  (sc == best_score && access_[s] < access_[best])))) {
        best = s;
        best_tier = tier;
        best_score = sc;
      }
    }
    if (best < 0) throw std::runtime_error("the expert cache is too small for one step");
    return best;
  }
  // ExpertArena::victim (engine.mm:749-757)
  int lfu_victim() {
    int best = -1;
    for (int s = 0; s < slots_; ++s) {
      if (stamp_[s] == clock_) continue;
      if (best < 0 || uses_[s] < uses_[best] || (uses_[s] == uses_[best] && stamp_[s] < stamp_[best])) best = s;
    }
    if (best < 0) throw std::runtime_error("the expert cache is too small for one step");
    return best;
  }
  // ExpertArena::touch (engine.mm:759-763)
  void touch() {
    if (++touches_ < std::max<long>((long)slots_ * 8, 64)) return;
    touches_ = 0;
    for (long& u : uses_) u = std::max<long>(1, u / 2);
  }

  int slots_;
  int64_t blob_;
  int files_, experts_;
  uint8_t* dev_;
  int32_t* map_;
  const uint8_t* pool_;
  int used_ = 0;
  long clock_ = 0, touches_ = 0, seq_ = 0;
  std::vector<long> owner_, stamp_, uses_, access_;
  std::vector<int> count_;
  bool route_ = false;
  std::vector<double> score_;
  std::vector<int32_t> quota_;
  std::unordered_map<int, hipEvent_t> layer_done_;
  std::vector<int32_t> host_map_;
  std::unordered_map<long, int> where_;
  int64_t hits_ = 0, misses_ = 0, copied_ = 0, fills_ = 0;
  hipStream_t copy_ = nullptr;
  hipEvent_t compute_done_ = nullptr, fills_done_ = nullptr;
  std::vector<Staging> staging_;
  unsigned next_staging_ = 0;
};

// Runs body(); a thrown error becomes status 1 with the message kept on the handle.
template <typename Body>
int with_cache(SlotCache* c, Body&& body) {
  if (!c) return 1;
  try {
    body();
    c->error.clear();
    return 0;
  } catch (const std::exception& e) {
    c->error = e.what();
  } catch (...) {
    c->error = "slot cache: unknown error";
  }
  return 1;
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT wm_slot_cache* wm_slot_cache_open(int32_t slots, int64_t blob_bytes, int32_t files, int32_t experts,
                                            void* device_slots, int32_t* device_map, const void* host_pool,
                                            char* err, size_t err_size) {
  auto report = [&](const std::string& m) {
    if (err && err_size) {
      std::strncpy(err, m.c_str(), err_size - 1);
      err[err_size - 1] = 0;
    }
  };
  if (slots < 1 || blob_bytes < 1 || files < 1 || experts < 1) {
    report("wm_slot_cache_open: slots, blob bytes, files and experts must be positive");
    return nullptr;
  }
  if (device_slots && !host_pool) {
    report("wm_slot_cache_open: a device-backed cache needs the host pool");
    return nullptr;
  }
  try {
    return reinterpret_cast<wm_slot_cache*>(
        new SlotCache(slots, blob_bytes, files, experts, device_slots, device_map, host_pool));
  } catch (const std::exception& e) {
    report(e.what());
  }
  return nullptr;
}

WM_EXPORT void wm_slot_cache_close(wm_slot_cache* cache) { delete reinterpret_cast<SlotCache*>(cache); }

WM_EXPORT const char* wm_slot_cache_error(const wm_slot_cache* cache) {
  return cache ? reinterpret_cast<const SlotCache*>(cache)->error.c_str() : "null slot cache";
}

WM_EXPORT int wm_slot_cache_plan(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                 int32_t* out_slots, int32_t* out_filled) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || (n > 0 && (!experts || !out_slots))) throw std::runtime_error("wm_slot_cache_plan: bad arguments");
    c->plan(file, experts, n, out_slots, out_filled);
  });
}

WM_EXPORT int wm_slot_cache_acquire(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                    int32_t* out_slots, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || (n > 0 && (!experts || !out_slots))) throw std::runtime_error("wm_slot_cache_acquire: bad arguments");
    c->acquire(file, experts, n, out_slots, as_stream(compute_stream));
  });
}

WM_EXPORT int wm_slot_cache_set_route(wm_slot_cache* cache, const double* scores, const int32_t* quotas) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->set_route(scores, quotas); });
}

WM_EXPORT int wm_slot_cache_read_layer(wm_slot_cache* cache, int32_t file, void* dst, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->read_layer(file, static_cast<uint8_t*>(dst), as_stream(compute_stream)); });
}

WM_EXPORT int wm_slot_cache_wait_layer(wm_slot_cache* cache, int32_t file, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->wait_layer(file, as_stream(compute_stream)); });
}

WM_EXPORT int wm_slot_cache_seed(wm_slot_cache* cache, int32_t file, const int32_t* experts, const int32_t* uses,
                                 int32_t n, const void* layer, int32_t* out_slots, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || (n > 0 && (!experts || !out_slots || !layer))) throw std::runtime_error("wm_slot_cache_seed: bad arguments");
    c->seed(file, experts, uses, n, static_cast<const uint8_t*>(layer), out_slots, as_stream(compute_stream));
  });
}

WM_EXPORT int wm_slot_cache_stats(const wm_slot_cache* cache, int64_t* out4) {
  if (!cache || !out4) return 1;
  reinterpret_cast<const SlotCache*>(cache)->stats(out4);
  return 0;
}

}  // extern "C"
