// HBM expert slot cache: the reference's expert arena (Native/QwenNative/engine.mm:649-778,
// and ExpertCache, runtime/deepseek_v4_ssd/expert_cache.py:1465-1945), on MI355X.
//
// Policy (host side, as ExpertArena::plan / victim / touch): a plan hands out one
// slot per requested expert; hits bump the slot's use count; misses take a free slot
// in order, else the least-used slot, oldest stamp among equals, never one handed out
// by the same plan; use counts halve (floor 1) every max(8 * slots, 64) touches.
//
// Route mode (ExpertCache with eviction_policy "route", expert_cache.py:1131-1181): every
// (file, expert) has a retention score and every file a slot quota, from the cache's own
// route-history policy (route_policy.h, fed by the routes it observes) or supplied by the
// caller. The victim is the resident expert with the lowest (tier, score, last access),
// never one handed out by the same plan, where tier 0 holds the files over their quota
// (or the incoming file at its quota) and tier 1 the rest.
//
// Layer reads and seeding (engine.mm:1647-1678; expert_cache.py:1399-1430, :2062-2085): a
// file's blobs, or a subset of them, are copied into a caller buffer (a prefill layer reads
// its experts from there while the next file is read into the other buffer); a subset is
// read in runs of consecutive experts of at most 32 blobs per copy. A file's experts can
// then be seeded into slots from that buffer with device-to-device copies: a given list
// with use counts (the native engine's seed_layer), or the prompt tail's hottest experts,
// ranked on the device from the routes and seeded into free slots only.
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

#include <memory>

#include "route_policy.h"
#include "wm_common.h"

namespace wm {

constexpr int kTailRows = 128;     // token rows of the prompt tail that rank experts for seeding
constexpr int kMaxReadBatch = 32;  // blobs per copy of a partial layer read

// The prompt tail's experts ranked for seeding (hot_tail_experts, qwen_streaming_policy.py:23-45):
// over the last 128 token rows of routes [rows, k], each expert's count and its latest
// position; experts ordered by count, then latest position (both descending), then id.
// out[0] = n = min(limit, experts seen); out[1 .. n] = the first n experts, least valuable
// first; out[1 + limit ..] their counts in the same order. One workgroup; ids outside
// [0, experts) are ignored.
__global__ void __launch_bounds__(1024) tail_rank_kernel(const int32_t* __restrict__ routes, int64_t rows, int k,
                                                         int experts, int limit, int32_t* __restrict__ out) {
  __shared__ int32_t count[1024], last[1024];
  const int t = threadIdx.x;
  for (int e = t; e < experts; e += 1024) {
    count[e] = 0;
    last[e] = -1;
  }
  __syncthreads();
  const int64_t first = rows > kTailRows ? rows - kTailRows : 0;
  const int n = (int)((rows - first) * k);
  for (int p = t; p < n; p += 1024) {
    const int e = routes[first * k + p];
    if (e >= 0 && e < experts) {
      atomicAdd(&count[e], 1);
      atomicMax(&last[e], p);
    }
  }
  __syncthreads();
  const bool seen = t < experts && count[t] > 0;
  const int n_seen = __syncthreads_count(seen);
  const int n_sel = n_seen < limit ? n_seen : limit;
  if (seen) {
    const int c = count[t], p = last[t];
    int rank = 0;
    for (int f = 0; f < experts; ++f) {
      const int cf = count[f];
      rank += cf > c || (cf == c && cf > 0 && (last[f] > p || (last[f] == p && f < t)));
    }
    if (rank < n_sel) {
      out[1 + (n_sel - 1 - rank)] = t;
      out[1 + limit + (n_sel - 1 - rank)] = c;
    }
  }
  if (t == 0) out[0] = n_sel;
}

// Ready experts of one plan as a bitmask passed by value (experts <= 1024), so splitting a
// call's pairs needs no host -> device copy (which would queue behind the fills).
struct ExpertBits {
  uint32_t w[32];
};

// The cached-first split of a call's pairs (indices [n]): ready[i] = the id when its expert is
// ready, else -1; late[i] = the id otherwise (ids outside [0, experts) and masked ids go to
// late, where the expert kernels treat them as they always do).
__global__ void __launch_bounds__(256) split_ready_kernel(const int32_t* __restrict__ indices, int64_t n,
                                                          ExpertBits bits, int experts, int32_t* __restrict__ ready,
                                                          int32_t* __restrict__ late) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int e = indices[i];
  const bool r = e >= 0 && e < experts && ((bits.w[e >> 5] >> (e & 31)) & 1u);
  ready[i] = r ? e : -1;
  late[i] = r ? -1 : e;
}

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
    fill_pending_.assign(slots, 0);
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
    try {
      start_fills();  // held copies were planned: the map and the arena already count them
    } catch (...) {
    }
    (void)hipStreamSynchronize(copy_);
    for (auto& kv : layer_done_) (void)hipEventDestroy(kv.second);
    for (auto& st : staging_) {
      (void)hipEventDestroy(st.done);
      (void)hipHostFree(st.row);
    }
    (void)hipEventDestroy(compute_done_);
    (void)hipEventDestroy(fills_done_);
    (void)hipStreamDestroy(copy_);
    if (tail_dev_) (void)hipFree(tail_dev_);
    if (tail_host_) (void)hipHostFree(tail_host_);
  }

  // One file's part of a plan: slots for `experts` of `file`; filled[i] = 1 where the
  // expert was missing and took a slot (it must be filled before use).
  struct Request {
    int file;
    const int32_t* experts;
    int n;
    int32_t* slots;
    int32_t* filled;
  };

  // ExpertArena::plan (engine.mm:679-707) over one or more files at once: every slot the
  // plan hands out is protected from the plan's own evictions, so a multi-file plan keeps
  // all of its files' experts resident together (what one launch over several layers needs).
  void plan_requests(const Request* req, int m) {
    for (int r = 0; r < m; ++r) {
      if (req[r].file < 0 || req[r].file >= files_) throw std::runtime_error("slot cache: file out of range");
      for (int i = 0; i < req[r].n; ++i)
        if (req[r].experts[i] < 0 || req[r].experts[i] >= experts_)
          throw std::runtime_error("slot cache: expert id out of range");
    }
    ++clock_;
    evicted_files_.clear();
    for (int r = 0; r < m; ++r) plan_one(req[r]);
  }

  void plan(int file, const int32_t* experts, int n, int32_t* out_slots, int32_t* filled) {
    start_fills();
    std::vector<int32_t> own(filled ? 0 : n);
    const Request r{file, experts, n, out_slots, filled ? filled : own.data()};
    plan_requests(&r, 1);
  }

  // In route mode with the cache's own policy, the requested ids count as routes of `file`
  // in the current phase (ExpertCache.get_many observes them, expert_cache.py:1483).
  void acquire(int file, const int32_t* experts, int n, int32_t* out_slots, hipStream_t compute) {
    start_fills();
    observe_request(file, experts, n);
    std::vector<int32_t> filled(n);
    const Request r{file, experts, n, out_slots, filled.data()};
    fill(&r, 1, compute, nullptr, true);
  }

  // One plan over several files (see plan_requests), filled like acquire.
  void acquire_files(const Request* req, int m, hipStream_t compute) {
    start_fills();
    for (int r = 0; r < m; ++r) observe_request(req[r].file, req[r].experts, req[r].n);
    fill(req, m, compute, nullptr, true);
  }

  // The cached-first acquire (engine.mm:2204-2234; ExpertCache.iter_ready,
  // expert_cache.py:1541-1645): out_ready[i] = 1 for experts already resident, whose slots
  // no fill of this plan touches (a plan never evicts a slot it hands out), so work on
  // compute_stream may use them at once; the misses are filled on the copy stream and
  // compute_stream waits for them only at wait_fills.
  // A hit on a slot whose fill (from an earlier acquire_ready) no compute stream has waited
  // for yet is not ready either: its copy may still be in flight.
  void acquire_ready(int file, const int32_t* experts, int n, int32_t* out_slots, int32_t* out_ready,
                     hipStream_t compute) {
    start_fills();
    observe_request(file, experts, n);
    std::vector<int32_t> filled(n);
    const Request r{file, experts, n, out_slots, filled.data()};
    fill(&r, 1, compute, nullptr, false);
    for (int i = 0; i < n; ++i) out_ready[i] = filled[i] || fill_pending_[out_slots[i]] ? 0 : 1;
  }
  void wait_fills(hipStream_t compute) {
    start_fills();
    if (pending_) check(hipStreamWaitEvent(compute, fills_done_, 0), "hipStreamWaitEvent");
    pending_ = false;
    std::fill(fill_pending_.begin(), fill_pending_.end(), 0);
  }

  // acquire_ready for one call's pairs, in the reference's order (engine.mm:2204-2230: the
  // ready pairs are submitted, then the reads): plan, then split the pairs on compute_stream
  // into ready and late index arrays (split_ready_kernel, the ready set passed by value).
  // The copy stream is made to wait for compute_stream's work up to here (which may still
  // read the slots being refilled), but the copies themselves are held back until
  // start_fills, so the caller can enqueue its ready-pair kernels first; any later call on
  // the cache (wait_fills included) starts them if the caller has not.
  void acquire_split(int file, const int32_t* experts, int n, int32_t* out_slots, int32_t* out_ready,
                     const int32_t* indices, int64_t pairs, int32_t* ready_idx, int32_t* late_idx,
                     hipStream_t compute) {
    start_fills();
    if (!dev_) throw std::runtime_error("slot cache: opened without device memory (policy only)");
    if (experts_ > 1024) throw std::runtime_error("slot cache: the pair split takes at most 1024 experts");
    observe_request(file, experts, n);
    std::vector<int32_t> filled(n);
    const Request r{file, experts, n, out_slots, filled.data()};
    plan_requests(&r, 1);
    ExpertBits bits{};
    for (int i = 0; i < n; ++i) {
      out_ready[i] = filled[i] || fill_pending_[out_slots[i]] ? 0 : 1;
      if (out_ready[i]) bits.w[experts[i] >> 5] |= 1u << (experts[i] & 31);
    }
    if (pairs > 0) {
      hipLaunchKernelGGL(split_ready_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, compute, indices,
                         pairs, bits, experts_, ready_idx, late_idx);
      check(hipGetLastError(), "split_ready_kernel");
    }
    if (!any_filled(&r, 1)) return;
    order_copies_after(compute);
    held_file_ = file;
    held_experts_.assign(experts, experts + n);
    held_slots_.assign(out_slots, out_slots + n);
    held_filled_ = filled;
    held_ = true;
  }

  // The copies acquire_split held back, now (a no-op when there are none).
  void start_fills() {
    if (!held_) return;
    held_ = false;
    const Request r{held_file_, held_experts_.data(), (int)held_experts_.size(), held_slots_.data(),
                    held_filled_.data()};
    issue_fills(&r, 1, nullptr);
  }

  // plan + copies of the misses: from the host pool, or with `layer` (a device copy of the
  // whole file) device to device. With compute_waits the compute stream waits for the
  // copies now, else at the next wait_fills.
  void fill(const Request* req, int m, hipStream_t compute, const uint8_t* layer, bool compute_waits) {
    if (!dev_) throw std::runtime_error("slot cache: opened without device memory (policy only)");
    plan_requests(req, m);
    enqueue_fills(req, m, compute, layer, compute_waits);
  }
  static bool any_filled(const Request* req, int m) {
    for (int r = 0; r < m; ++r)
      for (int i = 0; i < req[r].n; ++i)
        if (req[r].filled[i]) return true;
    return false;
  }
  // The slots being refilled may still be read by work already on the compute stream: the
  // copy stream's next work waits for it.
  void order_copies_after(hipStream_t compute) {
    check(hipEventRecord(compute_done_, compute), "hipEventRecord");
    check(hipStreamWaitEvent(copy_, compute_done_, 0), "hipStreamWaitEvent");
  }
  // The copies of a planned request's misses (fill after plan_requests).
  void enqueue_fills(const Request* req, int m, hipStream_t compute, const uint8_t* layer, bool compute_waits) {
    if (!any_filled(req, m)) {
      // every expert is a hit, but some may be slots an earlier acquire_ready is still
      // filling: work enqueued after an acquire must see them resident
      if (compute_waits) wait_fills(compute);
      return;
    }
    order_copies_after(compute);
    issue_fills(req, m, layer);
    if (compute_waits) wait_fills(compute);
  }
  // The copies themselves (the copy stream already ordered after the compute stream), the
  // expert -> slot map refresh, and the event wait_fills waits for.
  void issue_fills(const Request* req, int m, const uint8_t* layer) {
    // one copy per run of misses whose experts and slots both follow each other (free slots
    // are handed out in order, so a cold cache fills consecutive experts in one copy)
    for (int r = 0; r < m; ++r) {
      const Request& q = req[r];
      for (int i = 0; i < q.n;) {
        if (!q.filled[i]) {
          ++i;
          continue;
        }
        int run = 1;
        while (i + run < q.n && run < kMaxReadBatch && q.filled[i + run] && q.experts[i + run] == q.experts[i] + run &&
               q.slots[i + run] == q.slots[i] + run)
          ++run;
        const size_t bytes = (size_t)run * blob_;
        uint8_t* dst = dev_ + (size_t)q.slots[i] * blob_;
        if (layer)
          check(hipMemcpyAsync(dst, layer + (size_t)q.experts[i] * blob_, bytes, hipMemcpyDeviceToDevice, copy_),
                "hipMemcpyAsync");
        else
          check(hipMemcpyAsync(dst, pool_ + ((size_t)q.file * experts_ + q.experts[i]) * blob_, bytes,
                               hipMemcpyHostToDevice, copy_),
                "hipMemcpyAsync");
        copied_ += (int64_t)bytes;
        fills_ += run;
        ++copies_;
        for (int j = 0; j < run; ++j) fill_pending_[q.slots[i + j]] = 1;
        i += run;
      }
    }
    if (map_) {
      // Refresh the expert -> slot rows that changed through pinned staging rows: the
      // requested files', and the row of every other file that lost a slot to them (its
      // entry becomes -1, so kernels reading that file's table skip the expert instead of
      // reading another file's weights from the slot).
      std::vector<int> rows;
      for (int r = 0; r < m; ++r) rows.push_back(req[r].file);
      rows.insert(rows.end(), evicted_files_.begin(), evicted_files_.end());
      std::sort(rows.begin(), rows.end());
      rows.erase(std::unique(rows.begin(), rows.end()), rows.end());
      for (int f : rows) refresh_map_row(f);
    }
    check(hipEventRecord(fills_done_, copy_), "hipEventRecord");
    pending_ = true;
  }

  // ExpertArena::seed (engine.mm:1664-1678): plan `experts` of `file` (least valuable
  // first) with their use counts, filling the misses from `layer`, a device copy of the
  // whole file.
  void seed(int file, const int32_t* experts, const int32_t* uses, int n, const uint8_t* layer, int32_t* out_slots,
            hipStream_t compute) {
    start_fills();
    std::vector<int32_t> filled(n);
    const Request r{file, experts, n, out_slots, filled.data()};
    fill(&r, 1, compute, layer, true);
    for (int i = 0; i < n; ++i)
      if (uses) uses_[out_slots[i]] = std::max<long>(1, uses[i]);
  }

  // The file's blobs into dst (blob e at e * blob), on the copy stream after the compute
  // stream's earlier work (which may still read dst); wait_layer makes a stream wait for it.
  // With `experts` (sorted, unique) only those blobs are read, in runs of consecutive ids of
  // at most kMaxReadBatch blobs per copy (the reference's prefill expert reads,
  // expert_cache.py:2062-2085 with contiguous_batches, qwen_streaming_policy.py:7-20).
  void read_layer(int file, uint8_t* dst, hipStream_t compute, const int32_t* experts = nullptr, int n = -1) {
    start_fills();
    if (!dev_) throw std::runtime_error("slot cache: opened without device memory (policy only)");
    if (file < 0 || file >= files_) throw std::runtime_error("slot cache: file out of range");
    if (!dst) throw std::runtime_error("slot cache: null layer buffer");
    if (experts)
      for (int i = 0; i < n; ++i)
        if (experts[i] < 0 || experts[i] >= experts_ || (i > 0 && experts[i] <= experts[i - 1]))
          throw std::runtime_error("slot cache: expert ids must be sorted, unique and inside the model");
    check(hipEventRecord(compute_done_, compute), "hipEventRecord");
    check(hipStreamWaitEvent(copy_, compute_done_, 0), "hipStreamWaitEvent");
    const size_t file_bytes = (size_t)experts_ * blob_;
    const uint8_t* src = pool_ + (size_t)file * file_bytes;
    if (!experts) {
      check(hipMemcpyAsync(dst, src, file_bytes, hipMemcpyHostToDevice, copy_), "hipMemcpyAsync");
      copied_ += (int64_t)file_bytes;
      ++copies_;
    } else {
      for (int i = 0; i < n;) {
        int run = 1;
        while (i + run < n && run < kMaxReadBatch && experts[i + run] == experts[i] + run) ++run;
        const size_t at = (size_t)experts[i] * blob_, bytes = (size_t)run * blob_;
        check(hipMemcpyAsync(dst + at, src + at, bytes, hipMemcpyHostToDevice, copy_), "hipMemcpyAsync");
        copied_ += (int64_t)bytes;
        ++copies_;
        i += run;
      }
    }
    hipEvent_t& ev = layer_done_[file];
    if (!ev) check(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate");
    check(hipEventRecord(ev, copy_), "hipEventRecord");
  }
  void wait_layer(int file, hipStream_t compute) {
    auto it = layer_done_.find(file);
    if (it == layer_done_.end()) throw std::runtime_error("slot cache: wait for a file that was never read");
    check(hipStreamWaitEvent(compute, it->second, 0), "hipStreamWaitEvent");
  }

  // Prompt-tail seeding (ExpertCache._seed_from_batched_layer, expert_cache.py:1399-1430):
  // rank the experts of the last 128 token rows of routes [rows, k] (a device array
  // written on compute_stream) on the device, keep the first `limit`, drop those already
  // resident, and copy the most valuable of the rest into free slots only (a prediction
  // never evicts a demand-loaded expert) from `layer`, a device copy of the whole file.
  // Returns how many were seeded; out_experts / out_slots (host, >= limit entries) list them.
  int seed_tail(int file, const int32_t* routes, int64_t rows, int k, int limit, const uint8_t* layer,
                int32_t* out_experts, int32_t* out_slots, hipStream_t compute) {
    start_fills();
    if (!dev_) throw std::runtime_error("slot cache: opened without device memory (policy only)");
    if (file < 0 || file >= files_) throw std::runtime_error("slot cache: file out of range");
    if (rows < 0 || k < 1 || limit < 0 || experts_ > 1024)
      throw std::runtime_error("slot cache: bad tail seeding arguments (k >= 1, limit >= 0, experts <= 1024)");
    if (rows == 0 || limit == 0) return 0;
    if (!routes || !layer) throw std::runtime_error("slot cache: null routes or layer buffer");
    const size_t words = 1 + 2 * (size_t)limit;
    if (words > tail_words_) {
      if (tail_dev_) check(hipFree(tail_dev_), "hipFree");
      if (tail_host_) check(hipHostFree(tail_host_), "hipHostFree");
      tail_dev_ = nullptr;
      tail_host_ = nullptr;
      check(hipMalloc(reinterpret_cast<void**>(&tail_dev_), words * sizeof(int32_t)), "hipMalloc");
      check(hipHostMalloc(reinterpret_cast<void**>(&tail_host_), words * sizeof(int32_t), hipHostMallocDefault),
            "hipHostMalloc");
      tail_words_ = words;
    }
    hipLaunchKernelGGL(tail_rank_kernel, dim3(1), dim3(1024), 0, compute, routes, rows, k, experts_, limit, tail_dev_);
    check(hipGetLastError(), "tail_rank_kernel");
    check(hipMemcpyAsync(tail_host_, tail_dev_, words * sizeof(int32_t), hipMemcpyDeviceToHost, compute), "hipMemcpyAsync");
    check(hipStreamSynchronize(compute), "hipStreamSynchronize");
    const int ranked = tail_host_[0];
    std::vector<int32_t> pick;
    for (int i = 0; i < ranked; ++i) {
      const int e = tail_host_[1 + i];
      if (host_map_[(size_t)file * experts_ + e] < 0) pick.push_back(e);
    }
    const int free_slots = slots_ - used_;
    if ((int)pick.size() > free_slots) pick.erase(pick.begin(), pick.end() - free_slots);  // keep the most valuable
    if (pick.empty()) return 0;
    std::vector<int32_t> filled(pick.size());
    const Request r{file, pick.data(), (int)pick.size(), out_slots, filled.data()};
    fill(&r, 1, compute, layer, true);
    std::copy(pick.begin(), pick.end(), out_experts);
    return (int)pick.size();
  }

  // Route mode with caller-supplied scores [files][experts] and quotas [files], or off (NULL).
  void set_route(const double* scores, const int32_t* quotas) {
    policy_.reset();
    if (!scores) {
      route_ = false;
      return;
    }
    if (!quotas) throw std::runtime_error("slot cache: route scores need quotas");
    score_.assign(scores, scores + (size_t)files_ * experts_);
    quota_.assign(quotas, quotas + files_);
    route_ = true;
  }

  // Route mode with the cache's own route-history policy (files = layers), or off (top_k 0).
  void enable_policy(int top_k) {
    if (top_k <= 0) {
      policy_.reset();
      route_ = false;
      return;
    }
    policy_ = std::make_unique<RoutePolicy>(files_, experts_, slots_, top_k);
    route_ = true;
  }
  RoutePolicy& policy() {
    if (!policy_) throw std::runtime_error("slot cache: the route policy is not enabled");
    return *policy_;
  }
  bool has_policy() const { return policy_ != nullptr; }
  // "prefill" or "decode" phase of the observed routes; leaving a prefill rebalances
  // (ExpertCache.trace_routes, expert_cache.py:1088-1103).
  void set_phase(bool prefill) {
    if (policy_ && prefill_phase_ && !prefill) policy_->rebalance();
    prefill_phase_ = prefill;
  }
  bool prefill_phase() const { return prefill_phase_; }

  void stats(int64_t* out) const {
    out[0] = hits_;
    out[1] = misses_;
    out[2] = copied_;
    out[3] = fills_;
  }
  int64_t copies() const { return copies_; }
  int files() const { return files_; }
  int experts() const { return experts_; }

  std::string error;

 private:
  static constexpr int kStaging = 8;
  struct Staging {
    int32_t* row = nullptr;
    hipEvent_t done = nullptr;
  };

  void plan_one(const Request& q) {
    for (int i = 0; i < q.n; ++i) {
      const long key = (long)q.file * experts_ + q.experts[i];
      touch();
      auto found = where_.find(key);
      if (found != where_.end()) {
        const int s = found->second;
        q.slots[i] = s;
        stamp_[s] = clock_;
        access_[s] = ++seq_;
        ++uses_[s];
        ++hits_;
        q.filled[i] = 0;
        continue;
      }
      const int s = victim(q.file);
      if (owner_[s] >= 0) {
        where_.erase(owner_[s]);
        host_map_[owner_[s]] = -1;
        const int old_file = (int)(owner_[s] / experts_);
        --count_[old_file];
        if (std::find(evicted_files_.begin(), evicted_files_.end(), old_file) == evicted_files_.end())
          evicted_files_.push_back(old_file);
      }
      owner_[s] = key;
      where_[key] = s;
      host_map_[key] = s;
      ++count_[q.file];
      stamp_[s] = clock_;
      access_[s] = ++seq_;
      uses_[s] = 1;
      q.slots[i] = s;
      q.filled[i] = 1;
      ++misses_;
    }
  }

  void observe_request(int file, const int32_t* experts, int n) {
    if (policy_ && n > 0) policy_->observe(file, experts, n, prefill_phase_);
  }
  double route_score(long key) const { return policy_ ? policy_->scores()[key] : score_[key]; }
  int32_t route_quota(int f) const { return policy_ ? policy_->quotas()[f] : quota_[f]; }

  void refresh_map_row(int file) {
    Staging& st = staging_[next_staging_++ % kStaging];
    check(hipEventSynchronize(st.done), "hipEventSynchronize");
    std::memcpy(st.row, &host_map_[(size_t)file * experts_], (size_t)experts_ * sizeof(int32_t));
    check(hipMemcpyAsync(map_ + (size_t)file * experts_, st.row, (size_t)experts_ * sizeof(int32_t),
                         hipMemcpyHostToDevice, copy_),
          "hipMemcpyAsync");
    check(hipEventRecord(st.done, copy_), "hipEventRecord");
  }
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
      const int32_t q = route_quota(f);
      const int tier = count_[f] > q || (f == incoming && count_[f] >= q) ? 0 : 1;
      const double sc = route_score(owner_[s]);
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
  bool route_ = false, prefill_phase_ = false;
  std::vector<double> score_;
  std::vector<int32_t> quota_;
  std::unique_ptr<RoutePolicy> policy_;
  int32_t* tail_dev_ = nullptr;   // tail ranking output (device) and its pinned readback
  int32_t* tail_host_ = nullptr;
  size_t tail_words_ = 0;
  int64_t copies_ = 0;
  std::unordered_map<int, hipEvent_t> layer_done_;
  std::vector<int32_t> host_map_;
  std::vector<int> evicted_files_;  // files that lost a slot in the last plan
  std::unordered_map<long, int> where_;
  int64_t hits_ = 0, misses_ = 0, copied_ = 0, fills_ = 0;
  hipStream_t copy_ = nullptr;
  hipEvent_t compute_done_ = nullptr, fills_done_ = nullptr;
  bool pending_ = false;  // fills recorded in fills_done_ that no compute stream waited for yet
  std::vector<uint8_t> fill_pending_;
  // the copies of the last acquire_split, held back until start_fills
  bool held_ = false;
  int held_file_ = 0;
  std::vector<int32_t> held_experts_, held_slots_, held_filled_;  // per slot: filled by a copy behind pending_
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

WM_EXPORT int wm_slot_cache_acquire_ready(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                          int32_t* out_slots, int32_t* out_ready, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || (n > 0 && (!experts || !out_slots || !out_ready)))
      throw std::runtime_error("wm_slot_cache_acquire_ready: bad arguments");
    c->acquire_ready(file, experts, n, out_slots, out_ready, as_stream(compute_stream));
  });
}

WM_EXPORT int wm_slot_cache_acquire_split(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                          int32_t* out_slots, int32_t* out_ready, const int32_t* indices,
                                          int64_t pairs, int32_t* ready_indices, int32_t* late_indices,
                                          void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || pairs < 0 || (n > 0 && (!experts || !out_slots || !out_ready)) ||
        (pairs > 0 && (!indices || !ready_indices || !late_indices)))
      throw std::runtime_error("wm_slot_cache_acquire_split: bad arguments");
    c->acquire_split(file, experts, n, out_slots, out_ready, indices, pairs, ready_indices, late_indices,
                     as_stream(compute_stream));
  });
}

WM_EXPORT int wm_slot_cache_start_fills(wm_slot_cache* cache) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->start_fills(); });
}

WM_EXPORT int wm_slot_cache_wait_fills(wm_slot_cache* cache, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->wait_fills(as_stream(compute_stream)); });
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

WM_EXPORT int wm_slot_cache_stats(const wm_slot_cache* cache, int64_t* out5) {
  if (!cache || !out5) return 1;
  const SlotCache* c = reinterpret_cast<const SlotCache*>(cache);
  c->stats(out5);
  out5[4] = c->copies();
  return 0;
}

WM_EXPORT int wm_slot_cache_acquire_files(wm_slot_cache* cache, int32_t n_files, const int32_t* files,
                                          const int32_t* counts, const int32_t* experts, int32_t* out_slots,
                                          void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n_files < 0 || (n_files > 0 && (!files || !counts))) throw std::runtime_error("wm_slot_cache_acquire_files: bad arguments");
    std::vector<SlotCache::Request> req;
    std::vector<std::vector<int32_t>> filled(n_files);
    int64_t at = 0;
    for (int r = 0; r < n_files; ++r) {
      if (counts[r] < 0) throw std::runtime_error("wm_slot_cache_acquire_files: negative count");
      if (counts[r] > 0 && (!experts || !out_slots)) throw std::runtime_error("wm_slot_cache_acquire_files: bad arguments");
      filled[r].resize(counts[r]);
      req.push_back({files[r], experts + at, counts[r], out_slots + at, filled[r].data()});
      at += counts[r];
    }
    c->acquire_files(req.data(), n_files, as_stream(compute_stream));
  });
}

WM_EXPORT int wm_slot_cache_read_experts(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                         void* dst, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || (n > 0 && !experts)) throw std::runtime_error("wm_slot_cache_read_experts: bad arguments");
    c->read_layer(file, static_cast<uint8_t*>(dst), as_stream(compute_stream), experts, n);
  });
}

WM_EXPORT int wm_slot_cache_seed_tail(wm_slot_cache* cache, int32_t file, const int32_t* routes, int64_t rows,
                                      int32_t k, int32_t limit, const void* layer, int32_t* out_experts,
                                      int32_t* out_slots, int32_t* out_count, void* compute_stream) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (!out_count || (limit > 0 && (!out_experts || !out_slots)))
      throw std::runtime_error("wm_slot_cache_seed_tail: bad arguments");
    *out_count = c->seed_tail(file, routes, rows, k, limit, static_cast<const uint8_t*>(layer), out_experts, out_slots,
                              as_stream(compute_stream));
  });
}

WM_EXPORT int wm_slot_cache_route_policy(wm_slot_cache* cache, int32_t top_k) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->enable_policy(top_k); });
}

WM_EXPORT int wm_slot_cache_route_observe(wm_slot_cache* cache, int32_t file, const int32_t* experts, int64_t n,
                                          int32_t prefill) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    if (n < 0 || (n > 0 && !experts)) throw std::runtime_error("wm_slot_cache_route_observe: bad arguments");
    c->policy().observe(file, experts, n, prefill != 0);
  });
}

WM_EXPORT int wm_slot_cache_route_phase(wm_slot_cache* cache, int32_t prefill) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->set_phase(prefill != 0); });
}

WM_EXPORT int wm_slot_cache_route_begin_request(wm_slot_cache* cache) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->policy().begin_request(); });
}

WM_EXPORT int wm_slot_cache_route_record_read(wm_slot_cache* cache, int32_t file, double seconds) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->policy().record_read(file, seconds); });
}

WM_EXPORT int wm_slot_cache_route_rebalance(wm_slot_cache* cache) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] { c->policy().rebalance(); });
}

WM_EXPORT int wm_slot_cache_route_state(wm_slot_cache* cache, double* scores, int32_t* quotas, double* short_rates,
                                        double* long_rates, int64_t* tokens, double* read_cost, int64_t* counters) {
  SlotCache* c = reinterpret_cast<SlotCache*>(cache);
  return with_cache(c, [&] {
    RoutePolicy& p = c->policy();
    const int F = c->files(), E = c->experts();
    if (scores) std::copy(p.scores().begin(), p.scores().end(), scores);
    if (quotas) std::copy(p.quotas().begin(), p.quotas().end(), quotas);
    for (int f = 0; f < F; ++f) {
      for (int e = 0; e < E; ++e) {
        if (short_rates) short_rates[(size_t)f * E + e] = p.rate(f, e, false);
        if (long_rates) long_rates[(size_t)f * E + e] = p.rate(f, e, true);
      }
      if (tokens) {
        tokens[f] = p.decode_tokens(f);
        tokens[F + f] = p.prompt_tokens(f);
      }
      if (read_cost) read_cost[f] = p.read_cost(f);
    }
    if (counters) {
      counters[0] = p.rebalances();
      counters[1] = p.capacity();
    }
  });
}

}  // extern "C"
