// mer_slots.hip -- VRAM expert-slot cache fed from host memory.
//
// The GPU side of MER's RAM/SSD -> VRAM tier (the physical VRAM registry
// and generation-keyed admission of backend/mod.rs:548-1047 and
// expert_cache.rs:715-1350): a fixed arena of n_slots expert-sized slots in
// HBM, a device table expert id -> slot pointer (null = not resident) that
// the routed-expert entry points take as their expert table, least-recently
// used eviction, and uploads from (pinned) host memory on a copy stream of
// the cache's own, so they overlap the compute stream's work.
//
// Ordering, all by HIP events (no host waits on the hot path):
//   - an upload into a slot first waits for the last compute that used the
//     slot's previous expert (the slot's release event);
//   - the compute stream waits for the uploads of the experts it needs;
//   - table entries change only on the compute stream, by a small kernel
//     whose (id, pointer) pairs travel as launch arguments, after the
//     uploads they publish and after earlier work that read the old
//     entries.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/mer_hip.h"
#include "mer_internal.hpp"

namespace mer {

constexpr int kTableUpdatesPerLaunch = 48;

struct TableUpdate {
  uint32_t n;
  uint32_t id[kTableUpdatesPerLaunch];
  uint64_t ptr[kTableUpdatesPerLaunch];
};

__global__ __launch_bounds__(64) void slot_table_kernel(uint64_t *table, TableUpdate u) {
  for (uint32_t i = threadIdx.x; i < u.n; i += 64) table[u.id[i]] = u.ptr[i];
}

}  // namespace mer

struct mer_slot_cache {
  struct Slot {
    int64_t expert = -1;        // resident expert id, -1 = free
    uint64_t generation = 0;
    uint64_t last_use = 0;      // LRU tick
    hipEvent_t uploaded = nullptr;  // completion of the slot's last upload
    hipEvent_t released = nullptr;  // completion of the last compute using it
    bool upload_recorded = false;
    bool release_recorded = false;
  };
  int device = -1;
  int dtype = 0;
  size_t expert_bytes = 0;
  size_t n_experts = 0;
  uint8_t *arena = nullptr;
  uint64_t *d_table = nullptr;
  hipStream_t copy_stream = nullptr;
  std::vector<Slot> slots;
  std::unordered_map<uint32_t, uint32_t> where;  // expert id -> slot
  std::vector<uint32_t> last_prepared;            // slots of the last prepare
  uint64_t tick = 0;
  mer_slot_stats stats{};
  std::mutex mu;
};

namespace {

int slot_fail(int status, const char *msg) { return mer::report_error(status, msg); }

// Choose a slot for a new expert: a free slot, else the least recently used
// slot not in `needed`.  Returns -1 when every slot is needed.
int64_t pick_victim(mer_slot_cache *c, const std::vector<char> &needed) {
  int64_t best = -1;
  for (size_t s = 0; s < c->slots.size(); ++s) {
    if (needed[s]) continue;
    if (c->slots[s].expert < 0) return (int64_t)s;
    if (best < 0 || c->slots[s].last_use < c->slots[best].last_use) best = (int64_t)s;
  }
  return best;
}

int flush_table(mer_slot_cache *c, mer::TableUpdate &u, hipStream_t st) {
  if (u.n == 0) return MER_OK;
  hipLaunchKernelGGL(mer::slot_table_kernel, dim3(1), dim3(64), 0, st, c->d_table, u);
  hipError_t e = hipGetLastError();
  u.n = 0;
  if (e != hipSuccess) return mer::report_hip_error(e, MER_ERR_SUBMISSION, "slot table update");
  return MER_OK;
}

int table_set(mer_slot_cache *c, mer::TableUpdate &u, uint32_t id, const void *ptr, hipStream_t st) {
  u.id[u.n] = id;
  u.ptr[u.n] = (uint64_t)(uintptr_t)ptr;
  if (++u.n == mer::kTableUpdatesPerLaunch) return flush_table(c, u, st);
  return MER_OK;
}

// Record, on `st`, that the compute enqueued there so far may use the slots
// of the last prepare: an upload into one of them waits for this point.
int release_last(mer_slot_cache *c, hipStream_t st) {
  for (uint32_t s : c->last_prepared) {
    hipError_t e = hipEventRecord(c->slots[s].released, st);
    if (e != hipSuccess) return mer::report_hip_error(e, MER_ERR_SUBMISSION, "record slot release");
    c->slots[s].release_recorded = true;
  }
  return MER_OK;
}

// Admit ids[0..n): hits are touched, misses uploaded into free or least
// recently used slots.  Generations follow the physical registry's
// directional rule (backend/mod.rs:709-741): equal = hit; a newer stored
// generation rejects the request (residency miss) without disturbing the
// entry; an older stored generation is retired and the request installs.
// With `publish`, the compute stream `st` waits for every needed upload and
// the table entries of all n experts are (re)written on it; without (a
// prefetch), only evictions are written and no stream waits.
int admit(mer_slot_cache *c, const uint32_t *ids, const uint64_t *generations, const void *const *host_blobs,
          size_t n, hipStream_t st, bool publish, const std::vector<uint32_t> &keep) {
  auto gen_of = [&](size_t i) { return generations ? generations[i] : (uint64_t)0; };
  // validation pass: nothing changes unless the whole request is admissible
  // (a prefetch is a hint: it is cut to the ids that fit, in order)
  std::unordered_map<uint32_t, uint64_t> seen;
  std::unordered_set<uint32_t> kept_expert;
  size_t at_once = 0;
  for (uint32_t s : keep)
    if (c->slots[s].expert >= 0) {
      kept_expert.insert((uint32_t)c->slots[s].expert);
      ++at_once;
    }
  for (size_t i = 0; i < n; ++i) {
    if (ids[i] >= c->n_experts) return slot_fail(MER_ERR_RESIDENCY_MISS, "expert id beyond the cache's table");
    auto d = seen.find(ids[i]);
    if (d != seen.end()) {
      if (d->second != gen_of(i)) return slot_fail(MER_ERR_INVALID_LAYOUT, "one expert id requested at two generations");
      continue;
    }
    if (!kept_expert.count(ids[i]) && at_once + 1 > c->slots.size()) {
      if (publish)
        return slot_fail(MER_ERR_PHYSICAL_CAPACITY, "more distinct experts needed at once than the cache has slots");
      n = i;
      break;
    }
    if (!kept_expert.count(ids[i])) ++at_once;
    seen[ids[i]] = gen_of(i);
    auto it = c->where.find(ids[i]);
    if (it != c->where.end() && c->slots[it->second].generation > gen_of(i))
      return slot_fail(MER_ERR_RESIDENCY_MISS, "physical GPU residency has a newer logical generation");
    if (it == c->where.end() || c->slots[it->second].generation != gen_of(i))
      if (!host_blobs || !host_blobs[i]) return slot_fail(MER_ERR_RESIDENCY_MISS, "expert not resident and no host blob given");
  }

  std::vector<char> needed(c->slots.size(), 0);
  for (uint32_t s : keep) needed[s] = 1;
  std::vector<int64_t> slot_of(n, -1);
  for (size_t i = 0; i < n; ++i) {
    auto it = c->where.find(ids[i]);
    if (it != c->where.end() && c->slots[it->second].generation == gen_of(i)) {
      slot_of[i] = it->second;
      if (!needed[it->second]) {
        needed[it->second] = 1;
        if (publish) ++c->stats.hits;
      }
      c->slots[it->second].last_use = ++c->tick;
    }
  }
  mer::TableUpdate u{};
  int rc;
  for (size_t i = 0; i < n; ++i) {
    if (slot_of[i] >= 0) continue;
    auto it = c->where.find(ids[i]);
    if (it != c->where.end()) {
      if (c->slots[it->second].generation == gen_of(i)) {  // installed earlier in this call
        slot_of[i] = it->second;
        continue;
      }
      // older generation: retire it
      c->slots[it->second].expert = -1;
      c->where.erase(it);
      if ((rc = table_set(c, u, ids[i], nullptr, st))) return rc;
      ++c->stats.stale_retirements;
    }
    const int64_t v = pick_victim(c, needed);
    if (v < 0) return slot_fail(MER_ERR_RUNTIME_INVARIANT, "no victim slot after the capacity check");
    mer_slot_cache::Slot &s = c->slots[v];
    if (s.expert >= 0) {
      c->where.erase((uint32_t)s.expert);
      if ((rc = table_set(c, u, (uint32_t)s.expert, nullptr, st))) return rc;
      ++c->stats.evictions;
    }
    uint8_t *dst = c->arena + (size_t)v * c->expert_bytes;
    hipError_t e = hipSuccess;
    if (s.release_recorded) e = hipStreamWaitEvent(c->copy_stream, s.released, 0);
    if (e == hipSuccess) e = hipMemcpyAsync(dst, host_blobs[i], c->expert_bytes, hipMemcpyHostToDevice, c->copy_stream);
    if (e == hipSuccess) e = hipEventRecord(s.uploaded, c->copy_stream);
    if (e != hipSuccess) return mer::report_hip_error(e, MER_ERR_UPLOAD, "expert upload");
    s.upload_recorded = true;
    s.expert = ids[i];
    s.generation = gen_of(i);
    s.last_use = ++c->tick;
    c->where[ids[i]] = (uint32_t)v;
    needed[v] = 1;
    slot_of[i] = v;
    if (publish) ++c->stats.misses;
    else ++c->stats.prefetches;
    c->stats.bytes_uploaded += c->expert_bytes;
  }
  if (publish) {
    std::vector<char> waited(c->slots.size(), 0);
    for (size_t i = 0; i < n; ++i) {
      mer_slot_cache::Slot &s = c->slots[slot_of[i]];
      if (waited[slot_of[i]] || !s.upload_recorded) continue;
      waited[slot_of[i]] = 1;
      hipError_t e = hipStreamWaitEvent(st, s.uploaded, 0);
      if (e != hipSuccess) return mer::report_hip_error(e, MER_ERR_SUBMISSION, "wait for expert upload");
    }
    for (size_t i = 0; i < n; ++i)
      if ((rc = table_set(c, u, ids[i], c->arena + (size_t)slot_of[i] * c->expert_bytes, st))) return rc;
    c->last_prepared.clear();
    for (size_t s = 0; s < c->slots.size(); ++s)
      if (needed[s]) c->last_prepared.push_back((uint32_t)s);
  }
  return flush_table(c, u, st);
}

}  // namespace

extern "C" {

int mer_slot_cache_create(int dtype, size_t d_model, size_t d_ff, size_t n_slots, size_t n_experts,
                          mer_slot_cache **out) {
  int rc = mer::check_initialised();
  if (rc) return rc;
  if (!out) return slot_fail(MER_ERR_INVALID_LAYOUT, "null output handle");
  *out = nullptr;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0) return slot_fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
  if (n_slots == 0 || n_experts == 0 || n_experts > (1u << 24))
    return slot_fail(MER_ERR_INVALID_LAYOUT, "n_slots and n_experts must be positive (n_experts <= 2^24)");
  const size_t eb = mer_expert_weight_bytes(dtype, d_model, d_ff);
  if (eb == 0 || eb == SIZE_MAX) return slot_fail(MER_ERR_INVALID_LAYOUT, "bad expert shape");
  mer_slot_cache *c = new (std::nothrow) mer_slot_cache();
  if (!c) return slot_fail(MER_ERR_PHYSICAL_CAPACITY, "host allocation");
  c->dtype = dtype;
  c->expert_bytes = eb;
  c->n_experts = n_experts;
  hipError_t e = hipGetDevice(&c->device);
  if (e == hipSuccess) e = hipMalloc(&c->arena, eb * n_slots);
  if (e == hipSuccess) e = hipMalloc(&c->d_table, n_experts * sizeof(uint64_t));
  if (e == hipSuccess) e = hipMemset(c->d_table, 0, n_experts * sizeof(uint64_t));
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking);
  c->slots.resize(n_slots);
  for (auto &s : c->slots) {
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.uploaded, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.released, hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    mer_slot_cache_destroy(c);
    return mer::report_hip_error(e, MER_ERR_PHYSICAL_CAPACITY, "slot cache allocation");
  }
  *out = c;
  return MER_OK;
}

int mer_slot_cache_destroy(mer_slot_cache *c) {
  if (!c) return MER_OK;
  if (c->copy_stream) (void)hipStreamSynchronize(c->copy_stream);
  (void)hipDeviceSynchronize();
  for (auto &s : c->slots) {
    if (s.uploaded) (void)hipEventDestroy(s.uploaded);
    if (s.released) (void)hipEventDestroy(s.released);
  }
  if (c->copy_stream) (void)hipStreamDestroy(c->copy_stream);
  if (c->d_table) (void)hipFree(c->d_table);
  if (c->arena) (void)hipFree(c->arena);
  delete c;
  return MER_OK;
}

const void *const *mer_slot_cache_table(mer_slot_cache *c) {
  return c ? reinterpret_cast<const void *const *>(c->d_table) : nullptr;
}

int mer_slot_cache_prepare(mer_slot_cache *c, const uint32_t *ids, const uint64_t *generations,
                           const void *const *host_blobs, size_t n, void *stream) {
  if (!c) return slot_fail(MER_ERR_INVALID_LAYOUT, "null cache");
  if (n && !ids) return slot_fail(MER_ERR_INVALID_LAYOUT, "null ids");
  std::lock_guard<std::mutex> lk(c->mu);
  hipStream_t st = (hipStream_t)stream;
  int rc = release_last(c, st);
  if (rc) return rc;
  return admit(c, ids, generations, host_blobs, n, st, true, {});
}

int mer_slot_cache_prefetch(mer_slot_cache *c, const uint32_t *ids, const uint64_t *generations,
                            const void *const *host_blobs, size_t n, void *stream) {
  if (!c) return slot_fail(MER_ERR_INVALID_LAYOUT, "null cache");
  if (n && !ids) return slot_fail(MER_ERR_INVALID_LAYOUT, "null ids");
  std::lock_guard<std::mutex> lk(c->mu);
  hipStream_t st = (hipStream_t)stream;
  int rc = release_last(c, st);
  if (rc) return rc;
  // the slots of the last prepare stay: its compute may still be queued
  return admit(c, ids, generations, host_blobs, n, st, false, c->last_prepared);
}

int mer_slot_cache_release(mer_slot_cache *c, void *stream) {
  if (!c) return slot_fail(MER_ERR_INVALID_LAYOUT, "null cache");
  std::lock_guard<std::mutex> lk(c->mu);
  return release_last(c, (hipStream_t)stream);
}

int mer_hip_host_alloc(size_t bytes, void **out) {
  if (!out) return slot_fail(MER_ERR_INVALID_LAYOUT, "null output pointer");
  *out = nullptr;
  hipError_t e = hipHostMalloc(out, bytes ? bytes : 1, hipHostMallocDefault);
  if (e != hipSuccess) return mer::report_hip_error(e, MER_ERR_PHYSICAL_CAPACITY, "pinned host allocation");
  return MER_OK;
}

int mer_hip_host_free(void *p) {
  if (!p) return MER_OK;
  hipError_t e = hipHostFree(p);
  if (e != hipSuccess) return mer::report_hip_error(e, MER_ERR_RUNTIME_INVARIANT, "pinned host free");
  return MER_OK;
}

int mer_slot_cache_stats(mer_slot_cache *c, mer_slot_stats *out) {
  if (!c || !out) return slot_fail(MER_ERR_INVALID_LAYOUT, "null cache or output");
  std::lock_guard<std::mutex> lk(c->mu);
  *out = c->stats;
  out->resident = 0;
  for (const auto &s : c->slots) out->resident += s.expert >= 0;
  return MER_OK;
}

}  // extern "C"
