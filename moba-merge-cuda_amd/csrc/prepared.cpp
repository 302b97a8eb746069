// Prepared-decode driver: the host side of one decode step for a fixed set
// of cache slots, in native code.
//
// A step (src/moba_opt/prepared_decode.py:141-158 semantics) is:
//   1. plan one token per leased slot on the page pool lease (positions, and
//      the (logical, physical) page of every row that starts a page);
//   2. if any row starts a page, stage that delta in a pinned ring slot and
//      copy it to the device delta buffer on the stream (no host sync: a ring
//      slot is reused only after the event of its previous copy completed);
//   3. refresh the split schedule of the fused kernel when some row moved by
//      more than 1/8 since the last refresh (rare; also staged through pinned
//      memory with an event);
//   4. launch the step: moba_hip_decode_fused (route + attention + scatter +
//      closing mean, then the split merge), or the multi-kernel sequence for
//      shapes the fused kernel does not take, or one hipGraphLaunch of the
//      captured launches;
//   5. commit the plan on the lease.
// An "attend" is the same without the append (positions = lengths - 1).
// Everything the device reads is a persistent buffer, so a captured graph of
// step 4 replays any later step.  hipGraph capture happens here too (a
// private stream in thread-local capture mode), without a framework's graph
// object.  No call allocates device memory.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <utility>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/moba_hip.h"

void moba_set_error(const char* fmt, ...);

namespace {

constexpr int kRing = 16;  // pinned delta staging slots

struct Prepared {
  MobaPrepDesc d;
  std::vector<int32_t> ids;
  bool ids_identity = false;  // row i is slot i: the fused launch skips the ids load
  int32_t* pinned = nullptr;       // [kRing][2 * rows] delta staging, then the schedule
  int32_t* sched_pinned = nullptr;
  hipEvent_t ring_ev[kRing] = {};
  bool ring_used[kRing] = {};
  hipEvent_t sched_ev = nullptr;
  bool sched_used = false;
  int ring_next = 0;
  int64_t delta_uploads = 0;
  // The device delta holds grants of a plan that was never committed (its
  // launch failed, or the caller did not commit).  Every launch applies the
  // delta it finds, so the next plan uploads its own delta even without
  // grants (all -1): otherwise a later launch would write a page into the
  // table that the host pool still counts as free.  A committed delta may
  // stay: re-applying it rewrites an entry the table already holds.
  bool delta_uncommitted = false;
  bool pending = false;            // a planned step awaiting moba_prep_commit
  int64_t pending_version = 0;
  std::vector<int32_t> delta;      // [2 * rows] of the current plan
  std::vector<int32_t> sched_pos;  // positions of the last schedule (empty: none)
  std::vector<int32_t> sched_splits;
  std::vector<int32_t> sched_entries;
  hipGraphExec_t graph[2] = {nullptr, nullptr};  // attend, step
};

int fail(int code, const char* msg) {
  moba_set_error("%s", msg);
  return code;
}

int hip_fail(const char* what, hipError_t e) {
  moba_set_error("%s: %s", what, hipGetErrorString(e));
  return MOBA_ERR_LAUNCH;
}

// Expected tokens one (row, kv head) attends at position pos: the current
// chunk up to pos, plus the closed chunks at least one of `group` q heads
// selects when each picks `remote` of them (expected coverage of independent
// uniform picks).
double expected_tokens(int pos, int group, int remote, int chunk, bool dense) {
  if (dense) return pos + 1.0;
  const int cur = pos / chunk, own = pos - cur * chunk + 1;
  if (cur == 0 || remote == 0) return own;
  const double picks = std::min(remote, cur);
  return own + chunk * cur * (1.0 - std::pow(1.0 - picks / cur, group));
}

// Fixed cost of one workgroup of a (row, kv head), in tokens of attention:
// before it streams any K/V every workgroup recomputes the row's route, and
// each (head, closed chunk) item of it costs about as much time as
// kRouteTokensPerItem tokens of attention (route phases of the fused kernel
// against its attention rate; 0.6 measured best of 0, 0.3, 0.6 and 1.2).
constexpr double kRouteTokensPerItem = 0.6;
double route_tokens(int pos, int group, int chunk, bool dense) {
  if (dense) return 0.0;
  return kRouteTokensPerItem * group * (pos / chunk);
}

}  // namespace

extern "C" int moba_prep_sched_workgroups(int rows, int hkv, int workgroups, int max_splits) {
  const int r = rows * hkv;
  return std::max(r, std::min(workgroups, r * max_splits));
}

extern "C" int moba_prep_schedule(const int32_t* positions, int rows, int hkv, int group,
                                  int remote, int chunk, int dense, int workgroups,
                                  int max_splits, int32_t* entries, int32_t* splits) {
  if (rows < 1 || hkv < 1 || chunk < 1 || max_splits < 1)
    return fail(MOBA_ERR_ARG, "prep_schedule: bad sizes");
  const int r = rows * hkv;
  const int total = moba_prep_sched_workgroups(rows, hkv, workgroups, max_splits);
  std::vector<double> w(r), f(r);
  for (int i = 0; i < r; ++i) {
    const int pos = std::max(0, (int)positions[i / hkv]);
    w[i] = std::max(1.0, expected_tokens(pos, group, remote, chunk, dense != 0));
    f[i] = route_tokens(pos, group, chunk, dense != 0);
  }
  // Each row starts with one split; every further workgroup goes to the row
  // whose workgroups have the most to do, route plus expected tokens per
  // split (ties: lowest row), until the grid is used or every row has
  // max_splits.  This minimises the largest per-workgroup time, which
  // bounds the launch's tail.
  std::vector<int> s(r, 1);
  int free = total - r;
  std::vector<std::pair<double, int>> heap;
  heap.reserve(r);
  auto before = [](const std::pair<double, int>& x, const std::pair<double, int>& y) {
    return x.first < y.first || (x.first == y.first && x.second > y.second);
  };
  for (int i = 0; i < r; ++i)
    if (max_splits > 1) heap.emplace_back(f[i] + w[i], i);
  std::make_heap(heap.begin(), heap.end(), before);
  while (free > 0 && !heap.empty()) {
    std::pop_heap(heap.begin(), heap.end(), before);
    const int i = heap.back().second;
    heap.pop_back();
    ++s[i];
    --free;
    if (s[i] < max_splits) {
      heap.emplace_back(f[i] + w[i] / s[i], i);
      std::push_heap(heap.begin(), heap.end(), before);
    }
  }
  // entries (row * hkv + kv head, split, splits), interleaved across rows so
  // one row's splits spread over the launch; then the split counts
  int e = 0, smax = 0;
  for (int i = 0; i < r; ++i) smax = std::max(smax, s[i]);
  for (int k = 0; k < smax; ++k)
    for (int i = 0; i < r; ++i)
      if (k < s[i]) { entries[3 * e] = i; entries[3 * e + 1] = k; entries[3 * e + 2] = s[i]; ++e; }
  // the launch has `total` workgroups and the kernels read the split counts
  // after 3 * total entries: every workgroup must hold one
  if (e != total) return fail(MOBA_ERR_ARG, "prep_schedule: workgroups not fully assigned");
  for (int i = 0; i < r; ++i) {
    entries[3 * e + i] = s[i];
    if (splits) splits[i] = s[i];
  }
  return MOBA_OK;
}

namespace {

// Launches of one step (append) or attend on `st`; every pointer is a
// persistent buffer of the descriptor.
int launch(Prepared& p, bool append, hipStream_t st) {
  const MobaPrepDesc& d = p.d;
  if (d.fused) {
    return moba_hip_decode_fused(d.q, append ? d.k : nullptr, append ? d.v : nullptr, d.dtype,
                                 d.rows, d.hq, d.hkv, d.head_dim, d.k_cache, d.v_cache,
                                 d.page_size, d.table, d.table_width, d.lengths,
                                 p.ids_identity ? nullptr : d.ids_dev,
                                 d.positions, d.delta, d.means, d.max_chunks, d.chunk, d.width,
                                 d.remote, d.dense, append ? 2 : 1, d.splits, d.sched, d.n_sched,
                                 d.dense ? nullptr : d.selected, d.part_o, d.part_ml, d.out,
                                 d.lse, st);
  }
  int rc = append ? moba_hip_decode_step(d.table, d.table_width, d.lengths, d.ids_dev,
                                         d.positions, d.delta, d.rows, d.k, d.v, d.dtype,
                                         d.k_cache, d.v_cache, d.page_size, d.hkv, d.head_dim,
                                         d.chunk, d.means, d.max_chunks, st)
                  : moba_hip_decode_metadata(d.table, d.table_width, d.lengths, d.ids_dev,
                                             d.positions, d.delta, d.rows, 0, st);
  if (rc) return rc;
  if (!d.dense) {
    rc = moba_hip_decode_route(d.q, d.dtype, d.rows, d.hq, d.hkv, d.head_dim, d.means,
                               d.max_chunks, d.ids_dev, d.positions, d.chunk, d.width, d.remote,
                               d.scores, d.selected, d.items, d.item_counts, st);
    if (rc) return rc;
  }
  return moba_hip_paged_attention(d.q, d.dtype, d.rows, d.hq, d.hkv, d.head_dim, d.k_cache,
                                  d.v_cache, d.page_size, d.table, d.table_width, d.lengths,
                                  d.ids_dev, d.positions, d.dense ? nullptr : d.selected,
                                  d.dense ? 0 : d.remote + 1, d.dense ? nullptr : d.items,
                                  d.dense ? nullptr : d.item_counts, d.dense, d.chunk,
                                  d.max_chunks, d.part_o, d.part_ml, d.out, d.lse, st);
}

// Stages host data in pinned memory and copies it to the device on the
// stream; waits only if the staging slot's previous copy is still pending.
int stage_copy(void* dev, int32_t* slot, hipEvent_t ev, bool& used, const int32_t* src, size_t n,
               hipStream_t st) {
  if (used) {
    hipError_t e = hipEventSynchronize(ev);
    if (e != hipSuccess) return hip_fail("prepared decode: staging wait", e);
  }
  std::memcpy(slot, src, n * sizeof(int32_t));
  hipError_t e = hipMemcpyAsync(dev, slot, n * sizeof(int32_t), hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipEventRecord(ev, st);
  if (e != hipSuccess) return hip_fail("prepared decode: staging copy", e);
  used = true;
  return MOBA_OK;
}

// Refreshes the fused launch's schedule when a row moved by more than 1/8.
int refresh_schedule(Prepared& p, const int32_t* pos, hipStream_t st) {
  const MobaPrepDesc& d = p.d;
  if (!d.fused || d.sched == nullptr) return MOBA_OK;
  if (!p.sched_pos.empty()) {
    bool near = true;
    for (int i = 0; i < d.rows && near; ++i)
      near = (int64_t)std::abs(pos[i] - p.sched_pos[i]) * 8 <= std::max(p.sched_pos[i], 1);
    if (near) return MOBA_OK;
  }
  // the fused launch's workgroups serve virtual kv heads of at most 16 q heads
  const int hv = d.hkv * moba_hip_decode_fused_groups(d.hq, d.hkv);
  const int n = 3 * d.n_sched + d.rows * hv;
  std::vector<int32_t> splits(d.rows * hv);
  p.sched_entries.resize(n);
  int rc = moba_prep_schedule(pos, d.rows, hv, d.hq / hv, d.remote, d.chunk, d.dense,
                              d.n_sched, d.splits, p.sched_entries.data(), splits.data());
  if (rc) return rc;
  if (splits != p.sched_splits) {
    rc = stage_copy(d.sched, p.sched_pinned, p.sched_ev, p.sched_used, p.sched_entries.data(),
                    n, st);
    if (rc) return rc;
    p.sched_splits = splits;
  }
  p.sched_pos.assign(pos, pos + d.rows);
  return MOBA_OK;
}

void release(Prepared* p) {
  for (auto& g : p->graph) if (g) hipGraphExecDestroy(g);
  for (auto& e : p->ring_ev) if (e) hipEventDestroy(e);
  if (p->sched_ev) hipEventDestroy(p->sched_ev);
  if (p->pinned) hipHostFree(p->pinned);
  delete p;
}

}  // namespace

extern "C" int moba_prep_create(const MobaPrepDesc* desc, const int32_t* ids, void** out) {
  if (!desc || !ids || !out) return fail(MOBA_ERR_ARG, "prep_create: null argument");
  *out = nullptr;
  const MobaPrepDesc& d = *desc;
  if (d.rows < 1 || d.hq < 1 || d.hkv < 1 || d.lease == nullptr)
    return fail(MOBA_ERR_ARG, "prep_create: bad descriptor");
  const int hv = d.hkv * moba_hip_decode_fused_groups(d.hq, d.hkv);  // 0: not a fused shape
  if (d.fused && (hv < 1 || d.splits < 1 || d.splits > 64 || (d.sched && d.n_sched < d.rows * hv)))
    return fail(MOBA_ERR_ARG, "prep_create: bad fused schedule sizes");
  Prepared* p = new (std::nothrow) Prepared;
  if (!p) return fail(MOBA_ERR_ARG, "prep_create: out of host memory");
  p->d = d;
  p->ids.assign(ids, ids + d.rows);
  p->ids_identity = true;
  for (int i = 0; i < d.rows; ++i) p->ids_identity = p->ids_identity && ids[i] == i;
  p->delta.assign(2 * d.rows, -1);
  const size_t ring = (size_t)kRing * 2 * d.rows;
  const size_t sched = d.fused && d.sched ? (size_t)3 * d.n_sched + (size_t)d.rows * hv : 0;
  hipError_t e = hipHostMalloc((void**)&p->pinned, (ring + sched + 1) * sizeof(int32_t),
                               hipHostMallocDefault);
  if (e != hipSuccess) { p->pinned = nullptr; release(p); return hip_fail("prep_create: pinned staging", e); }
  p->sched_pinned = p->pinned + ring;
  for (auto& ev : p->ring_ev)
    if ((e = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) {
      release(p);
      return hip_fail("prep_create: event", e);
    }
  if ((e = hipEventCreateWithFlags(&p->sched_ev, hipEventDisableTiming)) != hipSuccess) {
    release(p);
    return hip_fail("prep_create: event", e);
  }
  *out = p;
  return MOBA_OK;
}

extern "C" void moba_prep_destroy(void* h) {
  if (h) release(static_cast<Prepared*>(h));
}

extern "C" int64_t moba_prep_delta_uploads(const void* h) {
  return h ? static_cast<const Prepared*>(h)->delta_uploads : -1;
}

extern "C" int moba_prep_plan(void* h, int append, void* stream, int32_t* positions) {
  Prepared* p = static_cast<Prepared*>(h);
  if (!p) return fail(MOBA_ERR_ARG, "prep_plan: null handle");
  const MobaPrepDesc& d = p->d;
  hipStream_t st = (hipStream_t)stream;
  int grants = 0, rc;
  p->pending = false;
  if (append) {
    rc = moba_pool_plan_step(d.lease, p->ids.data(), d.rows, positions, p->delta.data(), &grants,
                             &p->pending_version);
    if (rc) return rc;
  } else {
    const int32_t* len = moba_pool_lengths(d.lease);
    for (int i = 0; i < d.rows; ++i) {
      positions[i] = len[p->ids[i]] - 1;
      if (positions[i] < 0) return fail(MOBA_ERR_ARG, "query positions must refer to cached tokens");
    }
  }
  if (!append) std::fill(p->delta.begin(), p->delta.end(), -1);  // an attend grants nothing
  if (grants || p->delta_uncommitted) {
    const int slot = p->ring_next;
    p->ring_next = (slot + 1) % kRing;
    rc = stage_copy(d.delta, p->pinned + (size_t)slot * 2 * d.rows, p->ring_ev[slot],
                    p->ring_used[slot], p->delta.data(), 2 * (size_t)d.rows, st);
    if (rc) return rc;
    ++p->delta_uploads;
    p->delta_uncommitted = grants != 0;
  }
  if ((rc = refresh_schedule(*p, positions, st))) return rc;
  p->pending = append != 0;
  return MOBA_OK;
}

extern "C" int moba_prep_launch(void* h, int append, int use_graph, void* stream) {
  Prepared* p = static_cast<Prepared*>(h);
  if (!p) return fail(MOBA_ERR_ARG, "prep_launch: null handle");
  hipStream_t st = (hipStream_t)stream;
  if (use_graph) {
    hipGraphExec_t g = p->graph[append ? 1 : 0];
    if (!g) return fail(MOBA_ERR_ARG, append ? "capture('step') first" : "capture('attend') first");
    hipError_t e = hipGraphLaunch(g, st);
    if (e != hipSuccess) return hip_fail("prepared decode: graph launch", e);
    return MOBA_OK;
  }
  return launch(*p, append != 0, st);
}

extern "C" int moba_prep_commit(void* h) {
  Prepared* p = static_cast<Prepared*>(h);
  if (!p) return fail(MOBA_ERR_ARG, "prep_commit: null handle");
  if (!p->pending) return MOBA_OK;
  p->pending = false;
  const int rc = moba_pool_commit_step(p->d.lease, p->ids.data(), p->d.rows, p->delta.data(),
                                       p->pending_version);
  if (rc == MOBA_OK) p->delta_uncommitted = false;
  return rc;
}

extern "C" int moba_prep_run(void* h, int append, int use_graph, void* stream,
                             int32_t* positions) {
  Prepared* p = static_cast<Prepared*>(h);
  if (!p) return fail(MOBA_ERR_ARG, "prep_run: null handle");
  if (use_graph && !p->graph[append ? 1 : 0])
    return fail(MOBA_ERR_ARG, append ? "capture('step') first" : "capture('attend') first");
  int rc = moba_prep_plan(h, append, stream, positions);
  if (rc == MOBA_OK) rc = moba_prep_launch(h, append, use_graph, stream);
  if (rc == MOBA_OK) rc = moba_prep_commit(h);
  else p->pending = false;
  return rc;
}

extern "C" int moba_prep_capture(void* h, int append, void* stream) {
  Prepared* p = static_cast<Prepared*>(h);
  if (!p) return fail(MOBA_ERR_ARG, "prep_capture: null handle");
  hipGraphExec_t& slot = p->graph[append ? 1 : 0];
  if (slot) return fail(MOBA_ERR_ARG, "graph already captured");
  const MobaPrepDesc& d = p->d;
  // the schedule the replays read must be valid before the first replay
  std::vector<int32_t> pos(d.rows);
  const int32_t* len = moba_pool_lengths(d.lease);
  for (int i = 0; i < d.rows; ++i) pos[i] = std::max(0, len[p->ids[i]] - (append ? 0 : 1));
  hipStream_t user = (hipStream_t)stream;
  int rc = refresh_schedule(*p, pos.data(), user);
  if (rc) return rc;
  hipStream_t cs = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&cs, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail("prep_capture: stream", e);
  // the capture stream starts after the user stream's pending work
  hipEvent_t ev = nullptr;
  e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(ev, user);
  if (e == hipSuccess) e = hipStreamWaitEvent(cs, ev, 0);
  hipGraph_t graph = nullptr;
  if (e == hipSuccess) e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    rc = launch(*p, append != 0, cs);
    hipError_t e2 = hipStreamEndCapture(cs, &graph);
    if (rc == MOBA_OK && e2 != hipSuccess) e = e2;
  }
  if (e == hipSuccess && rc == MOBA_OK) e = hipGraphInstantiate(&slot, graph, nullptr, nullptr, 0);
  if (e == hipSuccess && rc == MOBA_OK) e = hipGraphUpload(slot, user);
  if (graph) hipGraphDestroy(graph);
  if (ev) hipEventDestroy(ev);
  hipStreamDestroy(cs);
  if (rc) return rc;
  if (e != hipSuccess) {
    if (slot) { hipGraphExecDestroy(slot); slot = nullptr; }
    return hip_fail("prep_capture", e);
  }
  return MOBA_OK;
}
