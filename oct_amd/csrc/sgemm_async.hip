// Asynchronous SGEMM tasks and the ordered-commit SGEMM batch.
//
// Reference contract (internal/prometheus/native):
//   task table and ids        reactor_sgemm.cpp:6028-6083 (4 records; id =
//                             generation << 4 | (index + 1); a record is reused
//                             only after its task was consumed or abandoned)
//   submit/query/consume/abandon  reactor_sgemm.cpp:6298-6502 (stages and
//                             detail codes reproduced call by call)
//   sync SGEMM while tasks are unconsumed is rejected  reactor_sgemm.cpp:4204-4211
//   batch                     reactor_batch.c:60-243 (plan, logical lanes,
//                             deterministic first-failure choice) and :244-560
//                             (stop admission on failure, drain, commit every
//                             output in entry order only when all succeeded)
//   public batch flag mask    reactor_sgemm.cpp:5953-6009
//
// MI355X design.  The reference moves each task through host-visible Vulkan
// buffers and a two-slot fence ring.  Here a submission slot owns a grow-only
// device arena (A|B|C), pinned host staging for the inputs and the output, and
// three HIP events.  Submit copies the caller's A and B into pinned memory (so
// the caller may reuse them at once), then enqueues upload -> MFMA SGEMM ->
// download on the runtime's stream and returns; query is hipEventQuery; consume
// copies the pinned result out.  A batch uploads entry after entry into one
// device arena, launches every SGEMM back to back on the same stream, downloads
// into a pinned staging arena, waits once per arena fill and commits to the
// caller's outputs only after every entry has completed.
#include <stdlib.h>
#include <string.h>

#include <new>
#include <vector>

#include "reactor_internal.h"

namespace prom {

namespace {

constexpr uint32_t kTaskCapacity = 4;     // PROM_SGEMM_ASYNC_MAX_TASKS
constexpr uint32_t kAsyncSlots = 2;       // PROM_SGEMM_SUBMISSION_RING_DEFAULT_DEPTH
constexpr uint32_t kRingMaxDepth = 4;     // PROM_SGEMM_SUBMISSION_RING_MAX_DEPTH
constexpr uint32_t kBatchMaxLogicalWidth = 8;
constexpr uint32_t kBatchPlanGeneration = 1;
constexpr uint32_t kBatchProductionFlags = 0xffu | PROM_BATCH_FLAG_PARTITION_CONTIGUOUS;
constexpr uint32_t kBatchTimedEntries = 64;
// Device bytes one batch arena fill may hold before the batch waits and reuses it.
constexpr size_t kBatchArenaBudget = (size_t)4 << 30;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Slot {
  uint32_t state = PROM_ASYNC_PHYSICAL_EMPTY;
  uint32_t generation = 0;
  uint64_t sequence = 0;
  void* dev = nullptr;
  size_t dev_bytes = 0;
  float* host_in = nullptr;
  size_t host_in_bytes = 0;
  float* host_out = nullptr;
  size_t host_out_bytes = 0;
  hipEvent_t start = nullptr, kernel_end = nullptr, done = nullptr;
};

struct Task {
  uint32_t active, generation, lifecycle, table_index;
  int public_id;
  uint32_t m, n, k;
  uint32_t slot, slot_generation;
  uint64_t sequence;
  uint32_t final_stage;
  int final_detail;
  uint32_t failure_class;
  uint32_t abandoned, quarantined, reap_pending, reap_completed, completion_confirmed;
  uint32_t timing_valid;
  uint64_t gpu_ns;
};

}  // namespace

struct AsyncState {
  Task tasks[kTaskCapacity] = {};
  Slot slots[kRingMaxDepth];
  uint32_t cursor = 0;
  uint64_t next_task_sequence = 1, next_slot_sequence = 1, next_batch_sequence = 1;
  uint64_t queue_full = 0, stale_rejects = 0, quarantine_events = 0;
  uint64_t reap_polls = 0, reap_success = 0, reap_waits = 0, reap_failures = 0;
  uint32_t max_in_flight = 0, max_quarantine_depth = 0;
  PrometheusSgemmBatchDiagnostics batch{};
  void* batch_dev = nullptr;
  size_t batch_dev_bytes = 0;
  float* batch_host = nullptr;
  size_t batch_host_bytes = 0;
  hipEvent_t batch_events[2 * kBatchTimedEntries] = {};
  bool batch_events_ready = false;
};

namespace {

// ---- buffers ----------------------------------------------------------------
bool grow_device(void** p, size_t* have, size_t need, hipStream_t stream) {
  if (*have >= need) return true;
  if (*p != nullptr) {
    if (hipStreamSynchronize(stream) != hipSuccess) return false;
    (void)hipFree(*p);
    *p = nullptr;
    *have = 0;
  }
  const size_t rounded = (need + (2u << 20) - 1) & ~(size_t)((2u << 20) - 1);
  if (hipMalloc(p, rounded) != hipSuccess) {
    (void)hipGetLastError();
    *p = nullptr;
    return false;
  }
  *have = rounded;
  return true;
}

bool grow_pinned(float** p, size_t* have, size_t need, hipStream_t stream) {
  if (*have >= need) return true;
  if (*p != nullptr) {
    if (hipStreamSynchronize(stream) != hipSuccess) return false;
    (void)hipHostFree(*p);
    *p = nullptr;
    *have = 0;
  }
  const size_t rounded = (need + (2u << 20) - 1) & ~(size_t)((2u << 20) - 1);
  void* q = nullptr;
  if (hipHostMalloc(&q, rounded, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  *p = static_cast<float*>(q);
  *have = rounded;
  return true;
}

bool ensure_slot_events(Slot& s) {
  if (s.done != nullptr) return true;
  return hipEventCreate(&s.start) == hipSuccess && hipEventCreate(&s.kernel_end) == hipSuccess &&
         hipEventCreate(&s.done) == hipSuccess;
}

bool checked_mul_u32(uint32_t a, uint32_t b, uint32_t* out) {
  const uint64_t v = (uint64_t)a * b;
  if (v > 0xffffffffull) return false;
  *out = (uint32_t)v;
  return true;
}

// ---- task table -------------------------------------------------------------
bool encode_task_id(uint32_t index, uint32_t generation, int* out) {
  const uint32_t id = ((generation & 0x07ffffffu) << 4u) | (index + 1u);
  if (id == 0u || (id & 0x80000000u) != 0u) return false;
  *out = (int)id;
  return true;
}

void release_task(Task* t) {
  const uint32_t generation = t->generation;
  memset(t, 0, sizeof(*t));
  t->generation = generation;
}

Task* allocate_task(AsyncState* st) {
  for (uint32_t off = 0; off < kTaskCapacity; ++off) {
    const uint32_t index = (st->cursor + off) % kTaskCapacity;
    Task* t = &st->tasks[index];
    if (t->active && t->lifecycle == PROM_ASYNC_STATE_CONSUMED && !t->reap_pending) release_task(t);
    if (!t->active) {
      uint32_t generation = t->generation + 1u;
      if (generation == 0u) generation = 1u;
      memset(t, 0, sizeof(*t));
      t->active = 1;
      t->table_index = index;
      t->generation = generation;
      t->lifecycle = PROM_ASYNC_STATE_IDLE;
      if (!encode_task_id(index, generation, &t->public_id)) {
        t->active = 0;
        return nullptr;
      }
      st->cursor = (index + 1u) % kTaskCapacity;
      return t;
    }
  }
  return nullptr;
}

Task* lookup_task(AsyncState* st, int task_id) {
  if (st == nullptr || task_id <= 0) return nullptr;
  const uint32_t low = (uint32_t)task_id & 0x0fu;
  const uint32_t generation = ((uint32_t)task_id >> 4u) & 0x07ffffffu;
  if (low == 0u || low > kTaskCapacity) return nullptr;
  Task* t = &st->tasks[low - 1u];
  if (!t->active || (t->generation & 0x07ffffffu) != generation || t->public_id != task_id) return nullptr;
  return t;
}

uint32_t outstanding(const AsyncState* st) {
  if (st == nullptr) return 0;
  uint32_t n = 0;
  for (const Task& t : st->tasks)
    if (t.active && t.lifecycle != PROM_ASYNC_STATE_CONSUMED) ++n;
  return n;
}

Slot* task_slot(AsyncState* st, Task* t) {
  if (t->slot >= kAsyncSlots) return nullptr;
  Slot* s = &st->slots[t->slot];
  return s->generation == t->slot_generation ? s : nullptr;
}

void count_quarantine(AsyncState* st) {
  uint32_t q = 0;
  for (uint32_t i = 0; i < kAsyncSlots; ++i)
    if (st->slots[i].state == PROM_ASYNC_PHYSICAL_QUARANTINED) ++q;
  if (q > st->max_quarantine_depth) st->max_quarantine_depth = q;
}

// A failed task keeps its slot quarantined until the slot's work is known to
// have finished (the reference's reap, reactor_sgemm.cpp:6120-6190).
void fail_task(AsyncState* st, Task* t, uint32_t failure_class, int detail) {
  t->lifecycle = PROM_ASYNC_STATE_FAILED;
  t->final_stage = PROM_STAGE_SUBMIT;
  t->final_detail = detail;
  t->failure_class = failure_class;
  Slot* s = task_slot(st, t);
  if (s != nullptr) {
    s->state = PROM_ASYNC_PHYSICAL_QUARANTINED;
    t->quarantined = 1;
    t->reap_pending = 1;
    st->quarantine_events++;
    count_quarantine(st);
  }
}

void reap(AsyncState* st, bool wait) {
  if (st == nullptr) return;
  for (Task& t : st->tasks) {
    if (!t.active || !t.reap_pending) continue;
    Slot* s = task_slot(st, &t);
    if (s == nullptr) {
      t.reap_pending = 0;
      t.quarantined = 0;
      continue;
    }
    st->reap_polls++;
    if (wait) {
      st->reap_waits++;
      (void)hipEventSynchronize(s->done);
    }
    const hipError_t e = hipEventQuery(s->done);
    if (e == hipSuccess) {
      t.reap_pending = 0;
      t.reap_completed = 1;
      t.quarantined = 0;
      t.completion_confirmed = 1;
      s->state = PROM_ASYNC_PHYSICAL_EMPTY;
      st->reap_success++;
      if (t.abandoned) {
        t.lifecycle = PROM_ASYNC_STATE_CONSUMED;
        release_task(&t);
      }
    } else if (e != hipErrorNotReady) {
      (void)hipGetLastError();
      st->reap_failures++;
    }
  }
}

void poll_task(Runtime* rt, AsyncState* st, Task* t) {
  if (t->lifecycle != PROM_ASYNC_STATE_SUBMITTED) return;
  Slot* s = task_slot(st, t);
  if (s == nullptr) {
    fail_task(st, t, PROM_ASYNC_FAILURE_OBSERVATION, PROM_DETAIL_ASYNC_FAILED);
    return;
  }
  if (rt->test_flags & PROM_TESTCFG_FAIL_ASYNC_POLL) {
    fail_task(st, t, PROM_ASYNC_FAILURE_OBSERVATION, PROM_DETAIL_INJECTED_ASYNC_POLL_FAILURE);
    return;
  }
  const hipError_t e = hipEventQuery(s->done);
  if (e == hipErrorNotReady) return;
  if (e != hipSuccess) {
    (void)hipGetLastError();
    fail_task(st, t, PROM_ASYNC_FAILURE_QUERY, PROM_DETAIL_ASYNC_FAILED);
    return;
  }
  t->lifecycle = PROM_ASYNC_STATE_READY;
  t->final_stage = PROM_STAGE_TRANSFER_OUT;
  t->completion_confirmed = 1;
  s->state = PROM_ASYNC_PHYSICAL_READY;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, s->start, s->kernel_end) == hipSuccess) {
    t->timing_valid = 1;
    t->gpu_ns = (uint64_t)((double)ms * 1.0e6);
  } else {
    (void)hipGetLastError();
  }
}

AsyncState* ensure_async(Runtime* rt) {
  if (rt->async == nullptr) rt->async = new (std::nothrow) AsyncState();
  return rt->async;
}

// ---- batch ------------------------------------------------------------------
uint32_t batch_requested_width(uint32_t flags) {
  const uint32_t w = flags & 0xffu;
  return w == 0u ? 1u : w;
}

uint32_t batch_lane(uint32_t entry, uint32_t count, uint32_t width, uint32_t flags) {
  if (flags & PROM_BATCH_FLAG_PARTITION_CONTIGUOUS) {
    if (count == 0u || width == 0u) return 0u;
    return (uint32_t)(((uint64_t)entry * width) / count);
  }
  return width == 0u ? 0u : entry % width;
}

uint32_t batch_test_fail_entry(uint32_t flags, uint32_t count) {
  const uint32_t encoded = (flags & PROM_BATCH_FLAG_TEST_FAIL_ENTRY_MASK) >> PROM_BATCH_FLAG_TEST_FAIL_ENTRY_SHIFT;
  if (encoded == 0u || count == 0u || encoded > count) return UINT32_MAX;
  return encoded - 1u;
}

void batch_diag_header(PrometheusSgemmBatchDiagnostics* d, uint32_t count, uint32_t flags) {
  memset(d, 0, sizeof(*d));
  d->last_batch_entry_count = count;
  d->requested_workers = batch_requested_width(flags);
  uint32_t eff = d->requested_workers > kBatchMaxLogicalWidth ? kBatchMaxLogicalWidth : d->requested_workers;
  if (count != 0u && eff > count) eff = count;
  d->effective_workers = eff;
  d->partition_policy = (flags & PROM_BATCH_FLAG_PARTITION_CONTIGUOUS) ? PROM_BATCH_PARTITION_CONTIGUOUS
                                                                       : PROM_BATCH_PARTITION_ROUND_ROBIN;
  d->plan_generation = kBatchPlanGeneration;
}

void batch_fail_diag(PrometheusSgemmBatchDiagnostics* d, uint32_t entry, uint32_t lane, uint32_t stage, int detail) {
  d->batch_state = PROM_BATCH_STATE_FAILED;
  d->failed_entry_id = entry;
  d->failed_worker_id = lane;
  d->failure_stage = stage;
  d->failure_detail = detail;
  d->failure_count = 1;
  d->first_failure_stable = 1;
  d->output_committed = 0;
}

int batch_execute(Runtime* rt, const PrometheusSgemmBatchEntry* entries, uint32_t count, uint32_t flags,
                  bool test_seams, uint32_t* out_stage, int* out_detail) {
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  AsyncState* st = ensure_async(rt);
  if (st == nullptr) {
    set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_INTERNAL_ERROR);
    return PROM_INTERNAL_ERROR;
  }
  PrometheusSgemmBatchDiagnostics& d = st->batch;
  if (!test_seams && (flags & ~kBatchProductionFlags) != 0u) {
    batch_diag_header(&d, count, flags);
    d.batch_state = PROM_BATCH_STATE_FAILED;
    d.failure_stage = PROM_STAGE_INIT;
    d.failure_detail = PROM_DETAIL_BATCH_UNSUPPORTED_OPTION;
    d.failure_count = 1;
    set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_DETAIL_BATCH_UNSUPPORTED_OPTION);
    return PROM_ERROR;
  }
  if (!rt->available) {
    set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_DETAIL_BATCH_EXECUTION_FAILED);
    return PROM_ERROR;
  }
  if (entries == nullptr || count == 0u) {
    set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_ERROR);
    return PROM_ERROR;
  }
  // Plan: validate every entry before any work is enqueued (reactor_batch.c:88-182).
  const uint32_t width = batch_requested_width(flags) > kBatchMaxLogicalWidth
                             ? kBatchMaxLogicalWidth
                             : batch_requested_width(flags);
  const uint32_t planned = width > count ? count : width;
  size_t host_total = 0;
  for (uint32_t i = 0; i < count; ++i) {
    const PrometheusSgemmBatchEntry& e = entries[i];
    uint32_t ac, bc, cc;
    if (e.a == nullptr || e.b == nullptr || e.c == nullptr || e.m == 0u || e.n == 0u || e.k == 0u ||
        !checked_mul_u32(e.m, e.k, &ac) || !checked_mul_u32(e.k, e.n, &bc) || !checked_mul_u32(e.m, e.n, &cc)) {
      batch_diag_header(&d, count, flags);
      batch_fail_diag(&d, i, batch_lane(i, count, planned, flags), PROM_STAGE_INIT, PROM_DETAIL_BATCH_PLAN_INVALID);
      set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_DETAIL_BATCH_PLAN_INVALID);
      return PROM_ERROR;
    }
    host_total += align256((size_t)cc * sizeof(float));
  }
  batch_diag_header(&d, count, flags);
  d.batch_state = PROM_BATCH_STATE_RUNNING;
  d.execution_mode = PROM_BATCH_EXECUTION_SINGLE_WORKER;
  d.worker_resource_mode = PROM_BATCH_WORKER_RESOURCE_SHARED;
  d.queue_topology_classification = PROM_BATCH_QUEUE_TOPOLOGY_SINGLE_QUEUE;
  d.queue_mapping_mode = PROM_BATCH_QUEUE_MAPPING_SINGLE_QUEUE_SERIALIZED;
  const uint32_t depth = rt->batch_ring_depth;
  d.physical_ring_depth_configured = depth;
  d.physical_ring_depth_effective = depth > kTaskCapacity ? kTaskCapacity : depth;
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t lane = batch_lane(i, count, planned, flags);
    if (lane < 8u) d.worker_assigned_count[lane]++;
  }

  // Pinned staging for every output: outputs reach the caller only at commit.
  if (!grow_pinned(&st->batch_host, &st->batch_host_bytes, host_total, cx.stream)) {
    batch_fail_diag(&d, 0, batch_lane(0, count, planned, flags), PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_HIP_ALLOC_FAILED);
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_HIP_ALLOC_FAILED);
    return PROM_ERROR;
  }
  if (!st->batch_events_ready) {
    bool ok = true;
    for (uint32_t i = 0; i < 2 * kBatchTimedEntries && ok; ++i) ok = hipEventCreate(&st->batch_events[i]) == hipSuccess;
    st->batch_events_ready = ok;
  }

  const uint32_t fail_entry = test_seams ? batch_test_fail_entry(flags, count) : UINT32_MAX;
  bool failed = false;
  uint32_t failed_entry = UINT32_MAX, failure_stage = PROM_STAGE_NONE;
  int failure_detail = 0;
  uint32_t next = 0, completed = 0, fill = 0;
  size_t host_off = 0;
  std::vector<size_t> host_offsets(count);
  for (uint32_t i = 0; i < count; ++i) {
    host_offsets[i] = host_off;
    host_off += align256((size_t)entries[i].m * entries[i].n * sizeof(float));
  }

  while (!failed && next < count) {
    // One arena fill: entries in order until the device budget is reached.
    const uint32_t first = next;
    size_t dev_need = 0;
    uint32_t last = first;
    while (last < count) {
      const PrometheusSgemmBatchEntry& e = entries[last];
      const size_t need = align256((size_t)e.m * e.k * 4) + align256((size_t)e.k * e.n * 4) +
                          align256((size_t)e.m * e.n * 4);
      if (last > first && dev_need + need > kBatchArenaBudget) break;
      dev_need += need;
      ++last;
    }
    if (!grow_device(&st->batch_dev, &st->batch_dev_bytes, dev_need, cx.stream)) {
      failed = true;
      failed_entry = first;
      failure_stage = PROM_STAGE_TRANSFER_IN;
      failure_detail = PROM_DETAIL_HIP_ALLOC_FAILED;
      break;
    }
    char* arena = static_cast<char*>(st->batch_dev);
    size_t off = 0;
    for (uint32_t i = first; i < last && !failed; ++i) {
      const PrometheusSgemmBatchEntry& e = entries[i];
      const size_t ab = (size_t)e.m * e.k * 4, bb = (size_t)e.k * e.n * 4, cb = (size_t)e.m * e.n * 4;
      float* da = reinterpret_cast<float*>(arena + off);
      off += align256(ab);
      float* db = reinterpret_cast<float*>(arena + off);
      off += align256(bb);
      float* dc = reinterpret_cast<float*>(arena + off);
      off += align256(cb);
      const uint32_t lane = batch_lane(i, count, planned, flags);
      if (upload_host(da, e.a, ab, cx.stream) != hipSuccess || upload_host(db, e.b, bb, cx.stream) != hipSuccess) {
        (void)hipGetLastError();
        failed = true;
        failed_entry = i;
        failure_stage = PROM_STAGE_TRANSFER_IN;
        failure_detail = PROM_DETAIL_HIP_COPY_FAILED;
        break;
      }
      const bool timed = st->batch_events_ready && i < kBatchTimedEntries;
      if (timed) (void)hipEventRecord(st->batch_events[2 * i], cx.stream);
      int path = 0;
      if (launch_sgemm_f32(da, db, dc, e.m, e.n, e.k, cx.stream, &path) != hipSuccess) {
        (void)hipGetLastError();
        failed = true;
        failed_entry = i;
        failure_stage = PROM_STAGE_SUBMIT;
        failure_detail = PROM_DETAIL_BATCH_QUEUE_SUBMIT_FAILED;
        break;
      }
      if (timed) (void)hipEventRecord(st->batch_events[2 * i + 1], cx.stream);
      if (hipMemcpyAsync(reinterpret_cast<char*>(st->batch_host) + host_offsets[i], dc, cb, hipMemcpyDeviceToHost,
                         cx.stream) != hipSuccess) {
        (void)hipGetLastError();
        failed = true;
        failed_entry = i;
        failure_stage = PROM_STAGE_TRANSFER_OUT;
        failure_detail = PROM_DETAIL_HIP_COPY_FAILED;
        break;
      }
      d.total_submits++;
      if (i < 64u) {
        d.m31_submission_sequence[i] = st->next_batch_sequence;
        d.m31_physical_slot_id[i] = fill;
      }
      st->next_batch_sequence++;
      if (lane < 8u) {
        d.worker_submit_count[lane]++;
        d.worker_event_count[lane] += 2u;
      }
      next = i + 1;
      // Test seams (reactor_batch.c:382-407): a failure observed after submission.
      if (test_seams) {
        if ((flags & PROM_BATCH_FLAG_FAIL_AFTER_FIRST_SUBMIT) && next == 1u) {
          failed = true;
          failed_entry = 0;
        } else if (next - 1u == fail_entry) {
          failed = true;
          failed_entry = fail_entry;
        } else if ((flags & PROM_BATCH_FLAG_TEST_DUAL_FAIL_FIRST_TWO) && next == 2u) {
          // entries 0 and 1 fail together; the lower entry id is the stable cause
          failed = true;
          failed_entry = 0;
        }
        if (failed) {
          failure_stage = PROM_STAGE_SUBMIT;
          failure_detail = PROM_DETAIL_BATCH_EXECUTION_FAILED;
        }
      }
    }
    const uint32_t in_flight = next - first;
    if (in_flight > d.max_in_flight) d.max_in_flight = in_flight;
    // Drain this fill (also on failure: every enqueued entry finishes before
    // the arena and the staging are reused).
    d.total_forced_waits++;
    if (hipStreamSynchronize(cx.stream) != hipSuccess) {
      (void)hipGetLastError();
      if (!failed) {
        failed = true;
        failed_entry = first;
        failure_stage = PROM_STAGE_SUBMIT;
        failure_detail = PROM_DETAIL_BATCH_FENCE_WAIT_FAILED;
      }
    }
    if (!failed) {
      for (uint32_t i = first; i < next; ++i) {
        const uint32_t lane = batch_lane(i, count, planned, flags);
        if (i < 64u) {
          d.m31_completion_status[i] = 1u;
          d.m31_completion_order[completed] = i;
          float ms = 0.f;
          if (st->batch_events_ready && hipEventElapsedTime(&ms, st->batch_events[2 * i], st->batch_events[2 * i + 1]) ==
                                            hipSuccess)
            d.m31_gpu_duration_ns[i] = (uint64_t)((double)ms * 1.0e6);
        }
        if (lane < 8u) {
          d.worker_completed_count[lane]++;
          d.worker_event_count[lane] += 1u;
        }
        ++completed;
      }
    }
    ++fill;
  }
  d.m31_completion_count = completed;
  d.current_in_flight = 0;
  if (failed || completed != count) {
    const uint32_t lane = failed_entry < count ? batch_lane(failed_entry, count, planned, flags) : UINT32_MAX;
    batch_fail_diag(&d, failed_entry, lane, failure_stage == PROM_STAGE_NONE ? PROM_STAGE_SUBMIT : failure_stage,
                    failure_detail == 0 ? PROM_ERROR : failure_detail);
    set_status(out_stage, out_detail, d.failure_stage, d.failure_detail);
    return PROM_ERROR;
  }
  // Ordered commit (reactor_batch.c:538-541).
  for (uint32_t i = 0; i < count; ++i) {
    host_memcpy(entries[i].c, reinterpret_cast<const char*>(st->batch_host) + host_offsets[i],
           (size_t)entries[i].m * entries[i].n * sizeof(float));
    if (i < 64u) d.m31_commit_order[i] = i;
  }
  d.m31_commit_count = count;
  d.output_committed = 1;
  d.batch_state = PROM_BATCH_STATE_SUCCEEDED;
  rt->successes++;
  set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, 0);
  return PROM_OK;
}

}  // namespace

// Called by the synchronous SGEMM entry and by destroy.
uint32_t async_outstanding(Runtime* rt) {
  if (rt == nullptr) return 0u;
  std::lock_guard<std::mutex> lock(ctx().mu);
  return outstanding(rt->async);
}

void async_release(Runtime* rt) {
  AsyncState* st = rt->async;
  if (st == nullptr) return;
  DeviceContext& cx = ctx();
  {
    std::lock_guard<std::mutex> lock(cx.mu);
    if (cx.available) (void)hipStreamSynchronize(cx.stream);
    for (Slot& s : st->slots) {
      if (s.dev) (void)hipFree(s.dev);
      if (s.host_in) (void)hipHostFree(s.host_in);
      if (s.host_out) (void)hipHostFree(s.host_out);
      if (s.start) (void)hipEventDestroy(s.start);
      if (s.kernel_end) (void)hipEventDestroy(s.kernel_end);
      if (s.done) (void)hipEventDestroy(s.done);
    }
    if (st->batch_dev) (void)hipFree(st->batch_dev);
    if (st->batch_host) (void)hipHostFree(st->batch_host);
    if (st->batch_events_ready)
      for (hipEvent_t e : st->batch_events) (void)hipEventDestroy(e);
  }
  delete st;
  rt->async = nullptr;
}

}  // namespace prom

using namespace prom;

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_submit_async(void* handle, const float* a, const float* b,
                                                                   uint32_t m, uint32_t n, uint32_t k,
                                                                   int* out_task_id, uint32_t* out_stage,
                                                                   int* out_detail_code) {
  if (out_task_id == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_ERROR);
    return PROM_ERROR;
  }
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  uint32_t ac, bc, cc;
  if (!rt->available || a == nullptr || b == nullptr || m == 0u || n == 0u || k == 0u || !checked_mul_u32(m, k, &ac) ||
      !checked_mul_u32(k, n, &bc) || !checked_mul_u32(m, n, &cc)) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_ERROR);
    return PROM_ERROR;
  }
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  AsyncState* st = ensure_async(rt);
  if (st == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_INTERNAL_ERROR);
    return PROM_INTERNAL_ERROR;
  }
  reap(st, false);
  for (Task& t : st->tasks)
    if (t.active) poll_task(rt, st, &t);
  Task* task = allocate_task(st);
  if (task == nullptr) {
    st->queue_full++;
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_ASYNC_QUEUE_FULL);
    return PROM_ERROR;
  }
  uint32_t slot_index = kAsyncSlots;
  for (uint32_t i = 0; i < kAsyncSlots; ++i)
    if (st->slots[i].state == PROM_ASYNC_PHYSICAL_EMPTY) {
      slot_index = i;
      break;
    }
  if (slot_index == kAsyncSlots) {
    release_task(task);
    st->queue_full++;
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_ASYNC_QUEUE_FULL);
    return PROM_ERROR;
  }
  Slot& s = st->slots[slot_index];
  s.state = PROM_ASYNC_PHYSICAL_PREPARING;
  s.generation++;
  s.sequence = st->next_slot_sequence++;
  const size_t ab = (size_t)ac * 4, bb = (size_t)bc * 4, cb = (size_t)cc * 4;
  if (!ensure_slot_events(s) || !grow_device(&s.dev, &s.dev_bytes, align256(ab) + align256(bb) + align256(cb), cx.stream) ||
      !grow_pinned(&s.host_in, &s.host_in_bytes, align256(ab) + bb, cx.stream) ||
      !grow_pinned(&s.host_out, &s.host_out_bytes, cb, cx.stream)) {
    s.state = PROM_ASYNC_PHYSICAL_EMPTY;
    release_task(task);
    set_status(out_stage, out_detail_code, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_HIP_ALLOC_FAILED);
    return PROM_ERROR;
  }
  // The caller's inputs are captured now; the device work runs after return.
  host_memcpy(s.host_in, a, ab);
  host_memcpy(reinterpret_cast<char*>(s.host_in) + align256(ab), b, bb);
  char* dev = static_cast<char*>(s.dev);
  float* da = reinterpret_cast<float*>(dev);
  float* db = reinterpret_cast<float*>(dev + align256(ab));
  float* dc = reinterpret_cast<float*>(dev + align256(ab) + align256(bb));
  int path = 0;
  bool ok = hipMemcpyAsync(dev, s.host_in, align256(ab) + bb, hipMemcpyHostToDevice, cx.stream) == hipSuccess &&
            hipEventRecord(s.start, cx.stream) == hipSuccess &&
            launch_sgemm_f32(da, db, dc, m, n, k, cx.stream, &path) == hipSuccess &&
            hipEventRecord(s.kernel_end, cx.stream) == hipSuccess &&
            hipMemcpyAsync(s.host_out, dc, cb, hipMemcpyDeviceToHost, cx.stream) == hipSuccess &&
            hipEventRecord(s.done, cx.stream) == hipSuccess;
  if (!ok) {
    (void)hipGetLastError();
    (void)hipStreamSynchronize(cx.stream);
    s.state = PROM_ASYNC_PHYSICAL_EMPTY;
    release_task(task);
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_ERROR);
    return PROM_ERROR;
  }
  s.state = PROM_ASYNC_PHYSICAL_SUBMITTED;
  task->m = m;
  task->n = n;
  task->k = k;
  task->slot = slot_index;
  task->slot_generation = s.generation;
  task->sequence = st->next_task_sequence++;
  task->final_detail = path;
  task->lifecycle = PROM_ASYNC_STATE_SUBMITTED;
  uint32_t busy = 0;
  for (uint32_t i = 0; i < kAsyncSlots; ++i)
    if (st->slots[i].state != PROM_ASYNC_PHYSICAL_EMPTY) ++busy;
  if (busy > st->max_in_flight) st->max_in_flight = busy;
  rt->requests++;
  *out_task_id = task->public_id;
  set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, 0);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_query_async(void* handle, int task_id,
                                                                  PrometheusAsyncStatus* out_status) {
  if (out_status == nullptr) return PROM_ERROR;
  memset(out_status, 0, sizeof(*out_status));
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  std::lock_guard<std::mutex> lock(ctx().mu);
  AsyncState* st = rt->async;
  reap(st, false);
  Task* t = lookup_task(st, task_id);
  if (t == nullptr) {
    out_status->lifecycle_state = PROM_ASYNC_STATE_IDLE;
    out_status->detail_code = PROM_DETAIL_ASYNC_NO_TASK;
    if (st != nullptr) st->stale_rejects++;
    return PROM_ERROR;
  }
  poll_task(rt, st, t);
  out_status->lifecycle_state = t->lifecycle;
  out_status->stage = t->final_stage == 0u ? (uint32_t)PROM_STAGE_SUBMIT : t->final_stage;
  out_status->detail_code = t->lifecycle == PROM_ASYNC_STATE_SUBMITTED ? PROM_DETAIL_ASYNC_NOT_READY : t->final_detail;
  out_status->ready = t->lifecycle == PROM_ASYNC_STATE_READY;
  out_status->failed = t->lifecycle == PROM_ASYNC_STATE_FAILED;
  out_status->consumed = t->lifecycle == PROM_ASYNC_STATE_CONSUMED;
  out_status->outstanding_tasks = outstanding(st);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_async_diagnostics(void* handle,
                                                                         PrometheusSgemmAsyncDiagnostics* out_diag) {
  if (out_diag == nullptr) return PROM_ERROR;
  memset(out_diag, 0, sizeof(*out_diag));
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  std::lock_guard<std::mutex> lock(ctx().mu);
  AsyncState* st = rt->async;
  out_diag->task_capacity = kTaskCapacity;
  if (st == nullptr) return PROM_OK;
  reap(st, false);
  out_diag->queue_full_count = st->queue_full;
  out_diag->stale_id_rejection_count = st->stale_rejects;
  out_diag->max_in_flight = st->max_in_flight;
  out_diag->quarantine_event_count = st->quarantine_events;
  out_diag->reap_poll_count = st->reap_polls;
  out_diag->reap_success_count = st->reap_success;
  out_diag->reap_wait_count = st->reap_waits;
  out_diag->reap_failure_count = st->reap_failures;
  out_diag->max_quarantine_depth = st->max_quarantine_depth;
  for (uint32_t i = 0; i < kTaskCapacity; ++i) {
    const Task& t = st->tasks[i];
    if (!t.active) continue;
    PrometheusSgemmAsyncTaskDiagnostics& dst = out_diag->tasks[i];
    out_diag->active_task_count++;
    if (t.lifecycle == PROM_ASYNC_STATE_SUBMITTED) out_diag->submitted_count++;
    if (t.lifecycle == PROM_ASYNC_STATE_READY) out_diag->ready_count++;
    if (t.lifecycle == PROM_ASYNC_STATE_FAILED) out_diag->failed_count++;
    if (t.lifecycle == PROM_ASYNC_STATE_CONSUMED) out_diag->consumed_count++;
    if (t.abandoned) out_diag->abandoned_count++;
    if (t.quarantined) out_diag->quarantined_slot_count++;
    dst.task_id = t.public_id;
    dst.generation = t.generation;
    dst.lifecycle_state = t.lifecycle;
    dst.physical_slot_id = t.slot;
    dst.physical_slot_generation = t.slot_generation;
    dst.submission_sequence = t.sequence;
    dst.timing_valid = t.timing_valid;
    dst.gpu_duration_ns = t.gpu_ns;
    dst.failure_detail = t.final_detail;
    dst.failure_class = t.failure_class;
    dst.abandoned = t.abandoned;
    const Slot* s = t.slot < kAsyncSlots ? &st->slots[t.slot] : nullptr;
    dst.physical_slot_state = (s != nullptr && s->generation == t.slot_generation) ? s->state
                                                                                  : (uint32_t)PROM_ASYNC_PHYSICAL_EMPTY;
    dst.quarantined = t.quarantined;
    dst.physical_completion_confirmed = t.completion_confirmed;
    dst.reap_pending = t.reap_pending;
    dst.reap_completed = t.reap_completed;
  }
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_consume_async(void* handle, int task_id, float* c,
                                                                    uint32_t c_len, uint32_t* out_stage,
                                                                    int* out_detail_code) {
  set_status(out_stage, out_detail_code, PROM_STAGE_NONE, 0);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  std::lock_guard<std::mutex> lock(ctx().mu);
  AsyncState* st = rt->async;
  reap(st, false);
  Task* t = lookup_task(st, task_id);
  if (t == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_ASYNC_INVALID_TASK);
    return PROM_ERROR;
  }
  poll_task(rt, st, t);
  if (t->lifecycle == PROM_ASYNC_STATE_SUBMITTED) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_ASYNC_NOT_READY);
    return PROM_ERROR;
  }
  if (t->lifecycle == PROM_ASYNC_STATE_FAILED) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT,
               t->final_detail != 0 ? t->final_detail : PROM_DETAIL_ASYNC_FAILED);
    return PROM_ERROR;
  }
  if (t->lifecycle == PROM_ASYNC_STATE_CONSUMED) {
    set_status(out_stage, out_detail_code, PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_ASYNC_ALREADY_CONSUMED);
    return PROM_ERROR;
  }
  const uint64_t required = (uint64_t)t->m * t->n;
  if (c == nullptr || c_len < required) {
    set_status(out_stage, out_detail_code, PROM_STAGE_TRANSFER_OUT, PROM_ERROR);
    return PROM_ERROR;
  }
  Slot* s = task_slot(st, t);
  if (s == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_ASYNC_FAILED);
    return PROM_ERROR;
  }
  host_memcpy(c, s->host_out, (size_t)required * sizeof(float));
  t->lifecycle = PROM_ASYNC_STATE_CONSUMED;
  s->state = PROM_ASYNC_PHYSICAL_EMPTY;
  rt->successes++;
  set_status(out_stage, out_detail_code, PROM_STAGE_TRANSFER_OUT, t->final_detail);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_abandon_async(void* handle, int task_id) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  std::lock_guard<std::mutex> lock(ctx().mu);
  AsyncState* st = rt->async;
  reap(st, false);
  Task* t = lookup_task(st, task_id);
  if (t == nullptr) return PROM_ERROR;
  poll_task(rt, st, t);
  if (t->lifecycle == PROM_ASYNC_STATE_SUBMITTED) return PROM_ERROR;
  t->abandoned = 1;
  if (t->lifecycle == PROM_ASYNC_STATE_FAILED && t->reap_pending) {
    // Caller interest ends now; the record retires once its slot has drained.
    reap(st, false);
    return PROM_OK;
  }
  Slot* s = task_slot(st, t);
  if (s != nullptr) s->state = PROM_ASYNC_PHYSICAL_EMPTY;
  t->lifecycle = PROM_ASYNC_STATE_CONSUMED;
  release_task(t);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_batch(void* handle, const PrometheusSgemmBatchEntry* entries,
                                                            uint32_t entry_count, uint32_t flags, uint32_t* out_stage,
                                                            int* out_detail_code) {
  set_status(out_stage, out_detail_code, PROM_STAGE_NONE, 0);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  return batch_execute(rt, entries, entry_count, flags, false, out_stage, out_detail_code);
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_batch_m31_test(void* handle,
                                                                     const PrometheusSgemmBatchEntry* entries,
                                                                     uint32_t entry_count, uint32_t flags,
                                                                     uint32_t* out_stage, int* out_detail_code) {
  set_status(out_stage, out_detail_code, PROM_STAGE_NONE, 0);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  return batch_execute(rt, entries, entry_count, flags, true, out_stage, out_detail_code);
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_batch_diagnostics(void* handle,
                                                                        PrometheusSgemmBatchDiagnostics* out_diag) {
  if (out_diag == nullptr) return PROM_ERROR;
  memset(out_diag, 0, sizeof(*out_diag));
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  std::lock_guard<std::mutex> lock(ctx().mu);
  if (rt->async != nullptr) *out_diag = rt->async->batch;
  return PROM_OK;
}

}  // extern "C"
