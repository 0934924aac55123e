// H2D expert fetch engine: pinned host pool rows -> device cache slots on a dedicated stream.
//
// Reference: ferry/csrc/expert_ops.cpp:94-142 (H2DEngine).  The copies of a fetch call wait (on
// the copy streams, GPU-side) for the last compute that read any of the call's slots (the
// "used" events of mark_used) and for earlier copies into those slots that are still in
// flight; events that have already fired when the call is made add no wait.  After the call's copies every lane records one event, which becomes the copy-done
// event of each slot of the call.  Besides the reference's host wait (wait_host), wait_stream
// makes a compute stream wait for the copies on the GPU, so that experts that are already
// resident can run while missing ones are still in flight.
//
// Two ways to copy, chosen per engine (ferry_h2d_set_engine):
//  * FERRY_H2D_DMA (the default, the reference's scheme): hipMemcpyAsync on kLanes DMA streams.
//    One DMA stream does not fill the host link (measured on MI355X: ~47 GB/s with one stream,
//    ~56.5 GB/s with two).  The call's rows, concatenated, are cut into kLanes equal byte
//    ranges, which keeps the lanes balanced whatever the number of misses.  The lanes are
//    joined back into the first stream after their copies.  Per copy only the hipMemcpyAsync
//    itself is queued: a stream wait or an event between two copies on a DMA stream costs tens
//    of microseconds of idle link.
//  * FERRY_H2D_KERNEL (possible when the pool has a device mapping and rows are 16-byte
//    multiples): one launch of h2d_copy_kernel per fetch call, on the kernel stream
//    (ferry_h2d_set_kernel_stream; initially the first stream), reads the pool over PCIe and
//    writes the slots.  One launch leaves no idle link time between rows, but its host reads
//    slow the HBM-bound kernels that run beside it.
// A slot is ready when the copy-done events of all its lanes have fired (in kernel mode every
// lane's event is the launch's).  The engine owns its streams (default priority) and events; it
// allocates no device memory.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

#include "../../include/ferry_amd.h"

namespace ferry {
void set_error(const char* fmt, ...);
void clear_error();
hipError_t h2d_copy_launch(const void* pool, void* cache, int64_t row_bytes, const int64_t* keys,
                           const int64_t* slots, int64_t n, hipStream_t stream);
}  // namespace ferry

namespace {

struct Event {
  hipEvent_t e = nullptr;
  ~Event() {
    if (e) (void)hipEventDestroy(e);
  }
};

}  // namespace

constexpr int kLanes = 2;

struct ferry_h2d {
  char* cache = nullptr;
  const char* pool = nullptr;
  const char* pool_dev = nullptr;     // the pool's device mapping (null: DMA copies only)
  int32_t kind = FERRY_H2D_DMA;
  hipStream_t kernel_stream = nullptr;  // stream of kernel-mode copies (initially stream[0])
  // per stream that kernel-mode copies have used: the done event of its latest copy launch
  std::vector<std::pair<hipStream_t, std::shared_ptr<Event>>> kernel_last;
  std::vector<int64_t> batch_of;      // per slot: last batch of rows that wrote it (one call)
  int64_t batch = 0;
  int64_t cache_rows = 0, pool_rows = 0, row_bytes = 0;
  int64_t part[kLanes + 1] = {};      // byte boundaries of the row parts
  int32_t device = 0;
  hipStream_t stream[kLanes] = {};
  hipEvent_t join = nullptr;          // joins the lanes into the first stream
  std::vector<std::shared_ptr<Event>> copy_done[kLanes];  // per lane, per slot
  std::vector<int64_t> copy_seq;      // per slot: sequence number of its last copy, -1 if none
  std::vector<std::shared_ptr<Event>> used;  // per slot: last compute that read it
  int64_t seq = 0;
  int64_t copies = 0;
};

// the copy kernel addresses 16-byte units through 32-bit row indices
static bool kernel_copy_ok(const ferry_h2d* h) {
  return h->pool_dev && h->row_bytes % 16 == 0 && (uintptr_t)h->pool_dev % 16 == 0 &&
         (uintptr_t)h->cache % 16 == 0 && h->pool_rows < (int64_t(1) << 31) &&
         h->cache_rows < (int64_t(1) << 31);
}

#define H2D_HIP(expr)                                                                     \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess) {                                                               \
      ferry::set_error("%s failed: %s", #expr, hipGetErrorString(_e));                   \
      return 3;                                                                           \
    }                                                                                     \
  } while (0)

extern "C" int ferry_h2d_create(void* cache, int64_t cache_rows, const void* pool,
                                int64_t pool_rows, int64_t row_bytes, int32_t device,
                                ferry_h2d** out) {
  ferry::clear_error();
  if (!out || !cache || !pool || cache_rows < 0 || pool_rows < 0 || row_bytes <= 0) {
    ferry::set_error("h2d_create: bad arguments");
    return 2;
  }
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, pool) != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();
    ferry::set_error("h2d_create: the pool must be pinned host memory");
    return 2;
  }
  H2D_HIP(hipSetDevice(device));
  std::unique_ptr<ferry_h2d> h(new ferry_h2d());
  h->cache = (char*)cache;
  h->pool = (const char*)pool;
  h->cache_rows = cache_rows;
  h->pool_rows = pool_rows;
  h->row_bytes = row_bytes;
  h->device = device;
  h->pool_dev = (const char*)attr.devicePointer;
  for (int l = 0; l <= kLanes; ++l) h->part[l] = row_bytes * l / kLanes / 256 * 256;
  h->part[kLanes] = row_bytes;
  for (int l = 0; l < kLanes; ++l) {
    H2D_HIP(hipStreamCreateWithFlags(&h->stream[l], hipStreamNonBlocking));
    h->copy_done[l].assign((size_t)cache_rows, nullptr);
  }
  H2D_HIP(hipEventCreateWithFlags(&h->join, hipEventDisableTiming));
  h->kernel_stream = h->stream[0];
  h->copy_seq.assign((size_t)cache_rows, -1);
  h->batch_of.assign((size_t)cache_rows, 0);
  h->used.assign((size_t)cache_rows, nullptr);
  *out = h.release();
  return 0;
}

extern "C" int ferry_h2d_destroy(ferry_h2d* h) {
  ferry::clear_error();
  if (!h) return 0;
  for (int l = 0; l < kLanes; ++l)
    if (h->stream[l]) (void)hipStreamSynchronize(h->stream[l]);
  for (auto& kl : h->kernel_last) (void)hipEventSynchronize(kl.second->e);
  for (int l = 0; l < kLanes; ++l) h->copy_done[l].clear();
  if (h->join) (void)hipEventDestroy(h->join);
  h->used.clear();
  for (int l = 0; l < kLanes; ++l)
    if (h->stream[l]) (void)hipStreamDestroy(h->stream[l]);
  delete h;
  return 0;
}

extern "C" int ferry_h2d_fetch(ferry_h2d* h, const int64_t* slots, const int64_t* keys,
                               int64_t n) {
  ferry::clear_error();
  if (n <= 0) return 0;
  // What a copy into a slot must follow: the last compute that read the slot (WAR) and any
  // earlier copy into it still in flight, on whichever lane or stream (WAW).  Events that have
  // fired when the call is made add no wait.
  std::vector<hipEvent_t> pending, checked;
  auto note = [&](const std::shared_ptr<Event>& ev) -> bool {
    if (!ev) return true;
    for (hipEvent_t e : checked)
      if (e == ev->e) return true;
    checked.push_back(ev->e);
    const hipError_t q = hipEventQuery(ev->e);
    if (q == hipErrorNotReady) {
      (void)hipGetLastError();  // a pending event is not an error
      pending.push_back(ev->e);
    } else if (q != hipSuccess) {
      ferry::set_error("hipEventQuery failed: %s", hipGetErrorString(q));
      return false;
    }
    return true;
  };
  for (int64_t i = 0; i < n; ++i) {
    const int64_t slot = slots[i], key = keys[i];
    if (slot < 0 || slot >= h->cache_rows || key < 0 || key >= h->pool_rows) {
      ferry::set_error("h2d_fetch: slot %lld / key %lld out of range", (long long)slot,
                       (long long)key);
      return 2;
    }
    if (!note(h->used[(size_t)slot])) return 3;
    for (int l = 0; l < kLanes; ++l)
      if (!note(h->copy_done[l][(size_t)slot])) return 3;
  }
  if (h->kind == FERRY_H2D_KERNEL) {
    hipStream_t s = h->kernel_stream;
    for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent(s, e, 0));
    // rows of one launch run concurrently: a slot named twice in the call starts a new
    // launch, so that the later row wins, as with copies in stream order
    int64_t b0 = 0;
    ++h->batch;
    for (int64_t i = 0; i <= n; ++i) {
      if (i < n && h->batch_of[(size_t)slots[i]] != h->batch) {
        h->batch_of[(size_t)slots[i]] = h->batch;
        continue;
      }
      H2D_HIP(ferry::h2d_copy_launch(h->pool_dev, h->cache, h->row_bytes, keys + b0, slots + b0,
                                     i - b0, s));
      if (i < n) {
        ++h->batch;
        h->batch_of[(size_t)slots[i]] = h->batch;
      }
      b0 = i;
    }
    auto ev = std::make_shared<Event>();
    H2D_HIP(hipEventCreateWithFlags(&ev->e, hipEventDisableTiming));
    H2D_HIP(hipEventRecord(ev->e, s));
    for (int l = 0; l < kLanes; ++l)
      for (int64_t i = 0; i < n; ++i) h->copy_done[l][(size_t)slots[i]] = ev;
    bool known = false;
    for (auto& kl : h->kernel_last)
      if (kl.first == s) {
        kl.second = ev;
        known = true;
      }
    if (!known) h->kernel_last.emplace_back(s, ev);
    for (int64_t i = 0; i < n; ++i) h->copy_seq[(size_t)slots[i]] = h->seq++;
    h->copies += n;
    return 0;
  }
  // No unconditional cross-lane wait: a lane waiting on an event that another DMA queue
  // records starts tens of microseconds late even when nothing is pending.
  for (int l = 0; l < kLanes; ++l)
    for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent(h->stream[l], e, 0));
  // The call's rows, concatenated, are cut into kLanes equal byte ranges, one per lane: a lane
  // copies about n / kLanes whole rows plus a part of the row its range ends in.  A call that
  // names a slot twice splits every row instead, whose in-lane order makes the later row win.
  bool repeated = false;
  ++h->batch;
  for (int64_t i = 0; i < n && !repeated; ++i) {
    repeated = h->batch_of[(size_t)slots[i]] == h->batch;
    h->batch_of[(size_t)slots[i]] = h->batch;
  }
  const int64_t rb = h->row_bytes;
  if (!repeated) {
    const int64_t total = n * rb;
    for (int l = 0; l < kLanes; ++l) {
      const int64_t lo = l == 0 ? 0 : total * l / kLanes / 256 * 256;
      const int64_t hi = l + 1 == kLanes ? total : total * (l + 1) / kLanes / 256 * 256;
      for (int64_t b = lo; b < hi;) {
        const int64_t i = b / rb, off = b - i * rb;
        const int64_t nb = (hi - b < rb - off) ? hi - b : rb - off;
        H2D_HIP(hipMemcpyAsync(h->cache + slots[i] * rb + off, h->pool + keys[i] * rb + off,
                               (size_t)nb, hipMemcpyHostToDevice, h->stream[l]));
        b += nb;
      }
    }
  } else {
    for (int64_t i = 0; i < n; ++i) {
      for (int l = 0; l < kLanes; ++l) {
        const int64_t b0 = h->part[l], nb = h->part[l + 1] - b0;
        if (nb > 0)
          H2D_HIP(hipMemcpyAsync(h->cache + slots[i] * rb + b0, h->pool + keys[i] * rb + b0,
                                 (size_t)nb, hipMemcpyHostToDevice, h->stream[l]));
      }
    }
  }
  for (int l = 0; l < kLanes; ++l) {
    auto ev = std::make_shared<Event>();
    H2D_HIP(hipEventCreateWithFlags(&ev->e, hipEventDisableTiming));
    H2D_HIP(hipEventRecord(ev->e, h->stream[l]));
    for (int64_t i = 0; i < n; ++i) h->copy_done[l][(size_t)slots[i]] = ev;
  }
  for (int64_t i = 0; i < n; ++i) h->copy_seq[(size_t)slots[i]] = h->seq++;
  h->copies += n;
  for (int l = 1; l < kLanes; ++l) {
    H2D_HIP(hipEventRecord(h->join, h->stream[l]));
    H2D_HIP(hipStreamWaitEvent(h->stream[0], h->join, 0));
  }
  return 0;
}

extern "C" int ferry_h2d_wait_host(ferry_h2d* h, const int64_t* slots, int64_t n) {
  ferry::clear_error();
  for (int64_t i = 0; i < n; ++i) {
    const int64_t slot = slots[i];
    if (slot < 0 || slot >= h->cache_rows) {
      ferry::set_error("h2d_wait_host: slot %lld out of range", (long long)slot);
      return 2;
    }
    if (h->copy_seq[(size_t)slot] >= 0)
      for (int l = 0; l < kLanes; ++l)
        H2D_HIP(hipEventSynchronize(h->copy_done[l][(size_t)slot]->e));
  }
  return 0;
}

extern "C" int ferry_h2d_wait_stream(ferry_h2d* h, const int64_t* slots, int64_t n,
                                     void* stream) {
  ferry::clear_error();
  // every still-running copy into the slots, each event once (copies into different slots
  // are not ordered with each other: DMA lanes, kernel-mode streams)
  std::vector<hipEvent_t> seen;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t slot = slots[i];
    if (slot < 0 || slot >= h->cache_rows) {
      ferry::set_error("h2d_wait_stream: slot %lld out of range", (long long)slot);
      return 2;
    }
    if (h->copy_seq[(size_t)slot] < 0) continue;
    for (int l = 0; l < kLanes; ++l) {
      const hipEvent_t e = h->copy_done[l][(size_t)slot]->e;
      bool dup = false;
      for (hipEvent_t x : seen) dup = dup || x == e;
      if (dup) continue;
      seen.push_back(e);
      const hipError_t q = hipEventQuery(e);
      if (q == hipSuccess) continue;
      if (q != hipErrorNotReady) {
        ferry::set_error("hipEventQuery failed: %s", hipGetErrorString(q));
        return 3;
      }
      (void)hipGetLastError();
      H2D_HIP(hipStreamWaitEvent((hipStream_t)stream, e, 0));
    }
  }
  return 0;
}

extern "C" int ferry_h2d_mark_used(ferry_h2d* h, const int64_t* slots, int64_t n, void* stream) {
  ferry::clear_error();
  if (n == 0) return 0;
  auto ev = std::make_shared<Event>();
  H2D_HIP(hipEventCreateWithFlags(&ev->e, hipEventDisableTiming));
  H2D_HIP(hipEventRecord(ev->e, (hipStream_t)stream));
  for (int64_t i = 0; i < n; ++i) {
    const int64_t slot = slots[i];
    if (slot < 0 || slot >= h->cache_rows) {
      ferry::set_error("h2d_mark_used: slot %lld out of range", (long long)slot);
      return 2;
    }
    h->used[(size_t)slot] = ev;
  }
  return 0;
}

extern "C" int ferry_h2d_synchronize(ferry_h2d* h) {
  ferry::clear_error();
  for (int l = 0; l < kLanes; ++l) H2D_HIP(hipStreamSynchronize(h->stream[l]));
  for (auto& kl : h->kernel_last) H2D_HIP(hipEventSynchronize(kl.second->e));
  return 0;
}

extern "C" int64_t ferry_h2d_copies(const ferry_h2d* h) { return h ? h->copies : 0; }

extern "C" int ferry_h2d_set_engine(ferry_h2d* h, int32_t kind) {
  ferry::clear_error();
  if (!h || (kind != FERRY_H2D_DMA && kind != FERRY_H2D_KERNEL)) {
    ferry::set_error("h2d_set_engine: bad arguments");
    return 2;
  }
  if (kind == FERRY_H2D_KERNEL && !kernel_copy_ok(h)) {
    ferry::set_error("h2d_set_engine: the copy kernel needs a device-mapped pool and 16-byte "
                     "aligned rows");
    return 2;
  }
  // no wait: every fetch follows the earlier copies into its slots, of either kind
  h->kind = kind;
  return 0;
}

extern "C" int ferry_h2d_set_kernel_stream(ferry_h2d* h, void* stream) {
  ferry::clear_error();
  if (!h) {
    ferry::set_error("h2d_set_kernel_stream: null engine");
    return 2;
  }
  h->kernel_stream = (hipStream_t)stream;
  return 0;
}

extern "C" int32_t ferry_h2d_engine(const ferry_h2d* h) { return h ? h->kind : -1; }

extern "C" void* ferry_h2d_stream(ferry_h2d* h) { return h ? (void*)h->stream[0] : nullptr; }
