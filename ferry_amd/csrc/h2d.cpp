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
#include <cstring>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/ferry_amd.h"
#include "pack_format.h"

namespace ferry {
void set_error(const char* fmt, ...);
void clear_error();
hipError_t h2d_copy_launch(const void* pool, void* cache, int64_t row_bytes, const int64_t* keys,
                           const int64_t* slots, int64_t n, hipStream_t stream);
hipError_t h2d_unpack_launch(const UnpackList& list, int64_t n, hipStream_t stream,
                             int64_t max_groups);
void pack_plan_rows(const uint16_t* pool, int64_t rows, int64_t n, int threads, PackPlan* plan);
int64_t plan_bytes(int64_t n, const PackPlan& plan);
void pack_write_rows(const uint16_t* pool, int64_t rows, int64_t n, int threads,
                     const PackPlan* plan, const int64_t* off, uint8_t* dst);
}  // namespace ferry

namespace {

// The engine's events order work of one device (copies after the reads of a slot, reads after
// its copies): none needs a system-scope fence, and leaving it out shortens every wait on them.
constexpr unsigned kEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;

// Engine events are recycled instead of created and destroyed per record (several per decode
// step): a HIP event that is destroyed while its record is still pending stays with the
// runtime until it fires, and a process's first few hundred decode steps ran about 3 % slower
// than later ones on freshly created events.  A released event goes back to a free list of its
// device and flags; re-recording it later does not disturb stream waits queued on its earlier
// record, and no engine state refers to it any more.
struct EventPool {
  std::mutex mu;
  struct Entry {
    int device;
    unsigned flags;
    hipEvent_t e;
  };
  std::vector<Entry> free;
};
constexpr size_t kEventPoolMax = 4096;

EventPool& event_pool() {
  static EventPool* pool = new EventPool();   // outlives every engine (never destroyed)
  return *pool;
}

hipError_t take_event(int device, unsigned flags, hipEvent_t* out) {
  {
    EventPool& p = event_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    for (size_t i = p.free.size(); i-- > 0;)
      if (p.free[i].device == device && p.free[i].flags == flags) {
        *out = p.free[i].e;
        p.free[i] = p.free.back();
        p.free.pop_back();
        return hipSuccess;
      }
  }
  return hipEventCreateWithFlags(out, flags);
}

void give_event(int device, unsigned flags, hipEvent_t e) {
  EventPool& p = event_pool();
  {
    std::lock_guard<std::mutex> lock(p.mu);
    if (p.free.size() < kEventPoolMax) {
      p.free.push_back({device, flags, e});
      return;
    }
  }
  (void)hipEventDestroy(e);
}

struct Event {
  hipEvent_t e = nullptr;
  hipStream_t stream = nullptr;   // the stream it was recorded on
  int64_t order = 0;              // record order among the engine's events
  int device = 0;
  unsigned flags = 0;
  // the slot reads it marks are known to be complete (ferry_h2d_wait_ready saw a kernel queued
  // after them write its ready words), though the event itself may not have fired yet
  bool reads_done = false;
  ~Event() {
    if (e) give_event(device, flags, e);
  }
};

// Of the events in `evs` (nulls allowed), those worth a wait: per stream only the newest, as a
// stream's events fire in record order; events that have fired already are dropped.  Returns
// false (error set) when a query fails.
bool pending_events(const std::vector<const std::shared_ptr<Event>*>& evs,
                    std::vector<hipEvent_t>* out) {
  std::vector<const Event*> newest;
  for (const std::shared_ptr<Event>* p : evs) {
    const Event* ev = p->get();
    if (!ev) continue;
    bool merged = false;
    for (const Event*& n : newest)
      if (n == ev || n->stream == ev->stream) {
        if (ev->order > n->order) n = ev;
        merged = true;
        break;
      }
    if (!merged) newest.push_back(ev);
  }
  for (const Event* ev : newest) {
    if (ev->reads_done) continue;
    const hipError_t q = hipEventQuery(ev->e);
    if (q == hipErrorNotReady) {
      (void)hipGetLastError();  // a pending event is not an error
      out->push_back(ev->e);
    } else if (q != hipSuccess) {
      ferry::set_error("hipEventQuery failed: %s", hipGetErrorString(q));
      return false;
    }
  }
  return true;
}

}  // namespace

constexpr int kLanes = 2;
// workgroups of a kernel-mode unpack launch (reads over the link): a few hundred workgroups
// keep far more reads in flight than the link's latency needs
constexpr int64_t kLinkUnpackGroups = 256;

// The packed copy of a pool (ferry_pack_pool): pinned host memory holding every row, packed or
// (when packing would not shrink it) raw, and per row its offset, size and form.  An engine
// fetches from it alone; the pool it was made from is no longer needed.
struct ferry_packed_pool {
  const char* pool = nullptr;         // the pool it was made from (for ferry_h2d_use_packed)
  int64_t rows = 0, row_bytes = 0;
  uint8_t* data = nullptr;
  const uint8_t* data_dev = nullptr;  // device mapping of data (null: DMA fetches only)
  std::vector<int64_t> off, size;
  std::vector<uint8_t> raw;           // per row: 1 when stored raw
  int64_t bytes = 0, packed_rows = 0, packed_bytes = 0, largest = 0;
};

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
  std::vector<int64_t> call_of;       // per slot: last packed DMA call that wrote it
  int64_t call = 0;
  // the last fetch call's groups of rows that become ready together (positions in the call,
  // each group's end, in call order): a packed DMA call's sub-batches, one group otherwise
  std::vector<int64_t> group_ends;
  // packed pool (ferry_h2d_use_packed): DMA copies move packed rows into device staging
  // buffers, and an unpack kernel writes the slots
  const ferry_packed_pool* packed = nullptr;
  uint8_t* ring = nullptr;            // device staging buffers, ring_rows x entry_bytes
  int64_t ring_rows = 0, entry_bytes = 0, ring_next = 0;
  std::vector<std::shared_ptr<Event>> ring_ev;  // per staging buffer: the unpack that read it
  hipStream_t unpack = nullptr;       // runs the unpacks; each waits for its rows' copies
  hipEvent_t lane_done[kLanes] = {};  // a lane's copies of one sub-batch
  int64_t cache_rows = 0, pool_rows = 0, row_bytes = 0;
  int64_t part[kLanes + 1] = {};      // byte boundaries of the row parts
  int32_t device = 0;
  hipStream_t stream[kLanes] = {};
  hipEvent_t join = nullptr;          // joins the lanes into the first stream
  std::vector<std::shared_ptr<Event>> copy_done[kLanes];  // per lane, per slot
  std::vector<int64_t> copy_seq;      // per slot: sequence number of its last copy, -1 if none
  std::vector<std::shared_ptr<Event>> used;  // per slot: last compute that read it
  std::shared_ptr<Event> marker;      // the latest event of ferry_h2d_mark_used_record
  // the last sub-batch of a packed call, unpacked later (ferry_h2d_set_defer_last): on the
  // stream of the first ferry_h2d_wait_stream that names one of its slots, else on the unpack
  // stream before anything else the engine does
  bool defer_last = false;
  struct {
    bool active = false;
    ferry::UnpackList ul;
    std::shared_ptr<Event> lane[kLanes];   // the lanes' copies of the sub-batch
    std::vector<int64_t> slots, entries;   // its slots and staging buffers
  } deferred;
  int64_t seq = 0;
  int64_t order = 0;                  // events recorded so far
  int64_t copies = 0;
};

#define H2D_HIP(expr)                                                                     \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess) {                                                               \
      ferry::set_error("%s failed: %s", #expr, hipGetErrorString(_e));                   \
      return 3;                                                                           \
    }                                                                                     \
  } while (0)

// a new engine event recorded on stream s
static hipError_t record_event(ferry_h2d* h, hipStream_t s, std::shared_ptr<Event>* out,
                               unsigned flags = kEventFlags) {
  auto ev = std::make_shared<Event>();
  hipError_t r = take_event(h->device, flags, &ev->e);
  if (r != hipSuccess) {
    ev->e = nullptr;
    return r;
  }
  ev->device = h->device;
  ev->flags = flags;
  r = hipEventRecord(ev->e, s);
  if (r != hipSuccess) return r;
  ev->stream = s;
  ev->order = ++h->order;
  *out = std::move(ev);
  return hipSuccess;
}

// Runs the deferred unpack (if any) on stream s, after the copies it reads; its slots and
// staging buffers are then ready at one event on s.
static int resolve_deferred(ferry_h2d* h, hipStream_t s) {
  auto& d = h->deferred;
  if (!d.active) return 0;
  d.active = false;
  std::vector<const std::shared_ptr<Event>*> evs;
  for (int l = 0; l < kLanes; ++l) evs.push_back(&d.lane[l]);
  std::vector<hipEvent_t> pending;
  if (!pending_events(evs, &pending)) return 3;
  for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent(s, e, 0));
  if (d.ul.n_rows > 0) H2D_HIP(ferry::h2d_unpack_launch(d.ul, h->row_bytes / 2, s, 0));
  std::shared_ptr<Event> ev;
  H2D_HIP(record_event(h, s, &ev));
  for (int64_t slot : d.slots)
    for (int l = 0; l < kLanes; ++l) h->copy_done[l][(size_t)slot] = ev;
  for (int64_t k : d.entries) h->ring_ev[(size_t)k] = ev;
  for (int l = 0; l < kLanes; ++l) d.lane[l].reset();
  return 0;
}

// the copy kernel addresses 16-byte units through 32-bit row indices; with a packed pool the
// unpack kernel reads the pool's device mapping instead (rows of a multiple of 32 values, each
// stored at a 256-byte multiple)
static bool kernel_copy_ok(const ferry_h2d* h) {
  if (h->packed)
    return h->packed->data_dev && (uintptr_t)h->packed->data_dev % 256 == 0 &&
           (uintptr_t)h->cache % 16 == 0;
  return h->pool_dev && h->row_bytes % 16 == 0 && (uintptr_t)h->pool_dev % 16 == 0 &&
         (uintptr_t)h->cache % 16 == 0 && h->pool_rows < (int64_t(1) << 31) &&
         h->cache_rows < (int64_t(1) << 31);
}

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
  H2D_HIP(hipEventCreateWithFlags(&h->join, kEventFlags));
  H2D_HIP(hipStreamCreateWithFlags(&h->unpack, hipStreamNonBlocking));
  for (int l = 0; l < kLanes; ++l)
    H2D_HIP(hipEventCreateWithFlags(&h->lane_done[l], kEventFlags));
  h->kernel_stream = h->stream[0];
  h->copy_seq.assign((size_t)cache_rows, -1);
  h->batch_of.assign((size_t)cache_rows, 0);
  h->call_of.assign((size_t)cache_rows, 0);
  h->used.assign((size_t)cache_rows, nullptr);
  *out = h.release();
  return 0;
}

extern "C" int ferry_h2d_destroy(ferry_h2d* h) {
  ferry::clear_error();
  if (!h) return 0;
  (void)resolve_deferred(h, h->unpack);
  for (int l = 0; l < kLanes; ++l)
    if (h->stream[l]) (void)hipStreamSynchronize(h->stream[l]);
  if (h->unpack) (void)hipStreamSynchronize(h->unpack);
  for (auto& kl : h->kernel_last) (void)hipEventSynchronize(kl.second->e);
  for (int l = 0; l < kLanes; ++l) h->copy_done[l].clear();
  h->ring_ev.clear();
  if (h->ring) (void)hipFree(h->ring);
  if (h->join) (void)hipEventDestroy(h->join);
  for (int l = 0; l < kLanes; ++l)
    if (h->lane_done[l]) (void)hipEventDestroy(h->lane_done[l]);
  if (h->unpack) (void)hipStreamDestroy(h->unpack);
  h->used.clear();
  for (int l = 0; l < kLanes; ++l)
    if (h->stream[l]) (void)hipStreamDestroy(h->stream[l]);
  delete h;
  return 0;
}

// Sub-batches of a packed fetch, counted from the call's end: the last holds about
// kSubBatchBytes, the one before it about twice that, and so on.  Only the last sub-batch's
// unpack follows the call's last copy (the others run while the lanes copy the rest), and a
// call of B bytes costs about log2(B / kSubBatchBytes) sets of launches and waits.
constexpr int64_t kSubBatchBytes = int64_t(4) << 20;

// floor(log2(remaining / kSubBatchBytes + 1)): a sub-batch closes where this drops
static int sub_batch_level(int64_t remaining) {
  int64_t q = remaining / kSubBatchBytes + 1;
  int level = 0;
  while (q > 1) {
    q >>= 1;
    ++level;
  }
  return level;
}

// DMA fetch on a packed pool.  The call's rows go in sub-batches (above; also at most
// kUnpackRows packed rows, at most one per staging buffer, no slot twice): the sub-batch's
// packed rows, concatenated, are cut into kLanes equal byte ranges that the lanes copy into
// staging buffers (rows that stayed raw go straight into their slots); the unpack stream waits
// for both lanes' copies of the sub-batch and runs one unpack launch that writes the slots, and
// every slot of the sub-batch is ready at the event after it.  The lanes never wait for the
// unpack stream (except to reuse a staging buffer that an unpack has yet to read, or when a
// sub-batch writes a slot that an earlier sub-batch of the call wrote), so each sub-batch's
// unpack runs while the lanes copy the next.
//
// A slot named twice in a call gets its rows in two sub-batches, and the later row must win,
// as with copies in stream order.  The two writes can be an unpack (unpack stream) and a raw
// row's lane copies (cut into per-lane byte ranges that differ between sub-batches), so before
// copying a sub-batch that rewrites a slot the lanes wait for the end of the previous
// sub-batch: its unpack ran after its own lane copies and, in stream order, after every earlier
// unpack of the call.
static int fetch_packed(ferry_h2d* h, const int64_t* slots, const int64_t* keys, int64_t n) {
  struct Seg {
    const char* src;
    char* dst;
    int64_t bytes;
  };
  const int64_t rb = h->row_bytes;
  const ferry_packed_pool* pp = h->packed;
  const int64_t per_batch = h->ring_rows < ferry::kUnpackRows ? h->ring_rows : ferry::kUnpackRows;
  int64_t remaining = 0;   // bytes of the call not yet in a sub-batch
  for (int64_t i = 0; i < n; ++i) remaining += pp->size[(size_t)keys[i]];
  ++h->call;
  std::shared_ptr<Event> prev;   // the end of the previous sub-batch of this call
  int64_t i0 = 0;
  while (i0 < n) {
    std::vector<Seg> segs;
    ferry::UnpackList ul;
    ul.n_rows = 0;
    std::vector<int64_t> entries;
    int64_t i1 = i0, total = 0;
    bool rewrites = false;   // writes a slot that an earlier sub-batch of the call wrote
    const int level = sub_batch_level(remaining);
    ++h->batch;   // a slot named twice starts a new sub-batch, so that the later row wins
    for (; i1 < n && (i1 == i0 || sub_batch_level(remaining - total) == level); ++i1) {
      const int64_t key = keys[i1];
      const size_t sl = (size_t)slots[i1];
      if (h->batch_of[sl] == h->batch) break;
      char* slot_ptr = h->cache + slots[i1] * rb;
      const char* src = (const char*)pp->data + pp->off[(size_t)key];
      if (pp->raw[(size_t)key]) {
        rewrites = rewrites || h->call_of[sl] == h->call;
        h->call_of[sl] = h->call;
        h->batch_of[sl] = h->batch;
        segs.push_back({src, slot_ptr, rb});
        total += rb;
        continue;
      }
      if (ul.n_rows == per_batch) break;
      rewrites = rewrites || h->call_of[sl] == h->call;
      h->call_of[sl] = h->call;
      h->batch_of[sl] = h->batch;
      const int64_t k = h->ring_next;
      h->ring_next = (k + 1) % h->ring_rows;
      char* st = (char*)h->ring + k * h->entry_bytes;
      segs.push_back({src, st, pp->size[(size_t)key]});
      total += pp->size[(size_t)key];
      ul.src[ul.n_rows] = (const uint8_t*)st;
      ul.dst[ul.n_rows] = (uint16_t*)slot_ptr;
      ul.raw[ul.n_rows] = 0;
      ++ul.n_rows;
      entries.push_back(k);
    }
    // a staging buffer is rewritten only after the unpack that last read it
    std::vector<hipEvent_t> waited;
    for (int64_t k : entries) {
      const auto& ev = h->ring_ev[(size_t)k];
      if (!ev) continue;
      bool dup = false;
      for (hipEvent_t x : waited) dup = dup || x == ev->e;
      if (dup) continue;
      waited.push_back(ev->e);
      const hipError_t q = hipEventQuery(ev->e);
      if (q == hipSuccess) continue;
      if (q != hipErrorNotReady) {
        ferry::set_error("hipEventQuery failed: %s", hipGetErrorString(q));
        return 3;
      }
      (void)hipGetLastError();
      for (int l = 0; l < kLanes; ++l) H2D_HIP(hipStreamWaitEvent(h->stream[l], ev->e, 0));
    }
    if (rewrites && prev)
      for (int l = 0; l < kLanes; ++l) H2D_HIP(hipStreamWaitEvent(h->stream[l], prev->e, 0));
    // each lane's byte range as copies; issued round-robin over the lanes, so that every lane
    // starts as early as the host can queue it
    std::vector<Seg> lane_segs[kLanes];
    for (int l = 0; l < kLanes; ++l) {
      const int64_t lo = l == 0 ? 0 : total * l / kLanes / 256 * 256;
      const int64_t hi = l + 1 == kLanes ? total : total * (l + 1) / kLanes / 256 * 256;
      int64_t at = 0;
      for (const Seg& sg : segs) {
        const int64_t a = lo > at ? lo : at;
        const int64_t b = hi < at + sg.bytes ? hi : at + sg.bytes;
        if (a < b) lane_segs[l].push_back({sg.src + (a - at), sg.dst + (a - at), b - a});
        at += sg.bytes;
      }
    }
    for (size_t j = 0;; ++j) {
      bool any = false;
      for (int l = 0; l < kLanes; ++l)
        if (j < lane_segs[l].size()) {
          const Seg& sg = lane_segs[l][j];
          H2D_HIP(hipMemcpyAsync(sg.dst, sg.src, (size_t)sg.bytes, hipMemcpyHostToDevice,
                                 h->stream[l]));
          any = true;
        }
      if (!any) break;
    }
    if (h->defer_last && i1 == n) {
      // the call's last sub-batch: its unpack waits for a stream that reads its slots
      auto& d = h->deferred;
      d.active = true;
      d.ul = ul;
      for (int l = 0; l < kLanes; ++l) H2D_HIP(record_event(h, h->stream[l], &d.lane[l]));
      d.slots.assign(slots + i0, slots + i1);
      d.entries = entries;
      for (int64_t i = i0; i < i1; ++i) {
        for (int l = 0; l < kLanes; ++l) h->copy_done[l][(size_t)slots[i]] = d.lane[l];
        h->copy_seq[(size_t)slots[i]] = h->seq++;
      }
      h->copies += i1 - i0;
      remaining -= total;
      h->group_ends.push_back(i1);
      i0 = i1;
      continue;
    }
    for (int l = 0; l < kLanes; ++l) {
      H2D_HIP(hipEventRecord(h->lane_done[l], h->stream[l]));
      H2D_HIP(hipStreamWaitEvent(h->unpack, h->lane_done[l], 0));
    }
    if (ul.n_rows > 0) H2D_HIP(ferry::h2d_unpack_launch(ul, rb / 2, h->unpack, 0));
    std::shared_ptr<Event> ev;
    H2D_HIP(record_event(h, h->unpack, &ev));
    for (int64_t i = i0; i < i1; ++i) {
      for (int l = 0; l < kLanes; ++l) h->copy_done[l][(size_t)slots[i]] = ev;
      h->copy_seq[(size_t)slots[i]] = h->seq++;
    }
    for (int64_t k : entries) h->ring_ev[(size_t)k] = ev;
    prev = ev;
    h->copies += i1 - i0;
    remaining -= total;
    h->group_ends.push_back(i1);
    i0 = i1;
  }
  return 0;
}

extern "C" int ferry_h2d_fetch(ferry_h2d* h, const int64_t* slots, const int64_t* keys,
                               int64_t n) {
  ferry::clear_error();
  h->group_ends.clear();
  if (n <= 0) return 0;
  if (resolve_deferred(h, h->unpack) != 0) return 3;
  // What a copy into a slot must follow: the last compute that read the slot (WAR) and any
  // earlier copy into it still in flight, on whichever lane or stream (WAW).  Events that have
  // fired when the call is made add no wait.
  std::vector<hipEvent_t> pending;
  std::vector<const std::shared_ptr<Event>*> evs;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t slot = slots[i], key = keys[i];
    if (slot < 0 || slot >= h->cache_rows || key < 0 || key >= h->pool_rows) {
      ferry::set_error("h2d_fetch: slot %lld / key %lld out of range", (long long)slot,
                       (long long)key);
      return 2;
    }
    evs.push_back(&h->used[(size_t)slot]);
    for (int l = 0; l < kLanes; ++l) evs.push_back(&h->copy_done[l][(size_t)slot]);
  }
  if (!pending_events(evs, &pending)) return 3;
  if (h->kind == FERRY_H2D_KERNEL) {
    hipStream_t s = h->kernel_stream;
    for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent(s, e, 0));
    // rows of one launch run concurrently: a slot named twice in the call starts a new
    // launch, so that the later row wins, as with copies in stream order
    if (h->packed) {
      // unpack launches that read the packed rows over the link and write the slots
      const ferry_packed_pool* pp = h->packed;
      ferry::UnpackList ul;
      ul.n_rows = 0;
      ++h->batch;
      for (int64_t i = 0; i <= n; ++i) {
        const bool flush = i == n || h->batch_of[(size_t)slots[i]] == h->batch ||
                           ul.n_rows == ferry::kUnpackRows;
        if (flush && ul.n_rows > 0) {
          H2D_HIP(ferry::h2d_unpack_launch(ul, h->row_bytes / 2, s, kLinkUnpackGroups));
          ul.n_rows = 0;
          ++h->batch;
        }
        if (i == n) break;
        const int64_t key = keys[i];
        h->batch_of[(size_t)slots[i]] = h->batch;
        ul.src[ul.n_rows] = pp->data_dev + pp->off[(size_t)key];
        ul.dst[ul.n_rows] = (uint16_t*)(h->cache + slots[i] * h->row_bytes);
        ul.raw[ul.n_rows] = pp->raw[(size_t)key];
        ++ul.n_rows;
      }
    } else {
      int64_t b0 = 0;
      ++h->batch;
      for (int64_t i = 0; i <= n; ++i) {
        if (i < n && h->batch_of[(size_t)slots[i]] != h->batch) {
          h->batch_of[(size_t)slots[i]] = h->batch;
          continue;
        }
        H2D_HIP(ferry::h2d_copy_launch(h->pool_dev, h->cache, h->row_bytes, keys + b0,
                                       slots + b0, i - b0, s));
        if (i < n) {
          ++h->batch;
          h->batch_of[(size_t)slots[i]] = h->batch;
        }
        b0 = i;
      }
    }
    std::shared_ptr<Event> ev;
    H2D_HIP(record_event(h, s, &ev));
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
    h->group_ends.push_back(n);
    return 0;
  }
  // No unconditional cross-lane wait: a lane waiting on an event that another DMA queue
  // records starts tens of microseconds late even when nothing is pending.
  for (int l = 0; l < kLanes; ++l)
    for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent(h->stream[l], e, 0));
  if (h->packed)   // the unpacks write the slots
    for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent(h->unpack, e, 0));
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
  if (h->packed) return fetch_packed(h, slots, keys, n);
  h->group_ends.push_back(n);
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
    std::shared_ptr<Event> ev;
    H2D_HIP(record_event(h, h->stream[l], &ev));
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
  if (resolve_deferred(h, h->unpack) != 0) return 3;
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
  // every still-running copy into the slots: per copy stream its newest such copy (copies into
  // different slots are not ordered with each other: DMA lanes, kernel-mode streams)
  // A deferred unpack of one of the slots runs on the waiting stream, after the waits for the
  // other slots' copies (those have fired or will fire first: the deferred sub-batch is the
  // last one copied), so that nothing stands between that unpack and the stream's next kernel.
  std::vector<const std::shared_ptr<Event>*> evs;
  bool resolve = false;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t slot = slots[i];
    if (slot < 0 || slot >= h->cache_rows) {
      ferry::set_error("h2d_wait_stream: slot %lld out of range", (long long)slot);
      return 2;
    }
    bool deferred = false;
    if (h->deferred.active)
      for (int64_t ds : h->deferred.slots) deferred = deferred || ds == slot;
    resolve = resolve || deferred;
    if (deferred || h->copy_seq[(size_t)slot] < 0) continue;
    for (int l = 0; l < kLanes; ++l) evs.push_back(&h->copy_done[l][(size_t)slot]);
  }
  std::vector<hipEvent_t> pending;
  if (!pending_events(evs, &pending)) return 3;
  for (hipEvent_t e : pending) H2D_HIP(hipStreamWaitEvent((hipStream_t)stream, e, 0));
  if (resolve && resolve_deferred(h, (hipStream_t)stream) != 0) return 3;
  return 0;
}

extern "C" int ferry_h2d_mark_used(ferry_h2d* h, const int64_t* slots, int64_t n, void* stream) {
  ferry::clear_error();
  if (n == 0) return 0;
  if (!h || !slots || n < 0) {
    ferry::set_error("h2d_mark_used: bad arguments");
    return 2;
  }
  for (int64_t i = 0; i < n; ++i)
    if (slots[i] < 0 || slots[i] >= h->cache_rows) {
      ferry::set_error("h2d_mark_used: slot %lld out of range", (long long)slots[i]);
      return 2;
    }
  std::shared_ptr<Event> ev;
  H2D_HIP(record_event(h, (hipStream_t)stream, &ev));
  for (int64_t i = 0; i < n; ++i) h->used[(size_t)slots[i]] = ev;
  return 0;
}

extern "C" int ferry_h2d_mark_used_record(ferry_h2d* h, const int64_t* slots, int64_t n,
                                          void* stream, void** event_out) {
  ferry::clear_error();
  if (!h || !event_out || n < 0 || (n > 0 && !slots)) {
    ferry::set_error("h2d_mark_used_record: bad arguments");
    return 2;
  }
  for (int64_t i = 0; i < n; ++i)
    if (slots[i] < 0 || slots[i] >= h->cache_rows) {
      ferry::set_error("h2d_mark_used_record: slot %lld out of range", (long long)slots[i]);
      return 2;
    }
  // a system-scope release, so that the host may read what the stream's kernels wrote to host
  // memory once the event has fired
  std::shared_ptr<Event> ev;
  H2D_HIP(record_event(h, (hipStream_t)stream, &ev, hipEventDisableTiming));
  for (int64_t i = 0; i < n; ++i) h->used[(size_t)slots[i]] = ev;
  h->marker = ev;
  *event_out = (void*)ev->e;
  return 0;
}

extern "C" int ferry_h2d_wait_ready(ferry_h2d* h, void* event, const int32_t* words, int64_t n,
                                    int32_t value) {
  ferry::clear_error();
  if (!h || !event || !words || n < 1 || !h->marker || (void*)h->marker->e != event) {
    ferry::set_error("h2d_wait_ready: bad arguments (event must be the latest "
                     "ferry_h2d_mark_used_record event)");
    return 2;
  }
  // Spin on the words (coherent host memory written by a kernel with a system-scope release);
  // every 1024 rounds the event is queried, so that a kernel that finished without writing them
  // is an error rather than an endless wait.
  auto all_set = [&]() {
    for (int64_t i = 0; i < n; ++i)
      if (__atomic_load_n(&words[i], __ATOMIC_ACQUIRE) != value) return false;
    return true;
  };
  for (uint64_t spin = 1;; ++spin) {
    if (all_set()) break;
    if ((spin & 1023) == 0) {
      const hipError_t q = hipEventQuery((hipEvent_t)event);
      if (q == hipSuccess) {
        if (all_set()) break;
        ferry::set_error("h2d_wait_ready: the stream passed the event but the ready words do not "
                         "hold %d", (int)value);
        return 3;
      }
      if (q != hipErrorNotReady) {
        ferry::set_error("hipEventQuery failed: %s", hipGetErrorString(q));
        return 3;
      }
      (void)hipGetLastError();   // a pending event is not an error
    }
  }
  // The kernel that wrote the words ran after every kernel queued before it on the event's
  // stream, so the slot reads the event marks are complete: later copies into those slots need
  // not wait for the event itself.
  h->marker->reads_done = true;
  return 0;
}

extern "C" int ferry_h2d_event_synchronize(ferry_h2d* h, void* event) {
  ferry::clear_error();
  if (!h || !event) {
    ferry::set_error("h2d_event_synchronize: bad arguments");
    return 2;
  }
  H2D_HIP(hipEventSynchronize((hipEvent_t)event));
  return 0;
}

extern "C" int ferry_h2d_synchronize(ferry_h2d* h) {
  ferry::clear_error();
  if (resolve_deferred(h, h->unpack) != 0) return 3;
  for (int l = 0; l < kLanes; ++l) H2D_HIP(hipStreamSynchronize(h->stream[l]));
  H2D_HIP(hipStreamSynchronize(h->unpack));
  for (auto& kl : h->kernel_last) H2D_HIP(hipEventSynchronize(kl.second->e));
  return 0;
}

extern "C" int ferry_h2d_reset(ferry_h2d* h) {
  ferry::clear_error();
  if (!h) {
    ferry::set_error("h2d_reset: null engine");
    return 2;
  }
  if (ferry_h2d_synchronize(h) != 0) return 3;
  // reads of the slots that callers' streams may still have in flight: the fetches after the
  // reset no longer know of them, so they end first
  std::vector<const Event*> reads;
  for (const auto& ev : h->used)
    if (ev && (reads.empty() || reads.back() != ev.get())) reads.push_back(ev.get());
  if (h->marker) reads.push_back(h->marker.get());
  for (size_t i = 0; i < reads.size(); ++i) {
    bool seen = false;
    for (size_t j = 0; j < i && !seen; ++j) seen = reads[j] == reads[i];
    if (!seen) H2D_HIP(hipEventSynchronize(reads[i]->e));
  }
  const size_t rows = (size_t)h->cache_rows;
  for (int l = 0; l < kLanes; ++l) h->copy_done[l].assign(rows, nullptr);
  h->copy_seq.assign(rows, -1);
  h->batch_of.assign(rows, 0);
  h->call_of.assign(rows, 0);
  h->call = 0;
  h->group_ends.clear();
  h->used.assign(rows, nullptr);
  h->ring_ev.assign(h->ring_ev.size(), nullptr);
  h->ring_next = 0;
  h->kernel_last.clear();
  h->marker.reset();
  h->kind = FERRY_H2D_DMA;
  h->kernel_stream = h->stream[0];
  h->defer_last = false;
  h->batch = 0;
  h->seq = 0;
  h->copies = 0;
  return 0;
}

extern "C" int64_t ferry_h2d_copies(const ferry_h2d* h) { return h ? h->copies : 0; }

extern "C" int64_t ferry_h2d_groups(const ferry_h2d* h, int64_t* ends, int64_t max_groups) {
  ferry::clear_error();
  if (!h || max_groups < 0 || (max_groups > 0 && !ends)) {
    ferry::set_error("h2d_groups: bad arguments");
    return -1;
  }
  const int64_t n = (int64_t)h->group_ends.size();
  for (int64_t i = 0; i < n && i < max_groups; ++i) ends[i] = h->group_ends[(size_t)i];
  return n;
}

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
  if (resolve_deferred(h, h->unpack) != 0) return 3;
  h->kind = kind;
  return 0;
}

extern "C" int ferry_h2d_set_defer_last(ferry_h2d* h, int32_t on) {
  ferry::clear_error();
  if (!h) {
    ferry::set_error("h2d_set_defer_last: null engine");
    return 2;
  }
  if (!on && resolve_deferred(h, h->unpack) != 0) return 3;
  h->defer_last = on != 0;
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

extern "C" int ferry_pack_pool(const void* pool, int64_t rows, int64_t row_bytes,
                               int32_t threads, ferry_packed_pool** out) {
  ferry::clear_error();
  if (!out || !pool || rows < 0 || row_bytes <= 0 || row_bytes % 64 != 0 ||
      row_bytes / 2 >= ((int64_t)1 << 32)) {
    ferry::set_error("pack_pool: needs rows of a multiple of 32 bf16 values (below 2^32)");
    return 2;
  }
  std::unique_ptr<ferry_packed_pool> pp(new ferry_packed_pool());
  pp->pool = (const char*)pool;
  pp->rows = rows;
  pp->row_bytes = row_bytes;
  const int64_t n = row_bytes / 2;
  std::vector<ferry::PackPlan> plan((size_t)rows);
  ferry::pack_plan_rows((const uint16_t*)pool, rows, n, threads, plan.data());
  pp->off.assign((size_t)rows, 0);
  pp->size.assign((size_t)rows, 0);
  pp->raw.assign((size_t)rows, 0);
  std::vector<int64_t> pack_off((size_t)rows, -1);   // rows to pack: their offset
  for (int64_t i = 0; i < rows; ++i) {
    int64_t b = ferry::plan_bytes(n, plan[(size_t)i]);
    if (b >= row_bytes) {   // no gain: the row is stored raw
      b = row_bytes;
      pp->raw[(size_t)i] = 1;
    } else {
      pack_off[(size_t)i] = pp->bytes;
      ++pp->packed_rows;
      pp->packed_bytes += b;
      pp->largest = b > pp->largest ? b : pp->largest;
    }
    pp->off[(size_t)i] = pp->bytes;
    pp->size[(size_t)i] = b;
    pp->bytes += b;
  }
  if (pp->bytes > 0) {
    void* mem = nullptr;
    H2D_HIP(hipHostMalloc(&mem, (size_t)pp->bytes, 0));
    pp->data = (uint8_t*)mem;
    void* dev = nullptr;
    if (hipHostGetDevicePointer(&dev, mem, 0) == hipSuccess)
      pp->data_dev = (const uint8_t*)dev;
    else
      (void)hipGetLastError();   // no device mapping: DMA fetches only
    ferry::pack_write_rows((const uint16_t*)pool, rows, n, threads, plan.data(), pack_off.data(),
                           pp->data);
    for (int64_t i = 0; i < rows; ++i)
      if (pp->raw[(size_t)i])
        std::memcpy(pp->data + pp->off[(size_t)i], (const char*)pool + i * row_bytes,
                    (size_t)row_bytes);
  }
  *out = pp.release();
  return 0;
}

extern "C" int ferry_packed_pool_stats(const ferry_packed_pool* pp, int64_t* packed_bytes,
                                       int64_t* packed_rows) {
  ferry::clear_error();
  if (!pp) {
    ferry::set_error("packed_pool_stats: null handle");
    return 2;
  }
  if (packed_bytes) *packed_bytes = pp->packed_bytes;
  if (packed_rows) *packed_rows = pp->packed_rows;
  return 0;
}

extern "C" int ferry_packed_pool_destroy(ferry_packed_pool* pp) {
  ferry::clear_error();
  if (!pp) return 0;
  if (pp->data) (void)hipHostFree(pp->data);
  delete pp;
  return 0;
}

static int ferry_h2d_use_packed_any(ferry_h2d* h, const ferry_packed_pool* pp,
                                    int64_t ring_rows);

extern "C" int ferry_h2d_use_packed(ferry_h2d* h, const ferry_packed_pool* pp,
                                    int64_t ring_rows) {
  ferry::clear_error();
  if (!h || !h->pool ||
      (pp && (pp->pool != h->pool || pp->rows != h->pool_rows || pp->row_bytes != h->row_bytes ||
              ring_rows < 1))) {
    ferry::set_error("h2d_use_packed: the packed pool was made from another pool, or no "
                     "staging buffer");
    return 2;
  }
  return ferry_h2d_use_packed_any(h, pp, ring_rows);
}

// attaches pp (null: detaches) to h, which fetches from it from now on
static int ferry_h2d_use_packed_any(ferry_h2d* h, const ferry_packed_pool* pp,
                                    int64_t ring_rows) {
  if (resolve_deferred(h, h->unpack) != 0) return 3;
  for (int l = 0; l < kLanes; ++l) H2D_HIP(hipStreamSynchronize(h->stream[l]));
  H2D_HIP(hipStreamSynchronize(h->unpack));
  h->ring_ev.clear();
  if (h->ring) {
    H2D_HIP(hipFree(h->ring));
    h->ring = nullptr;
  }
  h->packed = nullptr;
  h->ring_rows = h->entry_bytes = h->ring_next = 0;
  if (!pp) {
    if (h->kind == FERRY_H2D_KERNEL && !kernel_copy_ok(h)) h->kind = FERRY_H2D_DMA;
    return 0;
  }
  if (pp->packed_rows > 0) {
    void* rg = nullptr;
    H2D_HIP(hipMalloc(&rg, (size_t)(ring_rows * pp->largest)));
    h->ring = (uint8_t*)rg;
    h->ring_rows = ring_rows;
    h->entry_bytes = pp->largest;
    h->ring_ev.assign((size_t)ring_rows, nullptr);
  } else {
    h->ring_rows = 1;   // batches are never cut by the staging ring
  }
  h->packed = pp;
  if (h->kind == FERRY_H2D_KERNEL && !kernel_copy_ok(h)) h->kind = FERRY_H2D_DMA;
  return 0;
}

extern "C" int ferry_h2d_create_packed(void* cache, int64_t cache_rows,
                                       const ferry_packed_pool* pp, int32_t device,
                                       int64_t ring_rows, ferry_h2d** out) {
  ferry::clear_error();
  if (!out || !cache || !pp || cache_rows < 0 || ring_rows < 1) {
    ferry::set_error("h2d_create_packed: bad arguments");
    return 2;
  }
  H2D_HIP(hipSetDevice(device));
  std::unique_ptr<ferry_h2d> h(new ferry_h2d());
  h->cache = (char*)cache;
  h->pool = nullptr;   // every row comes from the packed pool
  h->cache_rows = cache_rows;
  h->pool_rows = pp->rows;
  h->row_bytes = pp->row_bytes;
  h->device = device;
  for (int l = 0; l <= kLanes; ++l) h->part[l] = h->row_bytes * l / kLanes / 256 * 256;
  h->part[kLanes] = h->row_bytes;
  for (int l = 0; l < kLanes; ++l) {
    H2D_HIP(hipStreamCreateWithFlags(&h->stream[l], hipStreamNonBlocking));
    h->copy_done[l].assign((size_t)cache_rows, nullptr);
  }
  H2D_HIP(hipEventCreateWithFlags(&h->join, kEventFlags));
  H2D_HIP(hipStreamCreateWithFlags(&h->unpack, hipStreamNonBlocking));
  for (int l = 0; l < kLanes; ++l)
    H2D_HIP(hipEventCreateWithFlags(&h->lane_done[l], kEventFlags));
  h->kernel_stream = h->stream[0];
  h->copy_seq.assign((size_t)cache_rows, -1);
  h->batch_of.assign((size_t)cache_rows, 0);
  h->call_of.assign((size_t)cache_rows, 0);
  h->used.assign((size_t)cache_rows, nullptr);
  ferry_h2d* raw = h.release();
  const int rc = ferry_h2d_use_packed_any(raw, pp, ring_rows);
  if (rc != 0) {
    ferry_h2d_destroy(raw);
    return rc;
  }
  *out = raw;
  return 0;
}

// With a packed pool attached, every sub-batch ends on the unpack stream (after both lanes'
// copies), so its queue ends with the call's last copy; otherwise the lanes join into stream[0].
extern "C" void* ferry_h2d_stream(ferry_h2d* h) {
  if (!h) return nullptr;
  return h->packed ? (void*)h->unpack : (void*)h->stream[0];
}
