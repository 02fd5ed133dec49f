// Turbo window engine: blocks rotate through a fixed window of device slots.
//
// Behaviour follows the reference's Rust TransferEngine (turbo_src/engine.rs):
// registration of per-parameter byte sizes (82-99), initialisation that pins
// host memory for every block and creates `window` empty slots (102-156),
// staging by host copy (159-175), a free-slot list (178-199), the
// forward/backward step that evicts the previous block and prefetches the next
// (304-341), and the location state machine cpu → h2d → gpu → d2h → cpu.
//
// What is different, on purpose:
//  * one pinned region per block with 256-byte aligned parameter offsets; a
//    slot given as one contiguous buffer receives a block in ONE copy;
//  * one H2D event per block instead of a single shared prefetch event, so
//    the compute stream waits exactly for the block it needs, on the device
//    (hipStreamWaitEvent), and the host never blocks in step();
//  * an eviction records a fence on its slot; a prefetch that reuses the slot
//    makes the prefetch stream wait for that fence instead of the host
//    draining the eviction stream first;
//  * write-back can be switched off per block (frozen weights are not copied
//    back to host memory on every eviction);
//  * a write-back copies only the chunks the block changed on the device: its H2D
//    is followed by chunk digests of the slot (on the prefetch stream), and the
//    write-back compares them (on the evict stream) and copies the changed runs
//    (sh_saveback_submit_chunks); the host region then holds the slot's bytes, as
//    after the reference's full copy (sh_turbo_set_writeback_chunks; SDMA only);
//  * write-back copies run on an SDMA engine (sh_saveback), not as
//    hipMemcpyAsync on the evict stream: HIP runs a pinned device-to-host copy
//    as a kernel on the compute units, and the compute kernels beside it run
//    many times slower. A prefetch that reuses the slot of a block being
//    written back, or reloads that block, then waits for the copy on the host
//    (an SDMA copy has no device-side wait). Tickets complete in order, so
//    the engine tracks the highest one known complete and releases the rest;
//  * step()'s lookahead prefetch does not make that host wait: a copy that
//    would wait is deferred to the next engine call (the block is marked h2d
//    with its slot taken, as the reference's step leaves it). The caller
//    queues the current block's compute first, and the write-back of that
//    block can start as soon as the one before it ends. In a forward-only
//    pass the last block keeps its slot, so a window of 3 rotates through 2
//    slots, and waiting in step() would hold every block's compute behind
//    the previous block's write-back.
#include <algorithm>
#include <deque>
#include <mutex>
#include <vector>

#include "sh_internal.h"

namespace {

constexpr uint64_t kParamAlign = 256;

uint64_t align_up(uint64_t x) { return (x + kParamAlign - 1) / kParamAlign * kParamAlign; }

struct Block {
  std::vector<uint64_t> sizes;
  std::vector<uint64_t> offsets;  // in the pinned region and in a contiguous slot
  uint64_t extent = 0;            // aligned bytes of the whole block
  uint8_t* host = nullptr;
  int location = SH_TURBO_CPU;
  int slot = -1;
  bool writeback = true;
  hipEvent_t h2d = nullptr;  // recorded after the block's H2D on the prefetch stream
  hipEvent_t d2h = nullptr;  // recorded after the block's eviction on the evict stream
  uint64_t d2h_ticket = 0;   // its write-back on the save-back engine (0: none pending)
  hipEvent_t t_start = nullptr, t_end = nullptr;  // timing events around the last H2D (timing mode)
  bool timed = false;
  uint64_t* digests = nullptr;  // device: chunk digests of the block's copy runs after its last H2D
  uint8_t* changed = nullptr;   // pinned: one byte per chunk, the write-back's comparison
  bool digested = false;        // the digests describe this residency's slot bytes
};

// A queued write-back ticket and, in timing mode, the span that records its copy times.
struct Pending {
  uint64_t ticket;
  int64_t span;  // index into sh_turbo::spans, -1: none
  bool chunked;  // a write-back of changed chunks: its bytes are known once it completes
};

struct Slot {
  std::vector<void*> ptrs;      // per-parameter mode (reference layout)
  std::vector<uint64_t> sizes;  // per-position capacity in per-parameter mode
  void* base = nullptr;         // contiguous mode
  uint64_t bytes = 0;
  int assigned = -1;
  hipEvent_t fence = nullptr;   // the last eviction out of this slot
  bool fenced = false;
  uint64_t fence_ticket = 0;    // that eviction's write-back on the save-back engine (0: none)
};

}  // namespace

struct sh_turbo {
  sh::Live<sh::kLiveTurbo> live;
  std::mutex mu;
  std::vector<Block> blocks;
  std::vector<Slot> slots;
  std::vector<int> free_slots;  // oldest release first
  hipStream_t prefetch = nullptr;
  hipStream_t evict = nullptr;
  hipEvent_t compute_mark = nullptr;
  sh_saveback* sb = nullptr;      // write-backs on an SDMA engine (null: on the evict stream)
  bool sdma = true;               // sh_turbo_set_save_back
  std::deque<Pending> tickets;    // write-back tickets not yet released, in order
  int64_t deferred = -1;          // a lookahead block marked h2d whose copy is not issued yet
  bool deferred_from_d2h = false; // ... and that was being written back itself
  uint64_t done_upto = 0;         // every ticket <= this one is complete (and released)
  int device = 0;
  bool initialized = false;
  bool timing = false;
  std::vector<sh_turbo_span> spans;  // write-backs and host waits recorded in timing mode
  uint64_t bytes_h2d = 0, bytes_d2h = 0;
  uint32_t chunk = 1u << 18;  // write-backs of changed chunks of this size (0: every byte)
};

namespace {

int check_block(sh_turbo* t, uint32_t b) {
  if (b >= t->blocks.size())
    return sh::fail(SH_ERR_STATE, "block %u out of range (%zu blocks)", b, t->blocks.size());
  return SH_OK;
}

int require_init(sh_turbo* t) {
  if (!t->initialized) return sh::fail(SH_ERR_STATE, "turbo engine is not initialized");
  return SH_OK;
}

// Device address of param p of block b inside slot s.
void* slot_param_ptr(const Slot& s, const Block& b, size_t p) {
  if (s.base) return static_cast<uint8_t*>(s.base) + b.offsets[p];
  return p < s.ptrs.size() ? s.ptrs[p] : nullptr;
}

int check_slot_fits(const Slot& s, const Block& b, uint32_t slot_index) {
  if (s.base) {
    if (b.extent > s.bytes)
      return sh::fail(SH_ERR_STATE, "slot %u holds %llu bytes, block needs %llu", slot_index,
                      (unsigned long long)s.bytes, (unsigned long long)b.extent);
    return SH_OK;
  }
  for (size_t p = 0; p < b.sizes.size(); ++p) {
    if (b.sizes[p] == 0) continue;
    if (p >= s.ptrs.size() || s.ptrs[p] == nullptr)
      return sh::fail(SH_ERR_STATE, "slot %u has no device pointer for param %zu", slot_index, p);
    if (b.sizes[p] > s.sizes[p])
      return sh::fail(SH_ERR_STATE, "slot %u param %zu holds %llu bytes, needs %llu", slot_index, p,
                      (unsigned long long)s.sizes[p], (unsigned long long)b.sizes[p]);
  }
  return SH_OK;
}

// Copies between a block's pinned region and its slot: one copy for a
// contiguous slot, else one per parameter (contiguous runs merged).
int copy_block(sh_turbo* t, const Block& b, const Slot& s, bool to_device, hipStream_t stream) {
  if (s.base) {
    if (b.extent == 0) return SH_OK;
    if (to_device)
      SH_HIP(hipMemcpyAsync(s.base, b.host, b.extent, hipMemcpyHostToDevice, stream));
    else
      SH_HIP(hipMemcpyAsync(b.host, s.base, b.extent, hipMemcpyDeviceToHost, stream));
    (to_device ? t->bytes_h2d : t->bytes_d2h) += b.extent;
    return SH_OK;
  }
  size_t p = 0, n = b.sizes.size();
  while (p < n) {
    if (b.sizes[p] == 0) { ++p; continue; }
    uint8_t* dev = static_cast<uint8_t*>(s.ptrs[p]);
    uint8_t* host = b.host + b.offsets[p];
    uint64_t len = b.sizes[p];
    size_t q = p + 1;
    while (q < n && b.sizes[q] != 0 && static_cast<uint8_t*>(s.ptrs[q]) == dev + len &&
           b.host + b.offsets[q] == host + len) {
      len += b.sizes[q];
      ++q;
    }
    if (to_device)
      SH_HIP(hipMemcpyAsync(dev, host, len, hipMemcpyHostToDevice, stream));
    else
      SH_HIP(hipMemcpyAsync(host, dev, len, hipMemcpyDeviceToHost, stream));
    (to_device ? t->bytes_h2d : t->bytes_d2h) += len;
    p = q;
  }
  return SH_OK;
}

// Releases the write-back tickets that have completed (they complete in order).
int reap_tickets(sh_turbo* t) {
  while (!t->tickets.empty()) {
    const uint64_t tk = t->tickets.front().ticket;
    const int64_t span = t->tickets.front().span;
    int st = sh_saveback_query(t->sb, tk);
    if (st == SH_ERR_NOT_READY) break;
    if (st != SH_OK) return st;
    if (t->tickets.front().chunked) {
      uint64_t bytes = 0;
      st = sh_saveback_ticket_bytes(t->sb, tk, &bytes);
      if (st != SH_OK) return st;
      t->bytes_d2h += bytes;
      if (span >= 0) t->spans[(size_t)span].bytes = bytes;
    }
    if (span >= 0) {
      // the copy engine's own start and end; none when a tool replaced the copies' signals
      uint64_t times[2] = {0, 0};
      if (sh_saveback_ticket_times(t->sb, tk, times) == SH_OK) {
        t->spans[(size_t)span].start_ns = times[0];
        t->spans[(size_t)span].end_ns = times[1];
      }
      sh::clear_error();
    }
    t->done_upto = tk;
    t->tickets.pop_front();
    st = sh_saveback_release(t->sb, tk);
    if (st != SH_OK) return st;
  }
  return SH_OK;
}

bool ticket_done(sh_turbo* t, uint64_t tk) {
  if (tk == 0 || tk <= t->done_upto) return true;
  if (reap_tickets(t) != SH_OK) return false;  // the failure surfaces in the next wait
  return tk <= t->done_upto;
}

// Host wait for a write-back ticket (and every earlier one), then releases them.
// In timing mode a wait for block b is recorded as a host-wait span.
int wait_ticket(sh_turbo* t, uint64_t tk, int64_t b = -1) {
  if (tk == 0 || tk <= t->done_upto) return SH_OK;
  uint64_t t0 = 0;
  if (t->timing && b >= 0 && sh_saveback_clock_ns(&t0) != SH_OK) t0 = 0;
  int st = sh_saveback_wait(t->sb, tk);
  if (st != SH_OK) return st;
  if (t0 != 0) {
    uint64_t t1 = 0;
    if (sh_saveback_clock_ns(&t1) == SH_OK)
      t->spans.push_back({(uint32_t)b, SH_TURBO_SPAN_HOST_WAIT, t0, t1, 0});
  }
  return reap_tickets(t);
}

// The copy runs of block b in slot s as (host, device, bytes): one for a contiguous slot, else
// one per run of parameters contiguous on both sides (the runs copy_block copies).
std::vector<sh_copy_item> block_runs(const Block& b, const Slot& s) {
  std::vector<sh_copy_item> items;
  if (s.base) {
    if (b.extent) items.push_back({b.host, s.base, b.extent});
    return items;
  }
  size_t p = 0, n = b.sizes.size();
  while (p < n) {
    if (b.sizes[p] == 0) { ++p; continue; }
    uint8_t* dev = static_cast<uint8_t*>(s.ptrs[p]);
    uint8_t* host = b.host + b.offsets[p];
    uint64_t len = b.sizes[p];
    size_t q = p + 1;
    while (q < n && b.sizes[q] != 0 && static_cast<uint8_t*>(s.ptrs[q]) == dev + len &&
           b.host + b.offsets[q] == host + len) {
      len += b.sizes[q];
      ++q;
    }
    items.push_back({host, dev, len});
    p = q;
  }
  return items;
}

// The write-back copies of block b out of slot s (every byte).
std::vector<sh_copy_item> writeback_items(sh_turbo* t, const Block& b, const Slot& s) {
  std::vector<sh_copy_item> items = block_runs(b, s);
  for (const sh_copy_item& it : items) t->bytes_d2h += it.bytes;
  return items;
}

uint64_t chunks_of(uint64_t bytes, uint32_t chunk) { return bytes / chunk + (bytes % chunk != 0 ? 1 : 0); }

// Chunks the digest buffers of block b need for any slot: every run is a merge of parameters,
// each at most its aligned size.
uint64_t chunk_capacity(const Block& b, uint32_t chunk) {
  uint64_t n = 0;
  for (uint64_t sz : b.sizes) n += chunks_of(align_up(sz), chunk);
  return n;
}

// Takes the chunk digests of block b's runs in slot s on the prefetch stream, after its H2D.
int digest_block(sh_turbo* t, Block& b, const Slot& s) {
  uint64_t first = 0;
  for (const sh_copy_item& r : block_runs(b, s)) {
    int rc = sh::launch_block_digest(r.src, r.bytes, t->chunk, b.digests + 2 * first, t->prefetch);
    if (rc != SH_OK) return rc;
    first += chunks_of(r.bytes, t->chunk);
  }
  b.digested = true;
  return SH_OK;
}

// A free slot for block b: one whose fence has passed if any, else the one
// released first (the prefetch stream then waits for its fence on the device).
int take_slot(sh_turbo* t, uint32_t b, int* out) {
  Block& blk = t->blocks[b];
  if (blk.slot >= 0) { *out = blk.slot; return SH_OK; }
  if (t->free_slots.empty())
    return sh::fail(SH_ERR_STATE, "No free GPU slots — increase window_size or evict a block");
  size_t pick = 0;
  for (size_t i = 0; i < t->free_slots.size(); ++i) {
    Slot& s = t->slots[t->free_slots[i]];
    if ((!s.fenced || hipEventQuery(s.fence) == hipSuccess) && ticket_done(t, s.fence_ticket)) { pick = i; break; }
  }
  int si = t->free_slots[pick];
  int rc = check_slot_fits(t->slots[si], blk, (uint32_t)si);
  if (rc != SH_OK) return rc;
  t->free_slots.erase(t->free_slots.begin() + (long)pick);
  t->slots[si].assigned = (int)b;
  blk.slot = si;
  *out = si;
  return SH_OK;
}

// Issues the H2D of block b into its assigned slot on the prefetch stream.
int issue_prefetch(sh_turbo* t, uint32_t b, bool from_d2h) {
  Block& blk = t->blocks[b];
  Slot& s = t->slots[blk.slot];
  int rc = SH_OK;
  // the pinned region may still be the target of this block's write-back
  if (from_d2h) {
    SH_HIP(hipStreamWaitEvent(t->prefetch, blk.d2h, 0));
    rc = wait_ticket(t, blk.d2h_ticket, b);
    if (rc != SH_OK) return rc;
    blk.d2h_ticket = 0;
  }
  if (s.fenced) {
    SH_HIP(hipStreamWaitEvent(t->prefetch, s.fence, 0));
    s.fenced = false;
  }
  // the slot may still be the source of the previous block's write-back
  rc = wait_ticket(t, s.fence_ticket, b);
  if (rc != SH_OK) return rc;
  s.fence_ticket = 0;
  if (t->timing) SH_HIP(hipEventRecord(blk.t_start, t->prefetch));
  rc = copy_block(t, blk, s, true, t->prefetch);
  if (rc != SH_OK) return rc;
  blk.digested = false;
  if (blk.digests != nullptr && blk.writeback) {
    rc = digest_block(t, blk, s);
    if (rc != SH_OK) return rc;
  }
  if (t->timing) {
    SH_HIP(hipEventRecord(blk.t_end, t->prefetch));
    blk.timed = true;
  }
  SH_HIP(hipEventRecord(blk.h2d, t->prefetch));
  blk.location = SH_TURBO_H2D;
  return SH_OK;
}

// After a failed issue_prefetch: block b goes back to where it was (its pinned region, or still
// being written back to it) and its slot back to the free list, so no later step or wait takes
// the slot's stale bytes, or a never-recorded H2D event, for the block's.
void undo_prefetch(sh_turbo* t, uint32_t b, bool from_d2h) {
  Block& blk = t->blocks[b];
  if (blk.slot >= 0) {
    t->slots[blk.slot].assigned = -1;
    t->free_slots.insert(t->free_slots.begin(), blk.slot);
  }
  blk.slot = -1;
  blk.location = from_d2h ? SH_TURBO_D2H : SH_TURBO_CPU;  // D2H until its event and ticket are done
}

// Issues a deferred lookahead copy (waiting on the host for the write-back it follows).
int flush_deferred(sh_turbo* t) {
  if (t->deferred < 0) return SH_OK;
  const uint32_t b = (uint32_t)t->deferred;
  const bool from_d2h = t->deferred_from_d2h;
  t->deferred = -1;
  const int rc = issue_prefetch(t, b, from_d2h);
  if (rc != SH_OK) undo_prefetch(t, b, from_d2h);
  return rc;
}

// Starts the H2D of block b into a free slot. With may_defer, a copy that would
// first wait on the host for a write-back out of the slot (or out of the block's
// own pinned region) is not issued yet: the block is marked h2d with its slot
// assigned, and the next engine call issues it. Within step() that lets the
// caller queue the current block's compute before the host blocks, so the
// write-back engine is not left waiting for that compute.
int async_prefetch(sh_turbo* t, uint32_t b, bool may_defer = false) {
  Block& blk = t->blocks[b];
  if (blk.location == SH_TURBO_GPU || blk.location == SH_TURBO_H2D) return SH_OK;
  int si = -1;
  int rc = take_slot(t, b, &si);
  if (rc != SH_OK) return rc;
  const bool from_d2h = blk.location == SH_TURBO_D2H;
  if (may_defer && t->deferred < 0 &&
      !(ticket_done(t, t->slots[si].fence_ticket) && (!from_d2h || ticket_done(t, blk.d2h_ticket)))) {
    t->deferred = b;
    t->deferred_from_d2h = from_d2h;
    blk.location = SH_TURBO_H2D;
    return SH_OK;
  }
  rc = issue_prefetch(t, b, from_d2h);
  if (rc != SH_OK) undo_prefetch(t, b, from_d2h);
  return rc;
}

// Evicts block b after the compute marked in t->compute_mark (recorded by the
// caller once every kernel that may read the slot is queued, and before
// anything later, such as the wait for the next block's H2D, is queued behind
// it: an eviction ordered after that wait would serialise each write-back
// behind the following load).
int async_evict(sh_turbo* t, uint32_t b) {
  Block& blk = t->blocks[b];
  if (blk.location == SH_TURBO_CPU || blk.location == SH_TURBO_D2H) return SH_OK;
  if (blk.slot < 0) return SH_OK;
  Slot& s = t->slots[blk.slot];
  // after the marked compute and after the block's own H2D
  SH_HIP(hipStreamWaitEvent(t->evict, t->compute_mark, 0));
  SH_HIP(hipStreamWaitEvent(t->evict, blk.h2d, 0));
  uint64_t ticket = 0;
  if (blk.writeback && t->sb && blk.digested) {
    // the slot's bytes since the H2D are digested: copy back the chunks that changed
    std::vector<sh_chunk_region> regions;
    uint64_t first = 0;
    for (const sh_copy_item& r : block_runs(blk, s)) {
      regions.push_back({r.dst, r.src, r.bytes, first});
      first += chunks_of(r.bytes, t->chunk);
    }
    // compared on the evict stream, right after the block's marked compute and its H2D
    int rc = sh_saveback_submit_chunks(t->sb, regions.data(), (uint32_t)regions.size(), t->chunk, blk.digests,
                                       blk.changed, t->evict, nullptr, 0, t->evict, &ticket);
    if (rc != SH_OK) return rc;
    int64_t span = -1;
    if (t->timing) {
      span = (int64_t)t->spans.size();
      t->spans.push_back({b, SH_TURBO_SPAN_WRITEBACK, 0, 0, 0});
    }
    t->tickets.push_back({ticket, span, true});
  } else if (blk.writeback && t->sb) {
    std::vector<sh_copy_item> items = writeback_items(t, blk, s);
    int rc = sh_saveback_submit(t->sb, items.data(), items.size(), t->evict, &ticket);
    if (rc != SH_OK) return rc;
    int64_t span = -1;
    if (t->timing) {
      uint64_t bytes = 0;
      for (const sh_copy_item& it : items) bytes += it.bytes;
      span = (int64_t)t->spans.size();
      t->spans.push_back({b, SH_TURBO_SPAN_WRITEBACK, 0, 0, bytes});
    }
    t->tickets.push_back({ticket, span, false});
  } else if (blk.writeback) {
    int rc = copy_block(t, blk, s, false, t->evict);
    if (rc != SH_OK) return rc;
  }
  blk.digested = false;
  SH_HIP(hipEventRecord(blk.d2h, t->evict));
  SH_HIP(hipEventRecord(s.fence, t->evict));
  s.fenced = true;
  s.fence_ticket = ticket;
  blk.d2h_ticket = ticket;
  s.assigned = -1;
  t->free_slots.push_back(blk.slot);
  blk.slot = -1;
  blk.location = SH_TURBO_D2H;
  return SH_OK;
}

int sync_prefetch(sh_turbo* t, uint32_t b, hipStream_t compute) {
  Block& blk = t->blocks[b];
  if (blk.location == SH_TURBO_GPU) return SH_OK;
  if (blk.location != SH_TURBO_H2D) {
    int rc = async_prefetch(t, b);
    if (rc != SH_OK) return rc;
  }
  SH_HIP(hipStreamWaitEvent(compute, blk.h2d, 0));
  blk.location = SH_TURBO_GPU;
  return SH_OK;
}

int sync_evict(sh_turbo* t) {
  SH_HIP(hipStreamSynchronize(t->evict));
  if (!t->tickets.empty()) {
    int rc = wait_ticket(t, t->tickets.back().ticket);
    if (rc != SH_OK) return rc;
  }
  for (Block& blk : t->blocks) {
    if (blk.location == SH_TURBO_D2H) blk.location = SH_TURBO_CPU;
    blk.d2h_ticket = 0;
  }
  for (Slot& s : t->slots) {
    s.fenced = false;
    s.fence_ticket = 0;
  }
  return SH_OK;
}

// d2h → cpu once the eviction has finished (the reference flips it in sync_evict)
void settle(sh_turbo* t, Block& blk) {
  if (blk.location == SH_TURBO_D2H && hipEventQuery(blk.d2h) == hipSuccess && ticket_done(t, blk.d2h_ticket)) {
    blk.location = SH_TURBO_CPU;
    blk.d2h_ticket = 0;
  }
}

}  // namespace

extern "C" int sh_turbo_create(sh_turbo** out) {
  sh::clear_error();
  if (!out) return sh::fail(SH_ERR_INVALID, "sh_turbo_create: null output");
  *out = new sh_turbo();
  return SH_OK;
}

extern "C" int sh_turbo_destroy(sh_turbo* t) {
  sh::clear_error();
  if (!t) return SH_OK;
  if (t->initialized) {
    (void)hipSetDevice(t->device);
    (void)hipStreamSynchronize(t->prefetch);
    (void)hipStreamSynchronize(t->evict);
  }
  if (t->sb) (void)sh_saveback_destroy(t->sb);  // waits for every write-back first
  for (Block& b : t->blocks) {
    if (b.host) (void)hipHostFree(b.host);
    if (b.h2d) (void)hipEventDestroy(b.h2d);
    if (b.d2h) (void)hipEventDestroy(b.d2h);
    if (b.t_start) (void)hipEventDestroy(b.t_start);
    if (b.t_end) (void)hipEventDestroy(b.t_end);
    if (b.digests) (void)hipFree(b.digests);
    if (b.changed) (void)hipHostFree(b.changed);
  }
  for (Slot& s : t->slots)  // device pointers belong to the caller
    if (s.fence) (void)hipEventDestroy(s.fence);
  if (t->compute_mark) (void)hipEventDestroy(t->compute_mark);
  if (t->prefetch) (void)hipStreamDestroy(t->prefetch);
  if (t->evict) (void)hipStreamDestroy(t->evict);
  delete t;
  return SH_OK;
}

extern "C" int sh_turbo_register_block(sh_turbo* t, const uint64_t* sizes, uint32_t n, uint32_t* index) {
  sh::clear_error();
  if (!t || !index || (n && !sizes)) return sh::fail(SH_ERR_INVALID, "sh_turbo_register_block: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  if (t->initialized) return sh::fail(SH_ERR_STATE, "register_block after initialize");
  Block b;
  b.sizes.assign(sizes, sizes + n);
  for (uint32_t i = 0; i < n; ++i) {
    b.offsets.push_back(b.extent);
    b.extent += align_up(sizes[i]);
  }
  *index = (uint32_t)t->blocks.size();
  t->blocks.push_back(std::move(b));
  return SH_OK;
}

extern "C" int sh_turbo_initialize(sh_turbo* t, int device, uint32_t window) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_initialize: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  if (t->initialized) return sh::fail(SH_ERR_STATE, "Already initialized");
  if (t->blocks.empty()) return sh::fail(SH_ERR_STATE, "No blocks registered");
  t->device = device;
  SH_HIP(hipSetDevice(device));
  SH_HIP(hipStreamCreateWithFlags(&t->prefetch, hipStreamNonBlocking));
  SH_HIP(hipStreamCreateWithFlags(&t->evict, hipStreamNonBlocking));
  SH_HIP(hipEventCreateWithFlags(&t->compute_mark, hipEventDisableTiming));
  if (t->sdma) {
    int rc = sh_saveback_create(device, &t->sb);
    if (rc != SH_OK) return rc;
  }
  size_t max_params = 0;
  for (const Block& b : t->blocks) max_params = std::max(max_params, b.sizes.size());
  std::vector<uint64_t> cap(max_params, 0);
  for (Block& b : t->blocks) {
    for (size_t p = 0; p < b.sizes.size(); ++p) cap[p] = std::max(cap[p], b.sizes[p]);
    if (b.extent) {
      void* h = nullptr;
      SH_HIP(hipHostMalloc(&h, b.extent, hipHostMallocDefault));
      b.host = static_cast<uint8_t*>(h);
    }
    SH_HIP(hipEventCreateWithFlags(&b.h2d, hipEventDisableTiming));
    SH_HIP(hipEventCreateWithFlags(&b.d2h, hipEventDisableTiming));
    const uint64_t nc = (t->sb && t->chunk) ? chunk_capacity(b, t->chunk) : 0;
    if (nc > 0) {
      SH_HIP(hipMalloc((void**)&b.digests, 16 * nc));
      void* h = nullptr;
      SH_HIP(hipHostMalloc(&h, nc, hipHostMallocDefault));
      b.changed = static_cast<uint8_t*>(h);
    }
  }
  const uint32_t w = std::min<uint32_t>(window, (uint32_t)t->blocks.size());
  for (uint32_t i = 0; i < w; ++i) {
    Slot s;
    s.ptrs.assign(max_params, nullptr);
    s.sizes = cap;
    SH_HIP(hipEventCreateWithFlags(&s.fence, hipEventDisableTiming));
    t->free_slots.push_back((int)t->slots.size());
    t->slots.push_back(std::move(s));
  }
  t->initialized = true;
  return SH_OK;
}

extern "C" int sh_turbo_set_save_back(sh_turbo* t, int sdma) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_set_save_back: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  if (t->initialized) return sh::fail(SH_ERR_STATE, "set_save_back after initialize");
  t->sdma = sdma != 0;
  return SH_OK;
}

extern "C" int sh_turbo_set_writeback_chunks(sh_turbo* t, uint32_t chunk_bytes) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_set_writeback_chunks: null engine");
  if (chunk_bytes % 16 != 0)
    return sh::fail(SH_ERR_INVALID, "sh_turbo_set_writeback_chunks: %u is not a multiple of 16", chunk_bytes);
  std::lock_guard<std::mutex> g(t->mu);
  if (t->initialized) return sh::fail(SH_ERR_STATE, "set_writeback_chunks after initialize");
  t->chunk = chunk_bytes;
  return SH_OK;
}

extern "C" int sh_turbo_stage_block(sh_turbo* t, uint32_t block, const void* const* src, uint32_t n) {
  sh::clear_error();
  if (!t || (n && !src)) return sh::fail(SH_ERR_INVALID, "sh_turbo_stage_block: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = require_init(t);
  if (rc == SH_OK) rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  Block& b = t->blocks[block];
  if (n != b.sizes.size()) return sh::fail(SH_ERR_STATE, "Expected %zu ptrs, got %u", b.sizes.size(), n);
  settle(t, b);
  if (b.location != SH_TURBO_CPU)
    return sh::fail(SH_ERR_STATE, "block %u is not in host memory (location %d)", block, b.location);
  std::vector<sh_copy_item> items;
  for (uint32_t p = 0; p < n; ++p) {
    if (b.sizes[p] == 0) continue;
    if (!src[p]) return sh::fail(SH_ERR_INVALID, "null source for param %u", p);
    items.push_back({b.host + b.offsets[p], src[p], b.sizes[p]});
  }
  return sh_host_copy_batch(items.data(), items.size(), 8);
}

extern "C" int sh_turbo_step(sh_turbo* t, uint32_t block, int direction, void* compute_stream) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_step: null engine");
  if (direction != SH_TURBO_FORWARD && direction != SH_TURBO_BACKWARD)
    return sh::fail(SH_ERR_INVALID, "direction must be 'forward' or 'backward'");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = require_init(t);
  if (rc == SH_OK) rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  SH_HIP(hipSetDevice(t->device));
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  // the previous block's last kernels are queued now; mark them before the
  // compute stream is made to wait for this block's H2D
  SH_HIP(hipEventRecord(t->compute_mark, compute));
  const uint32_t n = (uint32_t)t->blocks.size();
  const bool fwd = direction == SH_TURBO_FORWARD;
  const int64_t prev = fwd ? (int64_t)block - 1 : (int64_t)block + 1;
  const int64_t next = fwd ? (int64_t)block + 1 : (int64_t)block - 1;
  const bool has_prev = prev >= 0 && prev < n;
  if (t->deferred == (int64_t)block) {
    // this block's copy was deferred behind a write-back: queue the previous
    // block's write-back first, so the copy engine has it before the host
    // wait in the deferred copy ends (the block already holds its slot)
    if (has_prev) {
      rc = async_evict(t, (uint32_t)prev);
      if (rc != SH_OK) return rc;
    }
    rc = flush_deferred(t);
    if (rc == SH_OK) rc = sync_prefetch(t, block, compute);
    if (rc != SH_OK) return rc;
  } else {
    rc = flush_deferred(t);
    if (rc == SH_OK) rc = sync_prefetch(t, block, compute);
    if (rc != SH_OK) return rc;
    if (has_prev) {
      rc = async_evict(t, (uint32_t)prev);
      if (rc != SH_OK) return rc;
    }
  }
  if (next >= 0 && next < n) {
    // no slot for the lookahead block is not an error (engine.rs:334-337)
    if (async_prefetch(t, (uint32_t)next, true) != SH_OK) sh::clear_error();
  }
  return SH_OK;
}

extern "C" int sh_turbo_evict_sync(sh_turbo* t, uint32_t block, void* compute_stream) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_evict_sync: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = require_init(t);
  if (rc == SH_OK) rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  SH_HIP(hipSetDevice(t->device));
  SH_HIP(hipEventRecord(t->compute_mark, static_cast<hipStream_t>(compute_stream)));
  rc = flush_deferred(t);
  if (rc == SH_OK) rc = async_evict(t, block);
  if (rc != SH_OK) return rc;
  return sync_evict(t);
}

extern "C" int sh_turbo_drain(sh_turbo* t) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_drain: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  if (!t->initialized) return SH_OK;
  SH_HIP(hipSetDevice(t->device));
  int rc = flush_deferred(t);
  if (rc == SH_OK) rc = sync_evict(t);
  if (rc != SH_OK) return rc;
  SH_HIP(hipStreamSynchronize(t->prefetch));
  return SH_OK;
}

extern "C" int sh_turbo_gpu_ptr(sh_turbo* t, uint32_t block, uint32_t param, uint64_t* ptr) {
  sh::clear_error();
  if (!t || !ptr) return sh::fail(SH_ERR_INVALID, "sh_turbo_gpu_ptr: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  const Block& b = t->blocks[block];
  if (b.slot < 0) return sh::fail(SH_ERR_STATE, "Block has no GPU slot");
  if (param >= b.sizes.size()) return sh::fail(SH_ERR_STATE, "Param out of range");
  *ptr = (uint64_t)(uintptr_t)slot_param_ptr(t->slots[b.slot], b, param);
  return SH_OK;
}

extern "C" int sh_turbo_cpu_ptr(sh_turbo* t, uint32_t block, uint32_t param, uint64_t* ptr) {
  sh::clear_error();
  if (!t || !ptr) return sh::fail(SH_ERR_INVALID, "sh_turbo_cpu_ptr: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  const Block& b = t->blocks[block];
  if (param >= b.sizes.size()) return sh::fail(SH_ERR_STATE, "Param out of range");
  *ptr = b.host ? (uint64_t)(uintptr_t)(b.host + b.offsets[param]) : 0;
  return SH_OK;
}

extern "C" int sh_turbo_param_offset(sh_turbo* t, uint32_t block, uint32_t param, uint64_t* offset) {
  sh::clear_error();
  if (!t || !offset) return sh::fail(SH_ERR_INVALID, "sh_turbo_param_offset: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  const Block& b = t->blocks[block];
  if (param >= b.sizes.size()) return sh::fail(SH_ERR_STATE, "Param out of range");
  *offset = b.offsets[param];
  return SH_OK;
}

extern "C" int sh_turbo_set_slot_gpu_ptrs(sh_turbo* t, uint32_t slot, const uint64_t* ptrs, uint32_t n) {
  sh::clear_error();
  if (!t || (n && !ptrs)) return sh::fail(SH_ERR_INVALID, "sh_turbo_set_slot_gpu_ptrs: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  if (slot >= t->slots.size()) return sh::fail(SH_ERR_STATE, "Slot index out of range");
  Slot& s = t->slots[slot];
  if (s.assigned >= 0) return sh::fail(SH_ERR_STATE, "slot %u is occupied by block %d", slot, s.assigned);
  for (uint32_t i = 0; i < n && i < s.ptrs.size(); ++i) s.ptrs[i] = reinterpret_cast<void*>((uintptr_t)ptrs[i]);
  s.base = nullptr;
  s.bytes = 0;
  return SH_OK;
}

extern "C" int sh_turbo_set_slot_buffer(sh_turbo* t, uint32_t slot, void* base, uint64_t bytes) {
  sh::clear_error();
  if (!t || !base) return sh::fail(SH_ERR_INVALID, "sh_turbo_set_slot_buffer: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  if (slot >= t->slots.size()) return sh::fail(SH_ERR_STATE, "Slot index out of range");
  Slot& s = t->slots[slot];
  if (s.assigned >= 0) return sh::fail(SH_ERR_STATE, "slot %u is occupied by block %d", slot, s.assigned);
  if (reinterpret_cast<uintptr_t>(base) % kParamAlign)
    return sh::fail(SH_ERR_INVALID, "slot buffer must be %llu-byte aligned", (unsigned long long)kParamAlign);
  s.base = base;
  s.bytes = bytes;
  return SH_OK;
}

extern "C" int sh_turbo_slot_bytes(sh_turbo* t, uint64_t* bytes) {
  sh::clear_error();
  if (!t || !bytes) return sh::fail(SH_ERR_INVALID, "sh_turbo_slot_bytes: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  uint64_t m = 0;
  for (const Block& b : t->blocks) m = std::max(m, b.extent);
  *bytes = m;
  return SH_OK;
}

extern "C" int sh_turbo_set_writeback(sh_turbo* t, uint32_t block, int enable) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_set_writeback: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  t->blocks[block].writeback = enable != 0;
  return SH_OK;
}

extern "C" int sh_turbo_block_slot(sh_turbo* t, uint32_t block, int32_t* slot) {
  sh::clear_error();
  if (!t || !slot) return sh::fail(SH_ERR_INVALID, "sh_turbo_block_slot: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  *slot = block < t->blocks.size() ? t->blocks[block].slot : -1;
  return SH_OK;
}

extern "C" int sh_turbo_block_location(sh_turbo* t, uint32_t block, int* location) {
  sh::clear_error();
  if (!t || !location) return sh::fail(SH_ERR_INVALID, "sh_turbo_block_location: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  if (block >= t->blocks.size()) return sh::fail(SH_ERR_STATE, "Out of range");
  Block& b = t->blocks[block];
  if (t->initialized) settle(t, b);
  *location = b.location;
  return SH_OK;
}

extern "C" int sh_turbo_counts(sh_turbo* t, uint32_t* blocks, uint32_t* slots, uint32_t* free_slots) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_counts: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  if (blocks) *blocks = (uint32_t)t->blocks.size();
  if (slots) *slots = (uint32_t)t->slots.size();
  if (free_slots) *free_slots = (uint32_t)t->free_slots.size();
  return SH_OK;
}

extern "C" int sh_turbo_bytes(sh_turbo* t, uint64_t* h2d, uint64_t* d2h) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_bytes: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  if (h2d) *h2d = t->bytes_h2d;
  if (d2h) *d2h = t->bytes_d2h;
  return SH_OK;
}

extern "C" int sh_turbo_set_timing(sh_turbo* t, int enable) {
  sh::clear_error();
  if (!t) return sh::fail(SH_ERR_INVALID, "sh_turbo_set_timing: null engine");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = require_init(t);
  if (rc != SH_OK) return rc;
  SH_HIP(hipSetDevice(t->device));
  if (enable) {
    for (Block& b : t->blocks) {
      if (!b.t_start) SH_HIP(hipEventCreate(&b.t_start));
      if (!b.t_end) SH_HIP(hipEventCreate(&b.t_end));
      b.timed = false;
    }
    if (t->sb) {
      rc = sh_saveback_set_timing(t->sb, 1);
      if (rc != SH_OK) return rc;
    }
    t->spans.clear();
  }
  t->timing = enable != 0;
  return SH_OK;
}

extern "C" int sh_turbo_trace_spans(sh_turbo* t, sh_turbo_span* out, uint32_t cap, uint32_t* n) {
  sh::clear_error();
  if (!t || !n || (cap && !out)) return sh::fail(SH_ERR_INVALID, "sh_turbo_trace_spans: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = require_init(t);
  if (rc != SH_OK) return rc;
  // every recorded write-back has completed before its times are read
  for (auto it = t->tickets.rbegin(); it != t->tickets.rend(); ++it) {
    if (it->span < 0) continue;
    rc = wait_ticket(t, it->ticket);
    if (rc != SH_OK) return rc;
    break;
  }
  *n = (uint32_t)t->spans.size();
  std::copy_n(t->spans.begin(), std::min<size_t>(cap, t->spans.size()), out);
  return SH_OK;
}

extern "C" int sh_turbo_block_times(sh_turbo* t, uint32_t block, void* ref_event, float* out2) {
  sh::clear_error();
  if (!t || !ref_event || !out2) return sh::fail(SH_ERR_INVALID, "sh_turbo_block_times: null argument");
  std::lock_guard<std::mutex> g(t->mu);
  int rc = check_block(t, block);
  if (rc != SH_OK) return rc;
  Block& b = t->blocks[block];
  if (!b.timed) return sh::fail(SH_ERR_STATE, "block %u has no timed H2D", block);
  SH_HIP(hipEventSynchronize(b.t_end));
  hipEvent_t ref = static_cast<hipEvent_t>(ref_event);
  SH_HIP(hipEventElapsedTime(&out2[0], ref, b.t_start));
  SH_HIP(hipEventElapsedTime(&out2[1], ref, b.t_end));
  return SH_OK;
}
