// Host-bank pager: the refinement banks of every (stream, layer) key live in pinned host
// memory, and a few device slots stage them for the layer that runs (the paging of
// recap/host_banks.py:17-276, as native runtime).
//
// A key's bank is a fixed list of fields (the refinement, its log-mass, the partition, the
// kernel mask, the drift reference), each a byte range of known size; a slot holds one
// bank's fields in device memory the caller owns and binds once.  Three kinds of transfer:
//
//   stage_in   key -> slot, ordered on the caller's compute stream: waits for a prefetch of
//              that key into that slot if one was issued, else copies on the compute stream;
//   prefetch   key -> slot on the pager's prefetch stream, after the compute stream is done
//              with the slot (release) and the slot's last write-back has read it out;
//   stage_out  slot -> key on the pager's write-back stream, after the work queued so far on
//              the compute stream (the refresh that wrote the slot);
//   acquire    no transfer: the compute stream waits until the slot may be written without
//              a load (its last write-back has read it out, no prefetch is filling it).
//
// Events fence every reuse: per slot (released by compute, prefetched, written back) and per
// key (host copy written, host copy being read by a prefetch).  Streams are created
// non-blocking at the default priority.  One pager is driven by one host thread.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>
#include <vector>

#include "kernels.hpp"

namespace recap {

struct Fence {              // an event and whether it has been recorded since creation
  hipEvent_t ev = nullptr;
  bool set = false;
};

struct Slot {
  std::vector<void*> dev;   // bound device fields
  int64_t resident = -1;    // key whose data is (or, once prefetched, will be) here
  bool prefetched = false;  // a prefetch into this slot is pending consumption
  Fence ready;              // prefetch copies done (prefetch stream)
  Fence released;           // compute's last use of the slot (compute stream)
  Fence written;            // write-back copies out of the slot done (write-back stream)
};

struct Key {
  std::vector<void*> host;  // pinned host fields, allocated on first use
  std::vector<int64_t> cap; // bytes allocated per host field (>= the field's current size)
  bool stored = false;      // holds a bank written back by a refresh
  Fence written;            // last write-back into the host copy done
  Fence read;               // last prefetch out of the host copy done
};

struct Pager {
  int device = 0;
  std::vector<int64_t> bytes;
  std::vector<Slot> slots;
  std::vector<Key> keys;
  hipStream_t prefetch = nullptr, writeback = nullptr;
  Fence marker;             // a point on the compute stream the write-back stream waits for
  bool timing = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> copies;  // timed copy batches not yet folded
  double copied_ms = 0.0;   // folded batches: total milliseconds and count
  int64_t copied_batches = 0;
  int64_t host_bytes = 0;
  int64_t counts[4] = {0, 0, 0, 0};  // stage-ins taken from a prefetch, copied; prefetches; stage-outs
};

namespace {

hipError_t make_fence(Fence& f) {
  f.set = false;
  return hipEventCreateWithFlags(&f.ev, hipEventDisableTiming);
}

void drop_fence(Fence& f) {
  if (f.ev) (void)hipEventDestroy(f.ev);
  f.ev = nullptr;
  f.set = false;
}

hipError_t record(Fence& f, hipStream_t s) {
  hipError_t e = hipEventRecord(f.ev, s);
  if (e == hipSuccess) f.set = true;
  return e;
}

hipError_t wait(hipStream_t s, const Fence& f) {
  return f.set ? hipStreamWaitEvent(s, f.ev, 0) : hipSuccess;
}

#define HIP_TRY(expr)                          \
  do {                                         \
    const hipError_t _e = (expr);              \
    if (_e != hipSuccess) return _e;           \
  } while (0)

// Pinned host fields of key k for the current field sizes: a field not yet allocated (or
// freed by a resize that outgrew it) is allocated now.
hipError_t ensure_host(Pager& p, Key& k) {
  if (k.host.empty()) {
    k.host.assign(p.bytes.size(), nullptr);
    k.cap.assign(p.bytes.size(), 0);
  }
  for (size_t f = 0; f < p.bytes.size(); ++f) {
    if (k.host[f] != nullptr) continue;
    const int64_t n = p.bytes[f] > 0 ? p.bytes[f] : 1;
    HIP_TRY(hipHostMalloc(&k.host[f], (size_t)n, hipHostMallocDefault));
    k.cap[f] = n;
    p.host_bytes += n;
  }
  return hipSuccess;
}

// Folds timed copy batches whose end event has completed into the running total and
// destroys their events; with `wait`, waits for every batch first.  On an error the batch
// that raised it and the later ones are kept.
hipError_t fold_copies(Pager& p, bool wait) {
  size_t kept = 0, i = 0;
  hipError_t err = hipSuccess;
  for (; i < p.copies.size(); ++i) {
    const auto c = p.copies[i];
    hipError_t e = wait ? hipEventSynchronize(c.second) : hipEventQuery(c.second);
    if (!wait && e == hipErrorNotReady) {
      p.copies[kept++] = c;
      continue;
    }
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, c.first, c.second);
    if (e != hipSuccess) {
      err = e;
      break;
    }
    p.copied_ms += ms;
    ++p.copied_batches;
    (void)hipEventDestroy(c.first);
    (void)hipEventDestroy(c.second);
  }
  for (; i < p.copies.size(); ++i) p.copies[kept++] = p.copies[i];
  p.copies.resize(kept);
  return err;
}

// Copies every field between `dst` and `src` on `s`, bracketed by timing events when the
// pager times its copies.
hipError_t copy_fields(Pager& p, const std::vector<void*>& dst, const std::vector<void*>& src,
                       hipMemcpyKind kind, hipStream_t s) {
  hipEvent_t t0 = nullptr, t1 = nullptr;
  hipError_t e = hipSuccess;
  if (p.timing) {
    if (p.copies.size() >= 64) HIP_TRY(fold_copies(p, false));  // bounded event count
    e = hipEventCreate(&t0);
    if (e == hipSuccess) e = hipEventCreate(&t1);
    if (e == hipSuccess) e = hipEventRecord(t0, s);
  }
  for (size_t f = 0; f < p.bytes.size() && e == hipSuccess; ++f)
    if (p.bytes[f] > 0) e = hipMemcpyAsync(dst[f], src[f], (size_t)p.bytes[f], kind, s);
  if (p.timing) {
    if (e == hipSuccess) e = hipEventRecord(t1, s);
    if (e == hipSuccess) {
      p.copies.emplace_back(t0, t1);
    } else {  // a batch that did not complete its records is not timed
      if (t0) (void)hipEventDestroy(t0);
      if (t1) (void)hipEventDestroy(t1);
    }
  }
  return e;
}

}  // namespace

hipError_t pager_create(int64_t n_keys, int n_slots, const int64_t* field_bytes, int n_fields,
                        bool timing, Pager** out) {
  Pager* p = new Pager();
  p->timing = timing;
  p->bytes.assign(field_bytes, field_bytes + n_fields);
  hipError_t e = hipGetDevice(&p->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->prefetch, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->writeback, hipStreamNonBlocking);
  p->slots.resize((size_t)n_slots);
  p->keys.resize((size_t)n_keys);
  if (e == hipSuccess) e = make_fence(p->marker);
  for (Slot& s : p->slots) {
    if (e == hipSuccess) e = make_fence(s.ready);
    if (e == hipSuccess) e = make_fence(s.released);
    if (e == hipSuccess) e = make_fence(s.written);
  }
  for (Key& k : p->keys) {
    if (e == hipSuccess) e = make_fence(k.written);
    if (e == hipSuccess) e = make_fence(k.read);
  }
  if (e != hipSuccess) {
    pager_destroy(p);
    return e;
  }
  *out = p;
  return hipSuccess;
}

hipError_t pager_finish(Pager* p) {
  HIP_TRY(hipStreamSynchronize(p->prefetch));
  HIP_TRY(hipStreamSynchronize(p->writeback));
  for (Slot& s : p->slots) {
    if (s.released.set) HIP_TRY(hipEventSynchronize(s.released.ev));
    s.prefetched = false;   // a prefetch not taken by now is dropped (its data stays valid)
  }
  return hipSuccess;
}

void pager_destroy(Pager* p) {
  if (p == nullptr) return;
  if (p->prefetch) (void)hipStreamSynchronize(p->prefetch);
  if (p->writeback) (void)hipStreamSynchronize(p->writeback);
  for (Slot& s : p->slots) {
    if (s.released.set) (void)hipEventSynchronize(s.released.ev);
    drop_fence(s.ready);
    drop_fence(s.released);
    drop_fence(s.written);
  }
  for (Key& k : p->keys) {
    for (void* h : k.host)
      if (h) (void)hipHostFree(h);
    drop_fence(k.written);
    drop_fence(k.read);
  }
  for (auto& c : p->copies) {
    (void)hipEventDestroy(c.first);
    (void)hipEventDestroy(c.second);
  }
  drop_fence(p->marker);
  if (p->prefetch) (void)hipStreamDestroy(p->prefetch);
  if (p->writeback) (void)hipStreamDestroy(p->writeback);
  delete p;
}

int pager_slots(const Pager* p) { return (int)p->slots.size(); }
int64_t pager_keys(const Pager* p) { return (int64_t)p->keys.size(); }
int pager_fields(const Pager* p) { return (int)p->bytes.size(); }
int64_t pager_field_bytes(const Pager* p, int field) { return p->bytes[(size_t)field]; }
bool pager_bound(const Pager* p, int slot) { return !p->slots[(size_t)slot].dev.empty(); }
bool pager_stored(const Pager* p, int64_t key) { return p->keys[(size_t)key].stored; }
int64_t pager_host_bytes(const Pager* p) { return p->host_bytes; }
void pager_counts(const Pager* p, int64_t* out4) {
  for (int i = 0; i < 4; ++i) out4[i] = p->counts[i];
}

void pager_bind(Pager* p, int slot, void* const* fields) {
  Slot& s = p->slots[(size_t)slot];
  s.dev.assign(fields, fields + p->bytes.size());
  s.resident = -1;
  s.prefetched = false;
}

hipError_t pager_reserve(Pager* p, int64_t n_keys) {
  for (int64_t k = 0; k < n_keys && k < (int64_t)p->keys.size(); ++k)
    HIP_TRY(ensure_host(*p, p->keys[(size_t)k]));
  return hipSuccess;
}

hipError_t pager_stage_in(Pager* p, int64_t key, int slot, hipStream_t s) {
  Slot& sl = p->slots[(size_t)slot];
  Key& k = p->keys[(size_t)key];
  if (sl.prefetched && sl.resident == key) {
    sl.prefetched = false;
    ++p->counts[0];
    return wait(s, sl.ready);       // the prefetch stream already brought it in
  }
  // The copy below overwrites the slot on the compute stream: a prefetch still filling it
  // (for another key) and the slot's pending write-back must be done; the host copy must
  // be complete.  Compute's own earlier use of the slot is ordered by the stream.
  if (sl.prefetched) HIP_TRY(wait(s, sl.ready));
  sl.prefetched = false;
  HIP_TRY(wait(s, sl.written));
  HIP_TRY(wait(s, k.written));
  HIP_TRY(copy_fields(*p, sl.dev, k.host, hipMemcpyHostToDevice, s));
  sl.resident = key;
  ++p->counts[1];
  return hipSuccess;
}

hipError_t pager_prefetch(Pager* p, int64_t key, int slot) {
  Slot& sl = p->slots[(size_t)slot];
  Key& k = p->keys[(size_t)key];
  if (sl.prefetched && sl.resident == key) return hipSuccess;
  HIP_TRY(wait(p->prefetch, sl.released));   // compute has finished with the slot
  HIP_TRY(wait(p->prefetch, sl.written));    // its last contents have been written back
  HIP_TRY(wait(p->prefetch, k.written));     // the host copy is complete
  HIP_TRY(copy_fields(*p, sl.dev, k.host, hipMemcpyHostToDevice, p->prefetch));
  HIP_TRY(record(sl.ready, p->prefetch));
  HIP_TRY(record(k.read, p->prefetch));
  sl.resident = key;
  sl.prefetched = true;
  ++p->counts[2];
  return hipSuccess;
}

hipError_t pager_stage_out(Pager* p, int64_t key, int slot, hipStream_t s) {
  Slot& sl = p->slots[(size_t)slot];
  Key& k = p->keys[(size_t)key];
  HIP_TRY(ensure_host(*p, k));
  // A wait takes the event's latest record at the time of the call, so one marker event
  // serves every stage-out.
  HIP_TRY(record(p->marker, s));             // the refresh that wrote the slot
  HIP_TRY(wait(p->writeback, p->marker));
  HIP_TRY(wait(p->writeback, k.read));       // no prefetch is still reading the host copy
  HIP_TRY(copy_fields(*p, k.host, sl.dev, hipMemcpyDeviceToHost, p->writeback));
  HIP_TRY(record(sl.written, p->writeback));
  HIP_TRY(record(k.written, p->writeback));
  k.stored = true;
  sl.resident = key;
  sl.prefetched = false;
  ++p->counts[3];
  return hipSuccess;
}

hipError_t pager_acquire(Pager* p, int slot, hipStream_t s) {
  // The compute stream is about to write the slot without loading it (a first refresh): a
  // prefetch still filling it and its last write-back must be done first.
  Slot& sl = p->slots[(size_t)slot];
  if (sl.prefetched) HIP_TRY(wait(s, sl.ready));
  sl.prefetched = false;
  HIP_TRY(wait(s, sl.written));
  sl.resident = -1;
  return hipSuccess;
}

hipError_t pager_release(Pager* p, int slot, hipStream_t s) {
  return record(p->slots[(size_t)slot].released, s);
}

hipError_t pager_copy_time(Pager* p, double* total_ms, int64_t* n) {
  HIP_TRY(fold_copies(*p, true));
  *total_ms = p->copied_ms;
  *n = p->copied_batches;
  return hipSuccess;
}

hipError_t pager_resize(Pager* p, const int64_t* field_bytes) {
  // Every transfer in flight reads or writes the old geometry: let them end first.
  HIP_TRY(pager_finish(p));
  for (size_t f = 0; f < p->bytes.size(); ++f) p->bytes[f] = field_bytes[f];
  for (Key& k : p->keys) {
    for (size_t f = 0; f < k.host.size(); ++f) {
      if (k.host[f] == nullptr || k.cap[f] >= p->bytes[f]) continue;
      HIP_TRY(hipHostFree(k.host[f]));   // outgrown: reallocated on the key's next write-back
      p->host_bytes -= k.cap[f];
      k.host[f] = nullptr;
      k.cap[f] = 0;
    }
    k.stored = false;                    // a bank of the old geometry is no bank of the new
  }
  for (Slot& s : p->slots) {
    s.dev.clear();                       // the caller binds device fields of the new sizes
    s.resident = -1;
    s.prefetched = false;
  }
  return hipSuccess;
}

}  // namespace recap
