// c_api.cpp -- the C ABI of include/adaptq.h on top of the gfx950 kernels.
//
// Restates the contracts of the reference's core/adaptq_c_api.cpp:15-281
// (validation, per-head seeds, thread-local error strings, return codes) and
// attention.cpp:324-366 (head setup, append bookkeeping).  Differences, all
// deliberate:
//   * state lives in device HBM; appends are staged on the host and quantised
//     by one kernel launch per flush;
//   * nothing throws across the ABI; allocation failure returns NULL with an
//     ADAPTQ_ERR_ALLOC message (the reference lets bad_alloc escape,
//     ring_buffer.cpp:71-76);
//   * adaptq_mha_create fails as a whole if a head fails (the reference keeps
//     NULL heads, c_api.cpp:159-163).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/adaptq.h"
#include "device.hpp"
#include "launch.hpp"

// Workspace of the allocation-free decode (adaptq_plan_compute_device_static):
// one copy per GPU, held from the code object's load until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host it is only
// a stand-in for the symbol): set-up reads each device's address of it with
// hipGetSymbolAddress (DevSync::scratch) and that address is what kernels get.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

thread_local char tl_error[256] = "";

void set_error(const char *msg) { std::snprintf(tl_error, sizeof(tl_error), "%s", msg); }

void set_errorf(const char *fn, const char *what) {
  std::snprintf(tl_error, sizeof(tl_error), "%s: %s", fn, what);
}

void clear_error() { tl_error[0] = '\0'; }

bool require_handle(const void *h, const char *fn) {
  if (h) return true;
  set_errorf(fn, "null handle");
  return false;
}

bool require_pointer(const void *p, const char *fn, const char *param) {
  if (p) return true;
  char msg[256];
  std::snprintf(msg, sizeof(msg), "%s: null %s", fn, param);
  set_error(msg);
  return false;
}

bool hip_fail(hipError_t e, const char *fn) {
  if (e == hipSuccess) return false;
  char msg[256];
  std::snprintf(msg, sizeof(msg), "%s: HIP error: %s", fn, hipGetErrorString(e));
  set_error(msg);
  return true;
}

int next_pow2(int n) {
  if (n <= 1) return 1;
  if (n > (1 << 30)) return 1 << 30;
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

bool valid_bits(int b) { return b == 16 || (b >= 2 && b <= 4); }

// ---- Stream ordering ----
//
// Work on a context's ring is queued on two kinds of streams: the library's
// own stream per device (host-form calls: flushes of staged rows, host
// compute, reset) and callers' streams (the *_device entry points).  The
// library stream is a blocking stream, so the HIP null stream (NULL, torch's
// default stream) and it wait for each other's earlier work by themselves;
// for any other caller stream:
//   * after a device-form launch, the caller's stream is marked as carrying
//     device-form work (a table of up to 16 streams per device);
//   * before library-stream work, if any marked stream exists, the host waits
//     for the device once (wait_callers) and clears the marks;
//   * before a device-form launch, the caller's stream waits on an event
//     recorded after the library stream's latest work, unless the host has
//     already seen that work complete (no host wait).
// Library-stream submissions are numbered per device; `done` is the highest
// number the host has seen complete, so host waits (outputs of host-form
// calls, reuse of pinned staging memory, inspection) happen only when the
// work they need may still be running.  Device-form calls on different
// caller streams that touch the same contexts are ordered by the caller, as
// for any stream-taking library call.
constexpr int kMaxDevices = 64;
constexpr int kMaxCallerStreams = 16;

struct DevSync {
  std::mutex mu;
  hipStream_t lib = nullptr;
  hipEvent_t lib_ev = nullptr;
  uint64_t enq = 0;        // library-stream submissions so far
  uint64_t done = 0;       // submissions the host has seen complete
  uint64_t lib_ev_at = 0;  // submission count when lib_ev was recorded
  struct Caller {
    hipStream_t s;
    bool fresh;  // device-form work queued since the last wait_callers
  };
  Caller caller[kMaxCallerStreams];  // caller streams seen
  int n_caller = 0;
  int evict = 0;
  void *scratch = nullptr;  // this device's address of the static scratch
  // Allocation-free decodes share `scratch`: each call's stream waits for the
  // event recorded after the previous call (static_mu orders the
  // wait / launch / record sequences of concurrent host threads).
  std::mutex static_mu;
  hipEvent_t static_ev = nullptr;
  bool static_used = false;
};

DevSync g_dev[kMaxDevices];

DevSync *dev_sync(int dev) { return dev >= 0 && dev < kMaxDevices ? &g_dev[dev] : nullptr; }

// Per-device set-up, once, with the device current (caller holds d->mu):
// the library stream, its event and the device's address of the static
// scratch.  Everything a later call needs is made here, so the calls
// themselves create nothing.
hipError_t ensure_lib(DevSync *d) {
  if (d->lib) return hipSuccess;
  hipStream_t s = nullptr;
  // blocking (synchronises with the null stream), default priority
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamDefault);
  if (e != hipSuccess) return e;
  hipEvent_t ev = nullptr, sev = nullptr;
  e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&sev, hipEventDisableTiming);
  void *sp = nullptr;
  if (e == hipSuccess) e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
  if (e != hipSuccess) {
    if (ev) (void)hipEventDestroy(ev);
    if (sev) (void)hipEventDestroy(sev);
    (void)hipStreamDestroy(s);
    return e;
  }
  d->lib_ev = ev;
  d->static_ev = sev;
  d->scratch = sp;
  d->lib = s;
  return hipSuccess;
}

// Set-up of the current device (context creation calls it).
hipError_t init_device(int dev) {
  DevSync *d = dev_sync(dev);
  if (!d) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(d->mu);
  return ensure_lib(d);
}

// Caller holds d->mu: the device finishes the work queued so far on every
// caller stream that has carried device-form launches since the last such
// wait, before any library-stream work is queued.  The host waits for the
// device here rather than recording an event on each caller stream after
// each launch: a record per call cost about 3 us of host time and stretched
// the GPU timeline by as much, and a record made only now could touch a
// stream its owner has destroyed since.  Steady device-form use never gets
// here; a host-form call, reset, inspection or snapshot after device-form
// launches pays one device wait.
hipError_t wait_callers(DevSync *d) {
  bool any = false;
  for (int i = 0; i < d->n_caller; ++i) any = any || d->caller[i].fresh;
  if (!any) return hipSuccess;
  const int dev = (int)(d - g_dev);
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (cur >= 0 && cur != dev) {
    const hipError_t e2 = hipSetDevice(cur);
    if (e == hipSuccess) e = e2;
  }
  if (e != hipSuccess) return e;
  for (int i = 0; i < d->n_caller; ++i) d->caller[i].fresh = false;
  return hipSuccess;
}

// Before queueing library-stream work for a context on the current device:
// returns the library stream, which now waits for callers' queued work.
hipError_t lib_begin(int dev, hipStream_t *out) {
  DevSync *d = dev_sync(dev);
  if (!d) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(d->mu);
  hipError_t e = ensure_lib(d);
  if (e == hipSuccess) e = wait_callers(d);
  *out = d->lib;
  return e;
}

// After queueing library-stream work: its submission number.
uint64_t lib_end(int dev) {
  DevSync *d = dev_sync(dev);
  std::lock_guard<std::mutex> g(d->mu);
  return ++d->enq;
}

// The host waits until library-stream submission `upto` has completed.
hipError_t lib_wait(int dev, uint64_t upto) {
  DevSync *d = dev_sync(dev);
  if (!d) return hipErrorInvalidDevice;
  hipStream_t s;
  uint64_t target;
  {
    std::lock_guard<std::mutex> g(d->mu);
    if (d->done >= upto || !d->lib) return hipSuccess;
    s = d->lib;
    target = d->enq;
  }
  const hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> g(d->mu);
  if (d->done < target) d->done = target;
  return hipSuccess;
}

// Everything queued for the device so far -- library stream and callers'
// device-form launches -- has completed when this returns (inspection,
// snapshots, destruction).
hipError_t settle(int dev) {
  DevSync *d = dev_sync(dev);
  if (!d) return hipErrorInvalidDevice;
  uint64_t target;
  {
    std::lock_guard<std::mutex> g(d->mu);
    hipError_t e = ensure_lib(d);
    if (e == hipSuccess) e = wait_callers(d);
    if (e != hipSuccess) return e;
    target = d->enq;
  }
  return lib_wait(dev, target);
}

// The legacy null stream (NULL or hipStreamLegacy) and the blocking library
// stream order each other's work implicitly.
bool is_null_stream(hipStream_t s) { return s == nullptr || s == hipStreamLegacy; }

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st == hipStreamCaptureStatusActive;
}

// Before a device-form launch on caller stream s: s waits for the library
// stream's work that may still be running.  Under graph capture the host
// waits instead (an event from outside the capture cannot be waited on).
hipError_t caller_begin(int dev, hipStream_t s) {
  if (is_null_stream(s)) return hipSuccess;  // it waits for the blocking library stream
  DevSync *d = dev_sync(dev);
  if (!d) return hipErrorInvalidDevice;
  uint64_t target = 0;
  {
    std::lock_guard<std::mutex> g(d->mu);
    if (d->enq <= d->done) return hipSuccess;
    if (!capturing(s)) {
      if (d->lib_ev_at < d->enq) {
        const hipError_t e = hipEventRecord(d->lib_ev, d->lib);
        if (e != hipSuccess) return e;
        d->lib_ev_at = d->enq;
      }
      return hipStreamWaitEvent(s, d->lib_ev, 0);
    }
    target = d->enq;
  }
  return lib_wait(dev, target);
}

// After a device-form launch on caller stream s: note the stream, so that
// library-stream work waits for it (wait_callers).  Launches captured into a
// graph run at replay, outside this bookkeeping.
hipError_t caller_end(int dev, hipStream_t s) {
  if (is_null_stream(s)) return hipSuccess;  // later library-stream work waits for it
  DevSync *d = dev_sync(dev);
  if (!d) return hipErrorInvalidDevice;
  if (capturing(s)) return hipSuccess;
  std::lock_guard<std::mutex> g(d->mu);
  DevSync::Caller *c = nullptr;
  for (int i = 0; i < d->n_caller && !c; ++i)
    if (d->caller[i].s == s) c = &d->caller[i];
  if (!c) {
    if (!d->lib) return hipErrorNotInitialized;  // a context's creation sets the device up
    if (d->n_caller < kMaxCallerStreams) {
      c = &d->caller[d->n_caller];
      ++d->n_caller;
    } else {
      // reuse the slot of another stream once the device has finished the
      // work that stream carried
      c = &d->caller[d->evict];
      d->evict = (d->evict + 1) % kMaxCallerStreams;
      if (c->fresh) {
        const hipError_t e = wait_callers(d);  // before the slot forgets its stream
        if (e != hipSuccess) return e;
      }
    }
    c->s = s;
  }
  c->fresh = true;
  return hipSuccess;
}

// Any change to a context's host-visible ring state (staged rows, appends,
// resets, loads) moves this counter; a plan whose contexts have not changed
// since its last scan skips the scan.
std::atomic<uint64_t> g_epoch{1};

void bump_epoch() { g_epoch.fetch_add(1, std::memory_order_acq_rel); }

struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  hipError_t ensure(size_t need) {
    if (need <= bytes) return hipSuccess;
    if (p) (void)hipFree(p);  // hipFree waits for the device: no kernel still uses it
    p = nullptr;
    bytes = 0;
    size_t want = std::max(need, (size_t)4096);
    hipError_t e = hipMalloc(&p, want);
    if (e == hipSuccess) bytes = want;
    return e;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
};

// Pinned host memory that kernels read and write directly (device-visible
// pointer dp).  Whoever reuses or frees it first waits for the kernels that
// may still use it.
struct PinnedBuf {
  void *p = nullptr;
  void *dp = nullptr;
  size_t bytes = 0;
  hipError_t ensure(size_t need) {
    if (need <= bytes) return hipSuccess;
    release();
    const size_t want = std::max(need, (size_t)4096);
    hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
    if (e != hipSuccess) {
      p = nullptr;
      return e;
    }
    e = hipHostGetDevicePointer(&dp, p, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(p);
      p = dp = nullptr;
      return e;
    }
    bytes = want;
    return hipSuccess;
  }
  void release() {
    if (p) (void)hipHostFree(p);
    p = dp = nullptr;
    bytes = 0;
  }
};

constexpr int kStageTokens = 1024;
// Flushes of up to this many tokens per head are read by the append kernel
// straight from pinned host memory; larger ones go to the device in one
// asynchronous copy first.
constexpr int kDirectTokens = 64;

struct Ctx {
  std::mutex mu;
  int device = 0;
  int dim = 0, padded = 0, k_bits = 0, v_bits = 0, cap = 0, hyb = 0, k_pb = 0, v_pb = 0;
  float v_mass = 0.f;
  aq::RingState st{0, 0, 0, 0};
  aq::HeadDesc hd{};  // host copy of the device descriptor's pointers and config
  void *slab = nullptr;
  aq::HeadDesc *d_desc = nullptr;
  aq::HeadDesc **d_desc_list = nullptr;  // one entry: d_desc
  std::vector<float> stage_k, stage_v;
  int staged = 0;
  DevBuf d_stage, d_ws, d_items;
  PinnedBuf h_stage, h_io;  // staged rows for the append kernel; queries and outputs
  uint64_t stage_seq = 0;   // library-stream submission that last read h_stage
  int items_uploaded = 0;
};

struct Mha {
  std::vector<Ctx *> heads;
  int n_heads = 0;
  int device = 0;
  std::mutex mu;  // whole-MHA calls; taken before any head's lock
  DevBuf d_list;  // [n_heads] device pointers to the heads' descriptors
  DevBuf d_rep;   // [reps][n_heads] the same pointers repeated (multi-query launches)
  int rep_n = 0;  // reps held in d_rep
  DevBuf d_ws, d_io, d_stage;
  PinnedBuf h_stage, h_io;
  uint64_t stage_seq = 0;  // library-stream submission that last read h_stage
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Whether appending n tokens to these contexts copies any to a hybrid mirror
// (from the host's ring states; it picks the append's launch shape only).
bool any_mirror(const std::vector<Ctx *> &cs, int n) {
  for (const Ctx *c : cs)
    if (aq::mirror_count(c->st, n, c->cap, c->hyb) > 0) return true;
  return false;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (prev >= 0 && cur != prev) (void)hipSetDevice(prev);
  }
};

void free_ctx(Ctx *c) {
  if (!c) return;
  {
    DeviceGuard g(c->device);
    (void)settle(c->device);  // no queued kernel may still use the slab or the pinned rows
    if (c->slab) (void)hipFree(c->slab);
    c->d_stage.release();
    c->d_ws.release();
    c->d_items.release();
    c->h_stage.release();
    c->h_io.release();
  }
  delete c;
}

Ctx *create_ctx(int dim, int k_bits, int v_bits, int capacity, uint64_t seed, float v_mass,
                int hyb, const char *fn) {
  const int padded = next_pow2(dim);
  if (padded > aq::kMaxPadded) {
    set_errorf(fn, "head dimension too large (padded dimension > 1024)");
    return nullptr;
  }
  Ctx *c = new (std::nothrow) Ctx();
  if (!c) {
    set_errorf(fn, "host allocation failed");
    return nullptr;
  }
  if (hipGetDevice(&c->device) != hipSuccess || c->device < 0 || c->device >= kMaxDevices) {
    delete c;
    set_errorf(fn, "no HIP device available");
    return nullptr;
  }
  if (hip_fail(init_device(c->device), fn)) {
    delete c;
    return nullptr;
  }
  c->dim = dim;
  c->padded = padded;
  c->k_bits = k_bits;
  c->v_bits = v_bits;
  c->cap = capacity;
  c->hyb = hyb;
  c->v_mass = v_mass;
  c->k_pb = aq::packed_bytes(padded, k_bits);
  c->v_pb = aq::packed_bytes(padded, v_bits);

  // Rademacher signs, restating core/fwht.cpp:21-27 (xorshift64 13/7/17,
  // odd -> +1) for the padded length (quantizer.cpp:32-33).
  uint32_t sign_words[aq::kMaxSignWords] = {};
  {
    uint64_t s = seed ? seed : 0xdeadbeefcafe1234ULL;
    for (int i = 0; i < padded; ++i) {
      s ^= s << 13;
      s ^= s >> 7;
      s ^= s << 17;
      if (s & 1u) sign_words[i >> 5] |= 1u << (i & 31);
    }
  }

  const size_t cap_sz = (size_t)(capacity > 0 ? capacity : 0);
  size_t off = 0;
  const size_t o_desc = off;
  off += align256(sizeof(aq::HeadDesc));
  const size_t o_list = off;
  off += align256(sizeof(void *));
  const size_t o_signs = off;
  off += align256(sizeof(sign_words));
  const size_t o_kc = off;
  off += align256(cap_sz * c->k_pb);
  const size_t o_vc = off;
  off += align256(cap_sz * c->v_pb);
  const size_t o_ks = off;
  off += align256(cap_sz * 4);
  const size_t o_vs = off;
  off += align256(cap_sz * 4);
  const size_t o_rk = off;
  off += align256((size_t)hyb * dim * 4);
  const size_t o_rv = off;
  off += align256((size_t)hyb * dim * 4);

  if (hipMalloc(&c->slab, off) != hipSuccess || !c->slab) {
    (void)hipGetLastError();
    c->slab = nullptr;
    free_ctx(c);
    set_errorf(fn, "device allocation failed");
    return nullptr;
  }
  uint8_t *base = static_cast<uint8_t *>(c->slab);
  aq::HeadDesc &h = c->hd;
  h.k_codes = base + o_kc;
  h.v_codes = base + o_vc;
  h.k_scale = reinterpret_cast<float *>(base + o_ks);
  h.v_scale = reinterpret_cast<float *>(base + o_vs);
  h.raw_k = reinterpret_cast<float *>(base + o_rk);
  h.raw_v = reinterpret_cast<float *>(base + o_rv);
  h.signs = reinterpret_cast<uint32_t *>(base + o_signs);
  h.dim = dim;
  h.padded = padded;
  h.k_bits = k_bits;
  h.v_bits = v_bits;
  h.k_pb = c->k_pb;
  h.v_pb = c->v_pb;
  h.cap = capacity;
  h.hyb = hyb;
  h.v_mass = v_mass;
  h.st = aq::RingState{0, 0, 0, 0};
  c->d_desc = reinterpret_cast<aq::HeadDesc *>(base + o_desc);
  c->d_desc_list = reinterpret_cast<aq::HeadDesc **>(base + o_list);

  // Zeroed codes and scales of 1.0, as KVFlatBuffer::init leaves them
  // (ring_buffer.cpp:77-83).
  hipError_t e = hipMemset(c->slab, 0, off);
  if (e == hipSuccess) e = hipMemcpy(base + o_desc, &h, sizeof(h), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(base + o_list, &c->d_desc, sizeof(void *), hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(base + o_signs, sign_words, sizeof(sign_words), hipMemcpyHostToDevice);
  if (e == hipSuccess && cap_sz > 0) {
    std::vector<float> ones(cap_sz, 1.0f);
    e = hipMemcpy(base + o_ks, ones.data(), cap_sz * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(base + o_vs, ones.data(), cap_sz * 4, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    hip_fail(e, fn);
    free_ctx(c);
    return nullptr;
  }
  return c;
}

// Quantise the staged tokens (caller holds c->mu), on the library stream.
// The rows go through pinned memory (the kernel reads small batches from it
// directly) and the call does not wait for the kernel: the next flush waits
// before it reuses the pinned rows, and compute waits for its own outputs.
// host_wait = true (inspection, snapshots) also waits until every queued
// launch of the device has completed, callers' device-form launches included.
bool flush_locked(Ctx *c, const char *fn, bool host_wait = false) {
  if (c->staged == 0 && !host_wait) return true;
  DeviceGuard g(c->device);
  if (c->staged > 0) {
    if (hip_fail(lib_wait(c->device, c->stage_seq), fn)) return false;  // pinned rows reused
    const size_t n = (size_t)c->staged * c->dim;  // floats per side
    if (hip_fail(c->h_stage.ensure(2 * n * 4), fn)) return false;
    float *pk = static_cast<float *>(c->h_stage.p);
    std::memcpy(pk, c->stage_k.data(), n * 4);
    std::memcpy(pk + n, c->stage_v.data(), n * 4);
    const float *dk = static_cast<const float *>(c->h_stage.dp);
    hipStream_t s;
    hipError_t e = lib_begin(c->device, &s);
    if (e == hipSuccess && c->staged > kDirectTokens) {
      e = c->d_stage.ensure(2 * n * 4);
      if (e == hipSuccess)
        e = hipMemcpyAsync(c->d_stage.p, c->h_stage.p, 2 * n * 4, hipMemcpyHostToDevice, s);
      dk = static_cast<const float *>(c->d_stage.p);
    }
    if (e == hipSuccess)
      e = aq::launch_append(c->d_desc_list, 1, c->dim, c->padded, c->k_bits, c->v_bits, dk, dk + n,
                            c->staged, s, aq::mirror_count(c->st, c->staged, c->cap, c->hyb) > 0);
    if (hip_fail(e, fn)) return false;
    c->stage_seq = lib_end(c->device);
    c->st = aq::ring_after(c->st, c->staged, c->cap, c->hyb);
    c->staged = 0;
    c->stage_k.clear();
    c->stage_v.clear();
  }
  if (host_wait && hip_fail(settle(c->device), fn)) return false;
  return true;
}

void append_locked(Ctx *c, const float *key, const float *val) {
  c->stage_k.insert(c->stage_k.end(), key, key + c->dim);
  c->stage_v.insert(c->stage_v.end(), val, val + c->dim);
  ++c->staged;
  bump_epoch();
  if (c->staged >= kStageTokens) flush_locked(c, "adaptq_append");
}

enum class Mode { Dense, Hybrid, Sparse };

// The branch a context with ring state st takes (attention.cpp:480-660).
Mode mode_at(const Ctx *c, const aq::RingState &st) {
  const int n = st.size;
  if (c->hyb > 0 && n <= c->hyb && st.raw_count == n) return Mode::Hybrid;
  if (c->v_mass > 0.0f && c->k_bits != 16 && c->v_bits != 16) return Mode::Sparse;
  return Mode::Dense;
}

Mode mode_of(const Ctx *c) { return mode_at(c, c->st); }

// The shape of a dense decode step over contexts like c whose rings hold n
// tokens after the step's append, when one fused launch takes it.
bool step_shape(const Ctx *c, int n_items, int n_after, aq::DecodeShape *sh) {
  *sh = aq::DecodeShape{c->dim, c->padded, c->k_bits, c->v_bits, false, n_after};
  return c->cap > 0 && aq::decode_step_supported(n_items, *sh);
}

aq::StepAppend step_rows(const Ctx *c, const float *k, const float *v) {
  const float sp = sqrtf((float)c->padded);  // as launch_append passes them
  return aq::StepAppend{k, v, 1.0f / sp, sp};
}

// The item list of nq decodes of context c (caller holds c->mu).
bool ensure_items(Ctx *c, int nq, const char *fn) {
  if (nq <= c->items_uploaded) return true;
  if (hip_fail(c->d_items.ensure(sizeof(void *) * (size_t)nq), fn)) return false;
  std::vector<aq::HeadDesc *> items((size_t)nq, c->d_desc);
  if (hip_fail(hipMemcpy(c->d_items.p, items.data(), sizeof(void *) * nq, hipMemcpyHostToDevice), fn))
    return false;
  c->items_uploaded = nq;
  return true;
}

// One staged token and one query, the reference's per-step calls
// (attention.cpp:338-366 then :480-660): append and decode in one launch
// (launch_decode_step) when the step is a dense decode the fused kernel
// takes (caller holds c->mu).  Returns -2, having changed nothing, when it
// is not; the ring size, or -1 on error, otherwise.
int step_locked(Ctx *c, const float *query, float *out, const char *fn) {
  const aq::RingState after = aq::ring_after(c->st, 1, c->cap, c->hyb);
  aq::DecodeShape sh;
  if (mode_at(c, after) != Mode::Dense || !step_shape(c, 1, after.size, &sh)) return -2;
  DeviceGuard g(c->device);
  if (hip_fail(lib_wait(c->device, c->stage_seq), fn)) return -1;  // pinned rows reused
  const size_t d = (size_t)c->dim;
  const size_t io = align256(d * 4);
  if (hip_fail(c->h_stage.ensure(2 * d * 4), fn) || hip_fail(c->h_io.ensure(2 * io), fn) ||
      !ensure_items(c, 1, fn))
    return -1;
  float *pk = static_cast<float *>(c->h_stage.p);
  std::memcpy(pk, c->stage_k.data(), d * 4);
  std::memcpy(pk + d, c->stage_v.data(), d * 4);
  const float *dk = static_cast<const float *>(c->h_stage.dp);
  std::memcpy(c->h_io.p, query, d * 4);
  const float *dq = static_cast<const float *>(c->h_io.dp);
  float *dout = reinterpret_cast<float *>(static_cast<uint8_t *>(c->h_io.dp) + io);
  hipStream_t s;
  hipError_t e = lib_begin(c->device, &s);
  if (e == hipSuccess)
    e = aq::launch_decode_step(static_cast<aq::HeadDesc **>(c->d_items.p), 1, sh,
                               step_rows(c, dk, dk + d), dq, dout, s);
  if (hip_fail(e, fn)) return -1;
  c->stage_seq = lib_end(c->device);
  c->st = after;
  c->staged = 0;
  c->stage_k.clear();
  c->stage_v.clear();
  if (hip_fail(lib_wait(c->device, c->stage_seq), fn)) return -1;
  std::memcpy(out, static_cast<uint8_t *>(c->h_io.p) + io, d * 4);
  return after.size;
}

// Synchronous decode of nq queries against one head (caller holds c->mu).
// Queries and outputs pass through pinned memory the kernels read and write.
int compute_locked(Ctx *c, const float *queries, int nq, float *outs, const char *fn) {
  if (nq == 1 && c->staged == 1) {
    const int r = step_locked(c, queries, outs, fn);
    if (r != -2) return r;
  }
  if (!flush_locked(c, fn)) return -1;
  const int n = c->st.size;
  if (n == 0) {
    std::memset(outs, 0, sizeof(float) * (size_t)nq * c->dim);
    return 0;
  }
  DeviceGuard g(c->device);
  const Mode mode = mode_of(c);
  aq::DecodeShape sh{c->dim, c->padded, c->k_bits, c->v_bits, mode == Mode::Hybrid, n};
  const size_t io = align256((size_t)nq * c->dim * 4);
  if (hip_fail(c->h_io.ensure(2 * io), fn)) return -1;  // no kernel uses it between calls
  if (!ensure_items(c, nq, fn)) return -1;
  const size_t wsf = mode == Mode::Sparse ? aq::sparse_workspace_floats(nq, sh)
                                          : aq::decode_multi_workspace_floats(nq, 1, sh);
  if (hip_fail(c->d_ws.ensure(wsf * 4), fn)) return -1;
  std::memcpy(c->h_io.p, queries, (size_t)nq * c->dim * 4);
  const float *dq = static_cast<const float *>(c->h_io.dp);
  float *dout = reinterpret_cast<float *>(static_cast<uint8_t *>(c->h_io.dp) + io);
  auto **items = static_cast<aq::HeadDesc **>(c->d_items.p);
  hipStream_t s;
  hipError_t e = lib_begin(c->device, &s);
  if (e == hipSuccess)
    e = mode == Mode::Sparse
            ? aq::launch_decode_sparse(items, nq, sh, c->v_mass, dq, dout,
                                       static_cast<float *>(c->d_ws.p), s)
            : aq::launch_decode_multi(items, nq, 1, sh, dq, dout, static_cast<float *>(c->d_ws.p), s);
  if (e == hipSuccess) e = lib_wait(c->device, lib_end(c->device));
  if (hip_fail(e, fn)) return -1;
  std::memcpy(outs, static_cast<uint8_t *>(c->h_io.p) + io, (size_t)nq * c->dim * 4);
  return n;
}

// Empties the ring (caller holds c->mu).  The state reset is queued on the
// library stream after every queued launch of the device; nothing waits.
void reset_locked(Ctx *c) {
  c->staged = 0;
  c->stage_k.clear();
  c->stage_v.clear();
  c->st = aq::RingState{0, 0, 0, 0};
  bump_epoch();
  DeviceGuard g(c->device);
  hipStream_t s;
  hipError_t e = lib_begin(c->device, &s);
  if (e == hipSuccess) e = aq::launch_reset_state(c->d_desc_list, 1, s);
  if (e == hipSuccess) (void)lib_end(c->device);
  else hip_fail(e, "adaptq_reset");
}

// A plan binds contexts for batched device-pointer calls.  It caches the
// branch and the largest ring size of its contexts together with the epoch
// they were read at; while no context has changed since (g_epoch), the
// plan's calls read neither the contexts nor their locks.
struct Plan {
  std::vector<Ctx *> ctxs;
  int device = 0;
  DevBuf d_list, d_ws;
  std::mutex mu;          // one call on the plan at a time
  uint64_t seen = 0;      // epoch the cache below was read at (0: never)
  int max_n = 0;          // largest ring size
  Mode mode = Mode::Dense;
  bool mixed = false;     // non-empty contexts take different branches
};

// Scan of the plan's contexts (caller holds p->mu): flushes staged host
// appends (library stream) and caches branch and largest ring size.  With
// flush = false (the allocation-free entry point: a flush may allocate
// staging memory) staged host appends are an error instead.
bool plan_scan(Plan *p, const char *fn, bool flush = true) {
  if (p->seen != 0 && g_epoch.load(std::memory_order_acquire) == p->seen) return true;
  const uint64_t e0 = g_epoch.load(std::memory_order_acquire);
  int max_n = 0;
  bool have = false, mixed = false;
  Mode mode = Mode::Dense;
  for (Ctx *c : p->ctxs) {
    std::lock_guard<std::mutex> g(c->mu);
    if (!flush && c->staged > 0) {
      set_errorf(fn, "a context holds staged host appends; flush it first (adaptq_flush)");
      return false;
    }
    if (!flush_locked(c, fn)) return false;
    if (c->st.size > 0) {
      const Mode m = mode_of(c);
      if (have && m != mode) mixed = true;
      mode = m;
      have = true;
    }
    max_n = std::max(max_n, c->st.size);
  }
  p->max_n = max_n;
  p->mode = mode;
  p->mixed = mixed;
  p->seen = e0;
  return true;
}

// The batched decode of a plan on stream s (caller holds p->mu and has
// scanned).  d_ws: workspace of at least ws_floats floats.
int plan_launch_decode(Plan *p, const float *d_queries, float *d_outs, float *d_ws,
                       hipStream_t s, const char *fn) {
  if (p->mixed) {
    set_error(
        "adaptq_plan_compute_device: contexts take different branches (dense, sparse-V, "
        "hybrid); use one plan per branch or adaptq_compute");
    return -1;
  }
  const Ctx *c0 = p->ctxs[0];
  const int n_items = (int)p->ctxs.size();
  aq::DecodeShape sh{c0->dim, c0->padded, c0->k_bits, c0->v_bits, p->mode == Mode::Hybrid,
                     p->max_n};
  auto **items = static_cast<aq::HeadDesc **>(p->d_list.p);
  hipError_t e = caller_begin(p->device, s);
  if (e == hipSuccess)
    e = p->mode == Mode::Sparse && p->max_n > 0
            ? aq::launch_decode_sparse(items, n_items, sh, c0->v_mass, d_queries, d_outs, d_ws, s)
            : aq::launch_decode(items, n_items, sh, d_queries, d_outs, d_ws, s);
  if (e == hipSuccess) e = caller_end(p->device, s);
  if (hip_fail(e, fn)) return -1;
  return 0;
}

size_t plan_ws_floats(const Plan *p) {
  const Ctx *c0 = p->ctxs[0];
  const int n_items = (int)p->ctxs.size();
  aq::DecodeShape sh{c0->dim, c0->padded, c0->k_bits, c0->v_bits, p->mode == Mode::Hybrid,
                     p->max_n};
  return p->mode == Mode::Sparse && p->max_n > 0 ? aq::sparse_workspace_floats(n_items, sh)
                                                 : aq::decode_workspace_floats(n_items, sh);
}

// Locks every head of an MHA in index order (per-head calls take one head
// lock only, so the order cannot deadlock against them).
struct HeadLocks {
  std::vector<std::unique_lock<std::mutex>> locks;
  explicit HeadLocks(Mha *m) {
    locks.reserve(m->heads.size());
    for (Ctx *c : m->heads) locks.emplace_back(c->mu);
  }
};

// Quantise the staged tokens of every head (caller holds all head locks).
// When every head holds the same number of staged tokens -- the usual case,
// one token per head per step -- they go out through one pinned buffer and one
// append launch over all heads.  host_wait: as flush_locked.
bool flush_all_locked(Mha *m, const char *fn, bool host_wait = false) {
  const int S = m->heads[0]->staged;
  bool uniform = S > 0;
  bool any = false;
  for (Ctx *c : m->heads) {
    uniform = uniform && c->staged == S;
    any = any || c->staged > 0;
  }
  DeviceGuard g(m->device);
  if (!any) {
    if (host_wait && hip_fail(settle(m->device), fn)) return false;
    return true;
  }
  if (!uniform) {
    for (Ctx *c : m->heads)
      if (c->staged > 0 && !flush_locked(c, fn)) return false;
    if (host_wait && hip_fail(settle(m->device), fn)) return false;
    return true;
  }
  const Ctx *c0 = m->heads[0];
  const int H = m->n_heads;
  const size_t per = (size_t)S * c0->dim;  // floats per head and side
  if (hip_fail(lib_wait(m->device, m->stage_seq), fn)) return false;  // pinned rows reused
  if (hip_fail(m->h_stage.ensure(2 * per * H * 4), fn)) return false;
  float *pk = static_cast<float *>(m->h_stage.p), *pv = pk + per * H;
  for (int h = 0; h < H; ++h) {
    std::memcpy(pk + per * h, m->heads[h]->stage_k.data(), per * 4);
    std::memcpy(pv + per * h, m->heads[h]->stage_v.data(), per * 4);
  }
  const float *dk = static_cast<const float *>(m->h_stage.dp);
  hipStream_t s;
  hipError_t e = lib_begin(m->device, &s);
  if (e == hipSuccess && S > kDirectTokens) {
    e = m->d_stage.ensure(2 * per * H * 4);
    if (e == hipSuccess)
      e = hipMemcpyAsync(m->d_stage.p, m->h_stage.p, 2 * per * H * 4, hipMemcpyHostToDevice, s);
    dk = static_cast<const float *>(m->d_stage.p);
  }
  if (e == hipSuccess)
    e = aq::launch_append(static_cast<aq::HeadDesc **>(m->d_list.p), H, c0->dim, c0->padded,
                          c0->k_bits, c0->v_bits, dk, dk + per * H, S, s, any_mirror(m->heads, S));
  if (hip_fail(e, fn)) return false;
  m->stage_seq = lib_end(m->device);
  for (Ctx *c : m->heads) {
    c->st = aq::ring_after(c->st, S, c->cap, c->hyb);
    c->staged = 0;
    c->stage_k.clear();
    c->stage_v.clear();
  }
  if (host_wait && hip_fail(settle(m->device), fn)) return false;
  return true;
}

// One decode launch over all heads of an MHA (caller holds all head locks and
// has flushed).  Returns the common ring size, or -2 when the heads differ in
// size or branch (the caller then works head by head), or -1 on error.
// Queries/outs are device pointers; the launch is asynchronous on `s`.
// With reps > 1 the launch holds reps queries per head, ordered [rep][head]
// (item r * n_heads + h is head h).
int launch_all_locked(Mha *m, const float *dq, float *dout, hipStream_t s, const char *fn,
                      int reps = 1) {
  const Ctx *c0 = m->heads[0];
  const int n = c0->st.size;
  const Mode mode = mode_of(c0);
  for (const Ctx *c : m->heads)
    if (c->st.size != n || mode_of(c) != mode) return -2;
  const int H = m->n_heads * reps;
  aq::DecodeShape sh{c0->dim, c0->padded, c0->k_bits, c0->v_bits, mode == Mode::Hybrid,
                     n > 0 ? n : 1};
  const size_t wsf = mode == Mode::Sparse ? aq::sparse_workspace_floats(H, sh)
                                          : aq::decode_multi_workspace_floats(H, m->n_heads, sh);
  if (hip_fail(m->d_ws.ensure(wsf * 4), fn)) return -1;
  auto **items = static_cast<aq::HeadDesc **>(m->d_list.p);
  if (reps > 1) {
    if (m->rep_n != reps) {
      std::vector<aq::HeadDesc *> list((size_t)H);
      for (int i = 0; i < H; ++i) list[i] = m->heads[i % m->n_heads]->d_desc;
      m->rep_n = 0;
      if (hip_fail(m->d_rep.ensure(list.size() * sizeof(void *)), fn)) return -1;
      if (hip_fail(hipMemcpyAsync(m->d_rep.p, list.data(), list.size() * sizeof(void *),
                                  hipMemcpyHostToDevice, s),
                   fn) ||
          hip_fail(hipStreamSynchronize(s), fn))
        return -1;
      m->rep_n = reps;
    }
    items = static_cast<aq::HeadDesc **>(m->d_rep.p);
  }
  hipError_t e;
  if (n == 0)  // the decode kernels write zeros for empty rings
    e = aq::launch_decode(items, H, sh, dq, dout, static_cast<float *>(m->d_ws.p), s);
  else if (mode == Mode::Sparse)
    e = aq::launch_decode_sparse(items, H, sh, c0->v_mass, dq, dout,
                                 static_cast<float *>(m->d_ws.p), s);
  else  // reps queries per head: the multi-query kernel once there are enough
    e = aq::launch_decode_multi(items, H, m->n_heads, sh, dq, dout,
                                static_cast<float *>(m->d_ws.p), s);
  if (hip_fail(e, fn)) return -1;
  return n;
}

// A decode step over every head of an MHA whose heads each take one token
// (rows k, v [n_heads][dim], device or pinned memory) and one query: one
// fused launch (launch_decode_step) when every head's ring holds the same
// number of tokens after the append and the step is a dense decode the fused
// kernel takes (caller holds all head locks, nothing staged).  Returns -2,
// having launched nothing, when it is not; the common ring size, or -1.
int step_all_locked(Mha *m, const float *dk, const float *dv, const float *dq, float *dout,
                    hipStream_t s, const char *fn) {
  const Ctx *c0 = m->heads[0];
  const aq::RingState a0 = aq::ring_after(c0->st, 1, c0->cap, c0->hyb);
  for (const Ctx *c : m->heads) {
    const aq::RingState a = aq::ring_after(c->st, 1, c->cap, c->hyb);
    if (c->staged != 0 || a.size != a0.size || mode_at(c, a) != Mode::Dense) return -2;
  }
  aq::DecodeShape sh;
  if (!step_shape(c0, m->n_heads, a0.size, &sh)) return -2;
  if (hip_fail(aq::launch_decode_step(static_cast<aq::HeadDesc **>(m->d_list.p), m->n_heads, sh,
                                      step_rows(c0, dk, dv), dq, dout, s),
               fn))
    return -1;
  for (Ctx *c : m->heads) c->st = aq::ring_after(c->st, 1, c->cap, c->hyb);
  bump_epoch();
  return a0.size;
}

}  // namespace

extern "C" {

const char *adaptq_last_error(void) { return tl_error; }

adaptq_ctx_t adaptq_create(int dim, int k_bits, int v_bits, int capacity, uint64_t seed,
                           float v_mass, int hybrid_thresh) {
  if (dim <= 0 || !valid_bits(k_bits) || !valid_bits(v_bits) || capacity < 0 ||
      hybrid_thresh < 0) {
    set_error("adaptq_create: invalid dimensions or capacity");
    return nullptr;
  }
  return create_ctx(dim, k_bits, v_bits, capacity, seed, v_mass, hybrid_thresh, "adaptq_create");
}

void adaptq_destroy(adaptq_ctx_t h) { free_ctx(static_cast<Ctx *>(h)); }

void adaptq_append(adaptq_ctx_t h, const float *key, const float *val, int token_pos) {
  (void)token_pos;
  if (!require_handle(h, "adaptq_append") || !require_pointer(key, "adaptq_append", "key") ||
      !require_pointer(val, "adaptq_append", "val"))
    return;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  append_locked(c, key, val);
}

int adaptq_compute(adaptq_ctx_t h, const float *query, float *out) {
  if (!require_handle(h, "adaptq_compute") || !require_pointer(query, "adaptq_compute", "query") ||
      !require_pointer(out, "adaptq_compute", "out"))
    return -1;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  return compute_locked(c, query, 1, out, "adaptq_compute");
}

int adaptq_compute_batch(adaptq_ctx_t h, const float *queries, int num_queries, float *outs) {
  if (!require_handle(h, "adaptq_compute_batch")) return -1;
  if (num_queries < 0) {
    set_error("adaptq_compute_batch: negative num_queries");
    return -1;
  }
  if (num_queries > 0 && (!require_pointer(queries, "adaptq_compute_batch", "queries") ||
                          !require_pointer(outs, "adaptq_compute_batch", "outs")))
    return -1;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  if (num_queries == 0) {
    if (!flush_locked(c, "adaptq_compute_batch")) return -1;
    return c->st.size;
  }
  return compute_locked(c, queries, num_queries, outs, "adaptq_compute_batch");
}

void adaptq_reset(adaptq_ctx_t h) {
  if (!require_handle(h, "adaptq_reset")) return;
  Ctx *c = static_cast<Ctx *>(h);
  {
    std::lock_guard<std::mutex> g(c->mu);
    reset_locked(c);
  }
  clear_error();
}

size_t adaptq_kv_bytes(adaptq_ctx_t h) {
  if (!require_handle(h, "adaptq_kv_bytes")) return 0;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  aq::RingState s = aq::ring_after(c->st, c->staged, c->cap, c->hyb);
  return (size_t)s.size * (size_t)(c->k_pb + c->v_pb);
}

adaptq_mha_t adaptq_mha_create(int n_heads, int dim, int k_bits, int v_bits, int capacity,
                               uint64_t base_seed, float v_mass, int hybrid_thresh) {
  if (n_heads <= 0 || dim <= 0 || !valid_bits(k_bits) || !valid_bits(v_bits) || capacity < 0 ||
      hybrid_thresh < 0) {
    set_error("adaptq_mha_create: invalid parameters");
    return nullptr;
  }
  Mha *m = new (std::nothrow) Mha();
  if (!m) {
    set_error("adaptq_mha_create: host allocation failed");
    return nullptr;
  }
  m->n_heads = n_heads;
  m->heads.reserve(n_heads);
  for (int i = 0; i < n_heads; ++i) {
    const uint64_t seed = base_seed ^ ((uint64_t)i * 0xDEADBEEFCAFEULL);
    Ctx *c = create_ctx(dim, k_bits, v_bits, capacity, seed, v_mass, hybrid_thresh,
                        "adaptq_mha_create");
    if (!c) {
      for (Ctx *x : m->heads) free_ctx(x);
      delete m;
      return nullptr;
    }
    m->heads.push_back(c);
  }
  m->device = m->heads[0]->device;
  std::vector<aq::HeadDesc *> list((size_t)n_heads);
  for (int i = 0; i < n_heads; ++i) list[i] = m->heads[i]->d_desc;
  {
    DeviceGuard g(m->device);
    if (hip_fail(m->d_list.ensure(sizeof(void *) * (size_t)n_heads), "adaptq_mha_create") ||
        hip_fail(hipMemcpy(m->d_list.p, list.data(), sizeof(void *) * n_heads,
                           hipMemcpyHostToDevice),
                 "adaptq_mha_create")) {
      adaptq_mha_destroy(m);
      return nullptr;
    }
  }
  return m;
}

void adaptq_mha_destroy(adaptq_mha_t h) {
  if (!h) return;
  Mha *m = static_cast<Mha *>(h);
  {
    DeviceGuard g(m->device);
    (void)settle(m->device);  // no queued kernel may still use the heads or pinned rows
  }
  for (Ctx *c : m->heads) free_ctx(c);
  {
    DeviceGuard g(m->device);
    m->h_stage.release();
    m->h_io.release();
    m->d_list.release();
    m->d_rep.release();
    m->d_ws.release();
    m->d_io.release();
    m->d_stage.release();
  }
  delete m;
}

void adaptq_mha_append(adaptq_mha_t h, int head_idx, const float *key, const float *val,
                       int token_pos) {
  if (!require_handle(h, "adaptq_mha_append")) return;
  Mha *m = static_cast<Mha *>(h);
  if (head_idx < 0 || head_idx >= m->n_heads) {
    set_error("adaptq_mha_append: head_idx out of range");
    return;
  }
  if (!require_pointer(key, "adaptq_mha_append", "key") ||
      !require_pointer(val, "adaptq_mha_append", "val"))
    return;
  clear_error();
  adaptq_append(m->heads[head_idx], key, val, token_pos);
}

int adaptq_mha_compute(adaptq_mha_t h, int head_idx, const float *query, float *out) {
  if (!require_handle(h, "adaptq_mha_compute")) return -1;
  Mha *m = static_cast<Mha *>(h);
  if (head_idx < 0 || head_idx >= m->n_heads) {
    set_error("adaptq_mha_compute: head_idx out of range");
    return -1;
  }
  if (!require_pointer(query, "adaptq_mha_compute", "query") ||
      !require_pointer(out, "adaptq_mha_compute", "out"))
    return -1;
  clear_error();
  return adaptq_compute(m->heads[head_idx], query, out);
}

int adaptq_mha_compute_batch(adaptq_mha_t h, int head_idx, const float *queries,
                             int num_queries, float *outs) {
  if (!require_handle(h, "adaptq_mha_compute_batch")) return -1;
  Mha *m = static_cast<Mha *>(h);
  if (head_idx < 0 || head_idx >= m->n_heads) {
    set_error("adaptq_mha_compute_batch: head_idx out of range");
    return -1;
  }
  if (num_queries < 0) {
    set_error("adaptq_mha_compute_batch: negative num_queries");
    return -1;
  }
  if (num_queries > 0 && (!require_pointer(queries, "adaptq_mha_compute_batch", "queries") ||
                          !require_pointer(outs, "adaptq_mha_compute_batch", "outs")))
    return -1;
  clear_error();
  return adaptq_compute_batch(m->heads[head_idx], queries, num_queries, outs);
}

void adaptq_mha_reset(adaptq_mha_t h) {
  if (!require_handle(h, "adaptq_mha_reset")) return;
  Mha *m = static_cast<Mha *>(h);
  {
    std::lock_guard<std::mutex> gm(m->mu);
    HeadLocks locks(m);
    for (Ctx *c : m->heads) {
      c->staged = 0;
      c->stage_k.clear();
      c->stage_v.clear();
      c->st = aq::RingState{0, 0, 0, 0};
    }
    bump_epoch();
    // one state reset for every head, queued after the device's queued launches
    DeviceGuard g(m->device);
    hipStream_t s;
    hipError_t e = lib_begin(m->device, &s);
    if (e == hipSuccess)
      e = aq::launch_reset_state(static_cast<aq::HeadDesc **>(m->d_list.p), m->n_heads, s);
    if (e == hipSuccess) (void)lib_end(m->device);
    if (hip_fail(e, "adaptq_mha_reset")) return;
  }
  clear_error();
}

size_t adaptq_mha_total_kv_bytes(adaptq_mha_t h) {
  if (!require_handle(h, "adaptq_mha_total_kv_bytes")) return 0;
  Mha *m = static_cast<Mha *>(h);
  size_t total = 0;
  for (Ctx *c : m->heads) total += adaptq_kv_bytes(c);
  return total;
}

unsigned int adaptq_features(void) {
  return ADAPTQ_FEAT_HYBRID | ADAPTQ_FEAT_SPARSE_V | ADAPTQ_FEAT_HIP;
}

const char *adaptq_version(void) { return "3.2.0-hip-gfx950"; }

// ---- extensions ----

int adaptq_mha_append_all(adaptq_mha_t h, const float *keys, const float *vals, int token_pos) {
  (void)token_pos;
  const char *fn = "adaptq_mha_append_all";
  if (!require_handle(h, fn) || !require_pointer(keys, fn, "keys") ||
      !require_pointer(vals, fn, "vals"))
    return -1;
  Mha *m = static_cast<Mha *>(h);
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  const int dim = m->heads[0]->dim;
  for (int i = 0; i < m->n_heads; ++i) {
    Ctx *c = m->heads[i];
    c->stage_k.insert(c->stage_k.end(), keys + (size_t)i * dim, keys + (size_t)(i + 1) * dim);
    c->stage_v.insert(c->stage_v.end(), vals + (size_t)i * dim, vals + (size_t)(i + 1) * dim);
    ++c->staged;
  }
  bump_epoch();
  if (m->heads[0]->staged >= kStageTokens && !flush_all_locked(m, fn)) return -1;
  clear_error();
  return 0;
}

int adaptq_mha_compute_all(adaptq_mha_t h, const float *queries, float *outs) {
  const char *fn = "adaptq_mha_compute_all";
  if (!require_handle(h, fn) || !require_pointer(queries, fn, "queries") ||
      !require_pointer(outs, fn, "outs"))
    return -1;
  Mha *m = static_cast<Mha *>(h);
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  const int H = m->n_heads, dim = m->heads[0]->dim;
  DeviceGuard g(m->device);
  // one staged token per head (the Engine's decode step): the append rides in
  // the decode launch when the step allows it
  bool step = true;
  for (const Ctx *c : m->heads) step = step && c->staged == 1;
  const float *sk = nullptr;
  if (step) {
    if (hip_fail(lib_wait(m->device, m->stage_seq), fn)) return -1;  // pinned rows reused
    if (hip_fail(m->h_stage.ensure(2 * (size_t)H * dim * 4), fn)) return -1;
    float *pk = static_cast<float *>(m->h_stage.p);
    for (int i = 0; i < H; ++i) {
      std::memcpy(pk + (size_t)i * dim, m->heads[i]->stage_k.data(), (size_t)dim * 4);
      std::memcpy(pk + (size_t)(H + i) * dim, m->heads[i]->stage_v.data(), (size_t)dim * 4);
    }
    sk = static_cast<const float *>(m->h_stage.dp);
  }
  // queries and outputs through pinned memory the kernels read and write
  const size_t io = align256((size_t)H * dim * 4);
  if (hip_fail(m->h_io.ensure(2 * io), fn)) return -1;  // no kernel uses it between calls
  std::memcpy(m->h_io.p, queries, (size_t)H * dim * 4);
  const float *dq = static_cast<const float *>(m->h_io.dp);
  float *dout = reinterpret_cast<float *>(static_cast<uint8_t *>(m->h_io.dp) + io);
  if (step) {
    // the staged rows were copied out: the heads hold nothing staged while
    // the step is tried, and take the rows back when it does not run
    std::vector<int> held((size_t)H);
    for (int i = 0; i < H; ++i) {
      held[i] = m->heads[i]->staged;
      m->heads[i]->staged = 0;
    }
    hipStream_t s;
    int n = hip_fail(lib_begin(m->device, &s), fn)
                ? -1
                : step_all_locked(m, sk, sk + (size_t)H * dim, dq, dout, s, fn);
    if (n >= 0) {
      m->stage_seq = lib_end(m->device);
      for (Ctx *c : m->heads) {
        c->stage_k.clear();
        c->stage_v.clear();
      }
      if (hip_fail(lib_wait(m->device, m->stage_seq), fn)) return -1;
      std::memcpy(outs, static_cast<uint8_t *>(m->h_io.p) + io, (size_t)H * dim * 4);
      clear_error();
      return n;
    }
    for (int i = 0; i < H; ++i) m->heads[i]->staged = held[i];
    if (n == -1) return -1;
  }
  if (!flush_all_locked(m, fn)) return -1;
  hipStream_t s;
  if (hip_fail(lib_begin(m->device, &s), fn)) return -1;
  int n = launch_all_locked(m, dq, dout, s, fn);
  if (n == -2) {  // heads differ in size or branch: one head at a time
    n = 0;
    for (int i = 0; i < H; ++i) {
      const int r = compute_locked(m->heads[i], queries + (size_t)i * dim, 1,
                                   outs + (size_t)i * dim, fn);
      if (r < 0) return -1;
      if (i == 0) n = r;
    }
    clear_error();
    return n;
  }
  if (n < 0) return -1;
  if (hip_fail(lib_wait(m->device, lib_end(m->device)), fn)) return -1;
  std::memcpy(outs, static_cast<uint8_t *>(m->h_io.p) + io, (size_t)H * dim * 4);
  clear_error();
  return n;
}

int adaptq_mha_append_all_device(adaptq_mha_t h, const float *d_keys, const float *d_vals,
                                 int n_tokens, int first_pos, void *stream) {
  (void)first_pos;
  const char *fn = "adaptq_mha_append_all_device";
  if (!require_handle(h, fn) || !require_pointer(d_keys, fn, "d_keys") ||
      !require_pointer(d_vals, fn, "d_vals"))
    return -1;
  if (n_tokens < 0) {
    set_error("adaptq_mha_append_all_device: negative n_tokens");
    return -1;
  }
  Mha *m = static_cast<Mha *>(h);
  if (n_tokens == 0) return 0;
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  if (!flush_all_locked(m, fn)) return -1;
  const Ctx *c0 = m->heads[0];
  DeviceGuard g(m->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = caller_begin(m->device, s);
  if (e == hipSuccess)
    e = aq::launch_append(static_cast<aq::HeadDesc **>(m->d_list.p), m->n_heads, c0->dim,
                          c0->padded, c0->k_bits, c0->v_bits, d_keys, d_vals, n_tokens, s,
                          any_mirror(m->heads, n_tokens));
  if (e == hipSuccess) e = caller_end(m->device, s);
  if (hip_fail(e, fn)) return -1;
  for (Ctx *c : m->heads) c->st = aq::ring_after(c->st, n_tokens, c->cap, c->hyb);
  bump_epoch();
  return 0;
}

int adaptq_mha_compute_all_device(adaptq_mha_t h, const float *d_queries, float *d_outs,
                                  void *stream) {
  const char *fn = "adaptq_mha_compute_all_device";
  if (!require_handle(h, fn) || !require_pointer(d_queries, fn, "d_queries") ||
      !require_pointer(d_outs, fn, "d_outs"))
    return -1;
  Mha *m = static_cast<Mha *>(h);
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  if (!flush_all_locked(m, fn)) return -1;
  DeviceGuard g(m->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hip_fail(caller_begin(m->device, s), fn)) return -1;
  const int n = launch_all_locked(m, d_queries, d_outs, s, fn);
  if (n == -2) {
    set_error("adaptq_mha_compute_all_device: heads differ in ring size or branch; "
              "use adaptq_mha_compute_all");
    return -1;
  }
  if (n >= 0 && hip_fail(caller_end(m->device, s), fn)) return -1;
  return n;
}

int adaptq_mha_append_compute_all_device(adaptq_mha_t h, const float *d_keys,
                                         const float *d_vals, int token_pos,
                                         const float *d_queries, float *d_outs, void *stream) {
  (void)token_pos;
  const char *fn = "adaptq_mha_append_compute_all_device";
  if (!require_handle(h, fn) || !require_pointer(d_keys, fn, "d_keys") ||
      !require_pointer(d_vals, fn, "d_vals") || !require_pointer(d_queries, fn, "d_queries") ||
      !require_pointer(d_outs, fn, "d_outs"))
    return -1;
  Mha *m = static_cast<Mha *>(h);
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  if (!flush_all_locked(m, fn)) return -1;
  DeviceGuard g(m->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hip_fail(caller_begin(m->device, s), fn)) return -1;
  int n = step_all_locked(m, d_keys, d_vals, d_queries, d_outs, s, fn);
  if (n == -2) {  // the append and the decode as two launches
    const Ctx *c0 = m->heads[0];
    if (hip_fail(aq::launch_append(static_cast<aq::HeadDesc **>(m->d_list.p), m->n_heads, c0->dim,
                                   c0->padded, c0->k_bits, c0->v_bits, d_keys, d_vals, 1, s,
                                   any_mirror(m->heads, 1)),
                 fn))
      return -1;
    for (Ctx *c : m->heads) c->st = aq::ring_after(c->st, 1, c->cap, c->hyb);
    bump_epoch();
    n = launch_all_locked(m, d_queries, d_outs, s, fn);
    if (n == -2) {
      (void)caller_end(m->device, s);
      set_error("adaptq_mha_append_compute_all_device: heads differ in ring size or branch "
                "(the token was appended); use adaptq_mha_compute_all");
      return -1;
    }
  }
  if (n >= 0 && hip_fail(caller_end(m->device, s), fn)) return -1;
  return n;
}

// ---- ggml operator forms (GGML_OP_ADAPTQ_APPEND / GGML_OP_ADAPTQ_ATTN) ----

}  // extern "C"

namespace {

// Shape and stride checks shared by the ggml forms: dims must match the MHA,
// strides are byte strides of f32 rows (multiples of 4).
bool ggml_shape_ok(Mha *m, int head_dim, int n_heads, int n_rows, const size_t *strides,
                   int n_strides, const char *fn) {
  if (head_dim != m->heads[0]->dim || n_heads != m->n_heads) {
    set_errorf(fn, "tensor shape does not match the MHA (head_dim, n_heads)");
    return false;
  }
  if (n_rows < 0) {
    set_errorf(fn, "negative token or query count");
    return false;
  }
  for (int i = 0; i < n_strides; ++i)
    if (strides[i] % 4 != 0) {
      set_errorf(fn, "strides must be multiples of 4 bytes (f32 rows)");
      return false;
    }
  return true;
}

const float *row_at(const float *base, size_t a, size_t sa, size_t b, size_t sb) {
  return reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(base) + a * sa + b * sb);
}

}  // namespace

extern "C" {

int adaptq_ggml_append_f32(adaptq_mha_t h, const float *k, const float *v, int head_dim,
                           int n_heads, int n_tokens, size_t k_nb1, size_t k_nb2, size_t v_nb1,
                           size_t v_nb2, int first_pos) {
  (void)first_pos;
  const char *fn = "adaptq_ggml_append_f32";
  if (!require_handle(h, fn)) return -1;
  Mha *m = static_cast<Mha *>(h);
  const size_t st[4] = {k_nb1, k_nb2, v_nb1, v_nb2};
  if (!ggml_shape_ok(m, head_dim, n_heads, n_tokens, st, 4, fn)) return -1;
  if (n_tokens == 0) return 0;
  if (!require_pointer(k, fn, "k") || !require_pointer(v, fn, "v")) return -1;
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  for (int t = 0; t < n_tokens; ++t) {
    for (int i = 0; i < m->n_heads; ++i) {
      Ctx *c = m->heads[i];
      const float *kr = row_at(k, (size_t)i, k_nb1, (size_t)t, k_nb2);
      const float *vr = row_at(v, (size_t)i, v_nb1, (size_t)t, v_nb2);
      c->stage_k.insert(c->stage_k.end(), kr, kr + head_dim);
      c->stage_v.insert(c->stage_v.end(), vr, vr + head_dim);
      ++c->staged;
    }
    bump_epoch();
    if (m->heads[0]->staged >= kStageTokens && !flush_all_locked(m, fn)) return -1;
  }
  clear_error();
  return 0;
}

int adaptq_ggml_attn_f32(adaptq_mha_t h, const float *q, int head_dim, int n_heads, int n_queries,
                         size_t q_nb1, size_t q_nb2, float *dst, size_t d_nb1, size_t d_nb2) {
  const char *fn = "adaptq_ggml_attn_f32";
  if (!require_handle(h, fn)) return -1;
  Mha *m = static_cast<Mha *>(h);
  const size_t st[4] = {q_nb1, q_nb2, d_nb1, d_nb2};
  if (!ggml_shape_ok(m, head_dim, n_heads, n_queries, st, 4, fn)) return -1;
  if (n_queries > 0 && (!require_pointer(q, fn, "q") || !require_pointer(dst, fn, "dst")))
    return -1;
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  // the decode runs on the library stream after the flush's launches
  if (!flush_all_locked(m, fn)) return -1;
  const int H = m->n_heads, dim = head_dim;
  if (n_queries == 0) {
    clear_error();
    return m->heads[0]->st.size;
  }
  DeviceGuard g(m->device);
  // queries packed [query][head][dim] into pinned memory the kernels read;
  // outputs come back there in the same order
  const size_t rows = (size_t)n_queries * H;
  const size_t io = align256(rows * dim * 4);
  if (hip_fail(m->h_io.ensure(2 * io), fn)) return -1;  // no kernel uses it between calls
  float *pq = static_cast<float *>(m->h_io.p);
  float *po = reinterpret_cast<float *>(static_cast<uint8_t *>(m->h_io.p) + io);
  for (int j = 0; j < n_queries; ++j)
    for (int i = 0; i < H; ++i)
      std::memcpy(pq + ((size_t)j * H + i) * dim, row_at(q, (size_t)i, q_nb1, (size_t)j, q_nb2),
                  (size_t)dim * 4);
  const float *dq = static_cast<const float *>(m->h_io.dp);
  float *dout = reinterpret_cast<float *>(static_cast<uint8_t *>(m->h_io.dp) + io);
  hipStream_t s;
  if (hip_fail(lib_begin(m->device, &s), fn)) return -1;
  int n = launch_all_locked(m, dq, dout, s, fn, n_queries);
  if (n == -2) {  // heads differ in size or branch: head by head, all queries of a head at once
    std::vector<float> hq((size_t)n_queries * dim), ho((size_t)n_queries * dim);
    for (int i = 0; i < H; ++i) {
      for (int j = 0; j < n_queries; ++j)
        std::memcpy(hq.data() + (size_t)j * dim, pq + ((size_t)j * H + i) * dim, (size_t)dim * 4);
      const int r = compute_locked(m->heads[i], hq.data(), n_queries, ho.data(), fn);
      if (r < 0) return -1;
      if (i == 0) n = r;
      for (int j = 0; j < n_queries; ++j)
        std::memcpy(po + ((size_t)j * H + i) * dim, ho.data() + (size_t)j * dim, (size_t)dim * 4);
    }
  } else {
    if (n < 0) return -1;
    if (hip_fail(lib_wait(m->device, lib_end(m->device)), fn)) return -1;
  }
  for (int j = 0; j < n_queries; ++j)
    for (int i = 0; i < H; ++i)
      std::memcpy(const_cast<float *>(row_at(dst, (size_t)i, d_nb1, (size_t)j, d_nb2)),
                  po + ((size_t)j * H + i) * dim, (size_t)dim * 4);
  clear_error();
  return n;
}

int adaptq_ggml_append_f32_device(adaptq_mha_t h, const float *d_k, const float *d_v,
                                  int head_dim, int n_heads, int n_tokens, size_t k_nb1,
                                  size_t k_nb2, size_t v_nb1, size_t v_nb2, int first_pos,
                                  void *stream) {
  (void)first_pos;
  const char *fn = "adaptq_ggml_append_f32_device";
  if (!require_handle(h, fn)) return -1;
  Mha *m = static_cast<Mha *>(h);
  const size_t st[4] = {k_nb1, k_nb2, v_nb1, v_nb2};
  if (!ggml_shape_ok(m, head_dim, n_heads, n_tokens, st, 4, fn)) return -1;
  if (n_tokens == 0) return 0;
  if (!require_pointer(d_k, fn, "d_k") || !require_pointer(d_v, fn, "d_v")) return -1;
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  if (!flush_all_locked(m, fn)) return -1;
  const Ctx *c0 = m->heads[0];
  const int H = m->n_heads;
  DeviceGuard g(m->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // [head][token][dim] rows for the append launch
  const size_t half = align256((size_t)H * n_tokens * head_dim * 4);
  if (hip_fail(m->d_stage.ensure(2 * half), fn)) return -1;
  float *dk = static_cast<float *>(m->d_stage.p);
  float *dv = reinterpret_cast<float *>(static_cast<uint8_t *>(m->d_stage.p) + half);
  hipError_t e = caller_begin(m->device, s);
  if (e == hipSuccess) e = aq::launch_gather_rows(dk, d_k, H, n_tokens, head_dim, k_nb1, k_nb2, s);
  if (e == hipSuccess) e = aq::launch_gather_rows(dv, d_v, H, n_tokens, head_dim, v_nb1, v_nb2, s);
  if (e == hipSuccess)
    e = aq::launch_append(static_cast<aq::HeadDesc **>(m->d_list.p), H, c0->dim, c0->padded,
                          c0->k_bits, c0->v_bits, dk, dv, n_tokens, s, any_mirror(m->heads, n_tokens));
  if (e == hipSuccess) e = caller_end(m->device, s);
  if (hip_fail(e, fn)) return -1;
  for (Ctx *c : m->heads) c->st = aq::ring_after(c->st, n_tokens, c->cap, c->hyb);
  bump_epoch();
  return 0;
}

int adaptq_ggml_attn_f32_device(adaptq_mha_t h, const float *d_q, int head_dim, int n_heads,
                                int n_queries, size_t q_nb1, size_t q_nb2, float *d_dst,
                                size_t d_nb1, size_t d_nb2, void *stream) {
  const char *fn = "adaptq_ggml_attn_f32_device";
  if (!require_handle(h, fn)) return -1;
  Mha *m = static_cast<Mha *>(h);
  const size_t st[4] = {q_nb1, q_nb2, d_nb1, d_nb2};
  if (!ggml_shape_ok(m, head_dim, n_heads, n_queries, st, 4, fn)) return -1;
  if (n_queries > 0 && (!require_pointer(d_q, fn, "d_q") || !require_pointer(d_dst, fn, "d_dst")))
    return -1;
  std::lock_guard<std::mutex> gm(m->mu);
  HeadLocks locks(m);
  if (!flush_all_locked(m, fn)) return -1;
  if (n_queries == 0) return m->heads[0]->st.size;
  const int H = m->n_heads;
  DeviceGuard g(m->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t rows = (size_t)n_queries * H;
  const size_t io = align256(rows * head_dim * 4);
  if (hip_fail(m->d_io.ensure(2 * io), fn)) return -1;
  float *dq = static_cast<float *>(m->d_io.p);
  float *dout = reinterpret_cast<float *>(static_cast<uint8_t *>(m->d_io.p) + io);
  // queries as [query][head][dim]
  if (hip_fail(caller_begin(m->device, s), fn) ||
      hip_fail(aq::launch_gather_rows(dq, d_q, n_queries, H, head_dim, q_nb2, q_nb1, s), fn))
    return -1;
  const int n = launch_all_locked(m, dq, dout, s, fn, n_queries);
  if (n == -2) {
    set_error("adaptq_ggml_attn_f32_device: heads differ in ring size or branch; "
              "use adaptq_ggml_attn_f32");
    return -1;
  }
  if (n < 0) return -1;
  if (hip_fail(aq::launch_scatter_rows(d_dst, dout, n_queries, H, head_dim, d_nb2, d_nb1, s), fn) ||
      hip_fail(caller_end(m->device, s), fn))
    return -1;
  return n;
}

int adaptq_flush(adaptq_ctx_t h) {
  if (!require_handle(h, "adaptq_flush")) return -1;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  return flush_locked(c, "adaptq_flush", true) ? 0 : -1;
}

int adaptq_ring_info(adaptq_ctx_t h, int *head, int *size, int *capacity, int *padded_dim,
                     int *k_packed_bytes, int *v_packed_bytes) {
  if (!require_handle(h, "adaptq_ring_info")) return -1;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  if (!flush_locked(c, "adaptq_ring_info")) return -1;
  if (head) *head = c->st.head;
  if (size) *size = c->st.size;
  if (capacity) *capacity = c->cap;
  if (padded_dim) *padded_dim = c->padded;
  if (k_packed_bytes) *k_packed_bytes = c->k_pb;
  if (v_packed_bytes) *v_packed_bytes = c->v_pb;
  return 0;
}

int adaptq_read_slots(adaptq_ctx_t h, int first_slot, int count, uint8_t *k_codes,
                      uint8_t *v_codes, float *k_scale, float *v_scale) {
  if (!require_handle(h, "adaptq_read_slots")) return -1;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  if (first_slot < 0 || count < 0 || (long long)first_slot + count > c->cap) {
    set_error("adaptq_read_slots: slot range out of bounds");
    return -1;
  }
  // every queued launch of the device (callers' included) completes first
  if (!flush_locked(c, "adaptq_read_slots", true)) return -1;
  if (count == 0) return 0;
  DeviceGuard g2(c->device);
  const aq::HeadDesc &hd = c->hd;
  hipError_t e = hipSuccess;
  if (e == hipSuccess && k_codes)
    e = hipMemcpy(k_codes, hd.k_codes + (size_t)first_slot * c->k_pb, (size_t)count * c->k_pb,
                  hipMemcpyDeviceToHost);
  if (e == hipSuccess && v_codes)
    e = hipMemcpy(v_codes, hd.v_codes + (size_t)first_slot * c->v_pb, (size_t)count * c->v_pb,
                  hipMemcpyDeviceToHost);
  if (e == hipSuccess && k_scale)
    e = hipMemcpy(k_scale, hd.k_scale + first_slot, (size_t)count * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && v_scale)
    e = hipMemcpy(v_scale, hd.v_scale + first_slot, (size_t)count * 4, hipMemcpyDeviceToHost);
  if (hip_fail(e, "adaptq_read_slots")) return -1;
  // K rows stored in XOR byte order go back to the reference's order
  const int xmask = aq::kperm_mask(c->padded, c->k_bits);
  if (k_codes && xmask) {
    uint8_t tmp[64];
    for (int r = 0; r < count; ++r) {
      uint8_t *row = k_codes + (size_t)r * c->k_pb;
      const int x = (first_slot + r) & xmask;
      for (int j = 0; j < c->k_pb; ++j) tmp[j] = row[j ^ x];
      std::memcpy(row, tmp, (size_t)c->k_pb);
    }
  }
  return 0;
}

int adaptq_sparse_weights(adaptq_ctx_t h, const float *query, float *weights) {
  const char *fn = "adaptq_sparse_weights";
  if (!require_handle(h, fn) || !require_pointer(query, fn, "query") ||
      !require_pointer(weights, fn, "weights"))
    return -1;
  Ctx *c = static_cast<Ctx *>(h);
  std::lock_guard<std::mutex> g(c->mu);
  if (!flush_locked(c, fn)) return -1;
  if (c->st.size == 0) return 0;
  if (mode_of(c) != Mode::Sparse) {
    set_errorf(fn, "the context does not take the sparse-V branch");
    return -1;
  }
  std::vector<float> out((size_t)c->dim);
  const int n = compute_locked(c, query, 1, out.data(), fn);
  if (n < 0) return -1;
  // every sparse-V launch leaves item 0's per-token weights (ring order) at
  // the start of the workspace, and compute_locked has waited for it
  DeviceGuard g2(c->device);
  if (hip_fail(hipMemcpy(weights, c->d_ws.p, (size_t)n * 4, hipMemcpyDeviceToHost), fn)) return -1;
  return n;
}

adaptq_ctx_t adaptq_mha_head(adaptq_mha_t h, int head_idx) {
  if (!require_handle(h, "adaptq_mha_head")) return nullptr;
  Mha *m = static_cast<Mha *>(h);
  if (head_idx < 0 || head_idx >= m->n_heads) {
    set_error("adaptq_mha_head: head_idx out of range");
    return nullptr;
  }
  return m->heads[head_idx];
}

adaptq_plan_t adaptq_plan_create(const adaptq_ctx_t *ctxs, int n_ctx) {
  const char *fn = "adaptq_plan_create";
  if (!require_pointer(ctxs, fn, "ctxs")) return nullptr;
  if (n_ctx <= 0) {
    set_error("adaptq_plan_create: n_ctx must be positive");
    return nullptr;
  }
  Plan *p = new (std::nothrow) Plan();
  if (!p) {
    set_error("adaptq_plan_create: host allocation failed");
    return nullptr;
  }
  std::vector<aq::HeadDesc *> list((size_t)n_ctx);
  for (int i = 0; i < n_ctx; ++i) {
    Ctx *c = static_cast<Ctx *>(ctxs[i]);
    if (!c) {
      delete p;
      set_error("adaptq_plan_create: null context");
      return nullptr;
    }
    const Ctx *c0 = static_cast<Ctx *>(ctxs[0]);
    if (c->dim != c0->dim || c->k_bits != c0->k_bits || c->v_bits != c0->v_bits ||
        c->cap != c0->cap || c->hyb != c0->hyb || c->v_mass != c0->v_mass ||
        c->device != c0->device) {
      delete p;
      set_error("adaptq_plan_create: contexts differ in shape, bits, capacity, mode or device");
      return nullptr;
    }
    p->ctxs.push_back(c);
    list[i] = c->d_desc;
  }
  {
    // a context twice would take two slots from one ring state
    std::vector<Ctx *> sorted(p->ctxs);
    std::sort(sorted.begin(), sorted.end());
    if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end()) {
      delete p;
      set_error("adaptq_plan_create: a context appears more than once");
      return nullptr;
    }
  }
  p->device = p->ctxs[0]->device;
  DeviceGuard g(p->device);
  if (hip_fail(p->d_list.ensure(sizeof(void *) * (size_t)n_ctx), fn) ||
      hip_fail(hipMemcpy(p->d_list.p, list.data(), sizeof(void *) * n_ctx, hipMemcpyHostToDevice), fn)) {
    p->d_list.release();
    delete p;
    return nullptr;
  }
  return p;
}

void adaptq_plan_destroy(adaptq_plan_t h) {
  if (!h) return;
  Plan *p = static_cast<Plan *>(h);
  DeviceGuard g(p->device);
  p->d_list.release();
  p->d_ws.release();
  delete p;
}

int adaptq_plan_append_device(adaptq_plan_t h, const float *d_keys, const float *d_vals,
                              int n_tokens, int first_pos, void *stream) {
  (void)first_pos;
  const char *fn = "adaptq_plan_append_device";
  if (!require_handle(h, fn) || !require_pointer(d_keys, fn, "d_keys") ||
      !require_pointer(d_vals, fn, "d_vals"))
    return -1;
  if (n_tokens < 0) {
    set_error("adaptq_plan_append_device: negative n_tokens");
    return -1;
  }
  Plan *p = static_cast<Plan *>(h);
  if (n_tokens == 0) return 0;
  std::lock_guard<std::mutex> gp(p->mu);
  if (!plan_scan(p, fn)) return -1;
  DeviceGuard g(p->device);
  hipStream_t s = static_cast<hipStream_t>(stream);  // NULL = the HIP null stream
  const Ctx *c0 = p->ctxs[0];
  hipError_t e = caller_begin(p->device, s);
  if (e == hipSuccess)
    e = aq::launch_append(static_cast<aq::HeadDesc **>(p->d_list.p), (int)p->ctxs.size(), c0->dim,
                          c0->padded, c0->k_bits, c0->v_bits, d_keys, d_vals, n_tokens, s,
                          any_mirror(p->ctxs, n_tokens));
  if (e == hipSuccess) e = caller_end(p->device, s);
  if (hip_fail(e, fn)) return -1;
  // Every context takes the same n_tokens: update the host ring states and
  // the plan's cache in one pass, without the contexts' locks (calls that
  // touch the same contexts must not overlap a plan call).
  int max_n = 0;
  bool have = false, mixed = false;
  Mode mode = Mode::Dense;
  for (Ctx *c : p->ctxs) {
    c->st = aq::ring_after(c->st, n_tokens, c->cap, c->hyb);
    if (c->st.size > 0) {
      const Mode m = mode_of(c);
      if (have && m != mode) mixed = true;
      mode = m;
      have = true;
    }
    max_n = std::max(max_n, c->st.size);
  }
  p->max_n = max_n;
  p->mode = mode;
  p->mixed = mixed;
  // the states changed: other plans over these contexts must rescan; this
  // plan's cache stays valid unless someone else moved the epoch meanwhile
  uint64_t expect = p->seen;
  if (g_epoch.compare_exchange_strong(expect, expect + 1, std::memory_order_acq_rel))
    p->seen = expect + 1;
  else
    bump_epoch();
  return 0;
}

int adaptq_plan_compute_device_static(adaptq_plan_t h, const float *d_queries, float *d_outs,
                                      void *stream) {
  const char *fn = "adaptq_plan_compute_device_static";
  if (!require_handle(h, fn) || !require_pointer(d_queries, fn, "d_queries") ||
      !require_pointer(d_outs, fn, "d_outs"))
    return -1;
  Plan *p = static_cast<Plan *>(h);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (capturing(s)) {
    // the ordering event below cannot be waited on from inside a capture
    set_errorf(fn, "not supported on a stream under HIP graph capture");
    return -1;
  }
  std::lock_guard<std::mutex> gp(p->mu);
  if (!plan_scan(p, fn, false)) return -1;
  DevSync *d = dev_sync(p->device);
  void *ws = d ? d->scratch : nullptr;  // the device's address of `scratch`, set up at creation
  if (!ws || !d->static_ev) {
    set_errorf(fn, "the device's static scratch is not set up");
    return -1;
  }
  const size_t need = p->mixed ? 0 : plan_ws_floats(p) * 4;
  if (need > kScratchBytes) {
    char msg[256];
    std::snprintf(msg, sizeof(msg),
                  "%s: the decode needs %zu bytes of workspace, more than the static scratch's "
                  "%zu; use adaptq_plan_compute_device",
                  fn, need, kScratchBytes);
    set_error(msg);
    return -1;
  }
  DeviceGuard g(p->device);
  // calls on any stream or thread of this device run one after another on
  // the device: this call's work waits for the previous call's, and the
  // next call waits for this one's
  std::lock_guard<std::mutex> gs(d->static_mu);
  if (d->static_used && hip_fail(hipStreamWaitEvent(s, d->static_ev, 0), fn)) return -1;
  const int rc = plan_launch_decode(p, d_queries, d_outs, static_cast<float *>(ws), s, fn);
  // recorded also after a failed launch sequence, part of which may have run
  if (hip_fail(hipEventRecord(d->static_ev, s), fn)) return -1;
  d->static_used = true;
  return rc;
}

long long adaptq_plan_workspace_bytes(adaptq_plan_t h) {
  const char *fn = "adaptq_plan_workspace_bytes";
  if (!require_handle(h, fn)) return -1;
  Plan *p = static_cast<Plan *>(h);
  std::lock_guard<std::mutex> gp(p->mu);
  if (!plan_scan(p, fn, false)) return -1;
  return p->mixed ? 0 : (long long)(plan_ws_floats(p) * 4);
}

int adaptq_plan_compute_device(adaptq_plan_t h, const float *d_queries, float *d_outs,
                               void *stream) {
  const char *fn = "adaptq_plan_compute_device";
  if (!require_handle(h, fn) || !require_pointer(d_queries, fn, "d_queries") ||
      !require_pointer(d_outs, fn, "d_outs"))
    return -1;
  Plan *p = static_cast<Plan *>(h);
  std::lock_guard<std::mutex> gp(p->mu);
  if (!plan_scan(p, fn)) return -1;
  DeviceGuard g(p->device);
  if (!p->mixed && hip_fail(p->d_ws.ensure(plan_ws_floats(p) * 4), fn)) return -1;
  return plan_launch_decode(p, d_queries, d_outs, static_cast<float *>(p->d_ws.p),
                            static_cast<hipStream_t>(stream), fn);
}

}  // extern "C"

// ---- Packed-ring snapshots (AQSS v2) ----
//
// Layout (little-endian), as documented in reference replay/session_snapshot.h:16-40
// and written/read by session_snapshot.cpp:205-300:
//   u32 magic 0x41515353, u32 version 2, i32 n_layers, i32 n_heads, i32 dim,
//   i32 bits, i32 n_tokens, i32 n_heads_total, u64 flags
//   per head (layer-major): i32 layer, i32 head, i32 cache_size, i32 slot_bytes,
//     u64 data_bytes, data[cache_size * 2 * slot_bytes] (K slots then V slots),
//     i32 n_scales, f32 scales[2 * cache_size], i32 n_tags, u8 tags[2 * cache_size]
//   [flags & 2: per head i32 len + strategy state]  [flags & 1: token log]

namespace {

uint8_t snap_tag(int bits) { return bits == 16 ? 0xFF : (uint8_t)bits; }  // har_fixed.cpp:40-42, fp_passthrough.cpp:36

struct SnapOut {
  std::vector<uint8_t> buf;
  template <class T>
  void put(T v) {
    const uint8_t *p = reinterpret_cast<const uint8_t *>(&v);
    buf.insert(buf.end(), p, p + sizeof(T));
  }
  void put_bytes(const void *p, size_t n) {
    const uint8_t *b = static_cast<const uint8_t *>(p);
    buf.insert(buf.end(), b, b + n);
  }
};

struct SnapIn {
  const uint8_t *p;
  size_t n, off = 0;
  bool ok = true;
  template <class T>
  T get() {
    T v{};
    if (n - off < sizeof(T)) {
      ok = false;
      off = n;
      return v;
    }
    std::memcpy(&v, p + off, sizeof(T));
    off += sizeof(T);
    return v;
  }
  const uint8_t *take(uint64_t bytes) {
    if (bytes > n - off) {
      ok = false;
      off = n;
      return nullptr;
    }
    const uint8_t *r = p + off;
    off += (size_t)bytes;
    return r;
  }
};

// The rings of one head in logical order (oldest first), K rows in the
// reference's byte order.  Caller holds the head's lock and has flushed.
bool read_ring(Ctx *c, std::vector<uint8_t> &kc, std::vector<uint8_t> &vc,
               std::vector<float> &ks, std::vector<float> &vs, const char *fn) {
  const int n = c->st.size, cap = c->cap;
  kc.assign((size_t)n * c->k_pb, 0);
  vc.assign((size_t)n * c->v_pb, 0);
  ks.assign((size_t)n, 0.f);
  vs.assign((size_t)n, 0.f);
  if (n == 0) return true;
  DeviceGuard g(c->device);
  const aq::HeadDesc &hd = c->hd;
  hipError_t e = hipSuccess;
  std::vector<uint8_t> ak((size_t)cap * c->k_pb), av((size_t)cap * c->v_pb);
  std::vector<float> aks((size_t)cap), avs((size_t)cap);
  if (e == hipSuccess) e = hipMemcpy(ak.data(), hd.k_codes, ak.size(), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(av.data(), hd.v_codes, av.size(), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(aks.data(), hd.k_scale, aks.size() * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(avs.data(), hd.v_scale, avs.size() * 4, hipMemcpyDeviceToHost);
  if (hip_fail(e, fn)) return false;
  const int xmask = aq::kperm_mask(c->padded, c->k_bits);
  for (int i = 0; i < n; ++i) {
    const int slot = (int)(((long long)c->st.head - n + cap + i) % cap);
    const uint8_t *kr = ak.data() + (size_t)slot * c->k_pb;
    uint8_t *ko = kc.data() + (size_t)i * c->k_pb;
    const int x = slot & xmask;
    for (int j = 0; j < c->k_pb; ++j) ko[j] = kr[j ^ x];
    std::memcpy(vc.data() + (size_t)i * c->v_pb, av.data() + (size_t)slot * c->v_pb, c->v_pb);
    ks[i] = aks[slot];
    vs[i] = avs[slot];
  }
  return true;
}

// Rebuild a head's ring from logical-order rows: slots 0..n-1, head at n
// (mod cap), hybrid mirror empty.  Caller holds the head's lock.
bool write_ring(Ctx *c, int n, const uint8_t *kc, const uint8_t *vc, int row_stride,
                const float *ks, const float *vs, const char *fn) {
  {
    // appends still queued (library stream or callers') would land after the copies
    DeviceGuard g(c->device);
    if (hip_fail(settle(c->device), fn)) return false;
  }
  const int cap = c->cap;
  std::vector<uint8_t> ak((size_t)cap * c->k_pb, 0), av((size_t)cap * c->v_pb, 0);
  std::vector<float> aks((size_t)cap, 1.0f), avs((size_t)cap, 1.0f);
  const int xmask = aq::kperm_mask(c->padded, c->k_bits);
  for (int i = 0; i < n; ++i) {
    const uint8_t *kr = kc + (size_t)i * row_stride;
    uint8_t *ko = ak.data() + (size_t)i * c->k_pb;
    const int x = i & xmask;
    for (int j = 0; j < c->k_pb; ++j) ko[j ^ x] = kr[j];
    std::memcpy(av.data() + (size_t)i * c->v_pb, vc + (size_t)i * row_stride, c->v_pb);
    aks[i] = ks[i];
    avs[i] = vs[i];
  }
  aq::RingState st{cap > 0 ? n % cap : 0, n, 0, 0};
  DeviceGuard g(c->device);
  const aq::HeadDesc &hd = c->hd;
  hipError_t e = hipSuccess;
  if (e == hipSuccess && cap > 0) e = hipMemcpy(hd.k_codes, ak.data(), ak.size(), hipMemcpyHostToDevice);
  if (e == hipSuccess && cap > 0) e = hipMemcpy(hd.v_codes, av.data(), av.size(), hipMemcpyHostToDevice);
  if (e == hipSuccess && cap > 0) e = hipMemcpy(hd.k_scale, aks.data(), aks.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess && cap > 0) e = hipMemcpy(hd.v_scale, avs.data(), avs.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(&c->d_desc->st, &st, sizeof(st), hipMemcpyHostToDevice);
  if (hip_fail(e, fn)) return false;
  c->st = st;
  c->staged = 0;
  c->stage_k.clear();
  c->stage_v.clear();
  bump_epoch();
  return true;
}

bool snap_layers_ok(const adaptq_mha_t *layers, int n_layers, const char *fn) {
  if (!layers || n_layers <= 0) {
    set_errorf(fn, "need at least one MHA");
    return false;
  }
  for (int l = 0; l < n_layers; ++l)
    if (!require_handle(layers[l], fn)) return false;
  const Mha *m0 = static_cast<const Mha *>(layers[0]);
  const Ctx *c0 = m0->heads[0];
  for (int l = 1; l < n_layers; ++l) {
    const Mha *m = static_cast<const Mha *>(layers[l]);
    const Ctx *c = m->heads[0];
    if (m->n_heads != m0->n_heads || c->dim != c0->dim || c->k_bits != c0->k_bits ||
        c->v_bits != c0->v_bits || c->padded != c0->padded) {
      set_errorf(fn, "layers differ in n_heads, dim or bits");
      return false;
    }
  }
  return true;
}

}  // namespace

extern "C" {

int adaptq_snapshot_save(const adaptq_mha_t *layers, int n_layers, const char *path) {
  const char *fn = "adaptq_snapshot_save";
  if (!require_pointer(path, fn, "path") || !snap_layers_ok(layers, n_layers, fn)) return -1;
  const Mha *m0 = static_cast<const Mha *>(layers[0]);
  const Ctx *c0 = m0->heads[0];
  const int H = m0->n_heads;
  const int slot_bytes = std::max(c0->k_pb, c0->v_pb);
  SnapOut o;
  o.put<uint32_t>(0x41515353u);
  o.put<uint32_t>(2u);
  o.put<int32_t>(n_layers);
  o.put<int32_t>(H);
  o.put<int32_t>(c0->dim);
  o.put<int32_t>(c0->k_bits);
  const size_t ntok_at = o.buf.size();
  o.put<int32_t>(0);  // n_tokens: patched below
  o.put<int32_t>(n_layers * H);
  o.put<uint64_t>(0);  // no token log, no strategy state
  int n_tokens = 0;
  std::vector<uint8_t> kc, vc, pad((size_t)slot_bytes, 0);
  std::vector<float> ks, vs;
  for (int l = 0; l < n_layers; ++l) {
    Mha *m = static_cast<Mha *>(layers[l]);
    std::lock_guard<std::mutex> gm(m->mu);
    HeadLocks locks(m);
    if (!flush_all_locked(m, fn, true)) return -1;
    for (int h = 0; h < H; ++h) {
      Ctx *c = m->heads[h];
      if (!read_ring(c, kc, vc, ks, vs, fn)) return -1;
      const int n = c->st.size;
      n_tokens = std::max(n_tokens, n);
      o.put<int32_t>(l);
      o.put<int32_t>(h);
      o.put<int32_t>(n);
      o.put<int32_t>(slot_bytes);
      o.put<uint64_t>((uint64_t)n * 2 * slot_bytes);
      for (int i = 0; i < n; ++i) {
        o.put_bytes(kc.data() + (size_t)i * c->k_pb, c->k_pb);
        o.put_bytes(pad.data(), slot_bytes - c->k_pb);
      }
      for (int i = 0; i < n; ++i) {
        o.put_bytes(vc.data() + (size_t)i * c->v_pb, c->v_pb);
        o.put_bytes(pad.data(), slot_bytes - c->v_pb);
      }
      o.put<int32_t>(2 * n);
      o.put_bytes(ks.data(), (size_t)n * 4);
      o.put_bytes(vs.data(), (size_t)n * 4);
      o.put<int32_t>(2 * n);
      o.buf.insert(o.buf.end(), (size_t)n, snap_tag(c->k_bits));
      o.buf.insert(o.buf.end(), (size_t)n, snap_tag(c->v_bits));
    }
  }
  std::memcpy(o.buf.data() + ntok_at, &n_tokens, 4);
  FILE *f = std::fopen(path, "wb");
  if (!f) {
    set_errorf(fn, "cannot open the file for writing");
    return -1;
  }
  const bool ok = std::fwrite(o.buf.data(), 1, o.buf.size(), f) == o.buf.size();
  if (std::fclose(f) != 0 || !ok) {
    set_errorf(fn, "write error");
    return -1;
  }
  clear_error();
  return 0;
}

int adaptq_snapshot_load(const adaptq_mha_t *layers, int n_layers, const char *path) {
  const char *fn = "adaptq_snapshot_load";
  if (!require_pointer(path, fn, "path") || !snap_layers_ok(layers, n_layers, fn)) return -1;
  std::vector<uint8_t> file;
  {
    FILE *f = std::fopen(path, "rb");
    if (!f) {
      set_errorf(fn, "cannot open the file");
      return -1;
    }
    uint8_t chunk[1 << 16];
    size_t got;
    while ((got = std::fread(chunk, 1, sizeof(chunk), f)) > 0) file.insert(file.end(), chunk, chunk + got);
    std::fclose(f);
  }
  if (file.size() < 40) {
    set_errorf(fn, "file too small");
    return -1;
  }
  const Mha *m0 = static_cast<const Mha *>(layers[0]);
  const Ctx *c0 = m0->heads[0];
  const int H = m0->n_heads;
  SnapIn in{file.data(), file.size()};
  const uint32_t magic = in.get<uint32_t>(), version = in.get<uint32_t>();
  const int32_t nl = in.get<int32_t>(), nh = in.get<int32_t>(), dim = in.get<int32_t>();
  const int32_t bits = in.get<int32_t>(), ntok = in.get<int32_t>(), nht = in.get<int32_t>();
  const uint64_t flags = in.get<uint64_t>();
  (void)bits;
  if (magic != 0x41515353u) {
    set_errorf(fn, "invalid magic (not an AQSS file)");
    return -1;
  }
  if (version > 2u) {
    set_errorf(fn, "snapshot version newer than 2");
    return -1;
  }
  if (nl != n_layers || nh != H || dim != c0->dim || nht != nl * nh || ntok < 0) {
    set_errorf(fn, "snapshot shape does not match the MHAs (layers, heads, dim)");
    return -1;
  }
  struct Block {
    int layer, head, n, slot_bytes;
    const uint8_t *data;
    const uint8_t *scales;  // 2n f32, possibly unaligned in the file buffer
    const uint8_t *tags;
  };
  std::vector<Block> blocks((size_t)nht);
  std::vector<char> seen((size_t)nht, 0);
  const int slot_bytes = std::max(c0->k_pb, c0->v_pb);
  for (auto &b : blocks) {
    b.layer = in.get<int32_t>();
    b.head = in.get<int32_t>();
    b.n = in.get<int32_t>();
    b.slot_bytes = in.get<int32_t>();
    const uint64_t data_bytes = in.get<uint64_t>();
    if (!in.ok || b.layer < 0 || b.layer >= nl || b.head < 0 || b.head >= nh) {
      set_errorf(fn, in.ok ? "invalid head coordinates" : "truncated snapshot");
      return -1;
    }
    const Ctx *c = static_cast<const Mha *>(layers[b.layer])->heads[b.head];
    if (b.n < 0 || b.n > c->cap || b.slot_bytes != slot_bytes ||
        data_bytes != (uint64_t)b.n * 2 * (uint64_t)slot_bytes) {
      set_errorf(fn, "head storage does not fit the MHA (cache size, slot bytes)");
      return -1;
    }
    b.data = in.take(data_bytes);
    const int32_t n_scales = in.get<int32_t>();
    b.scales = in.take(n_scales == 2 * b.n ? (uint64_t)n_scales * 4 : ~0ull);
    const int32_t n_tags = in.get<int32_t>();
    b.tags = in.take(n_tags == 2 * b.n ? (uint64_t)n_tags : ~0ull);
    if (!in.ok) {
      set_errorf(fn, "truncated or inconsistent head block");
      return -1;
    }
    for (int i = 0; i < b.n; ++i)
      if (b.tags[i] != snap_tag(c->k_bits) || b.tags[b.n + i] != snap_tag(c->v_bits)) {
        set_errorf(fn, "format tags do not match the MHA's bit widths");
        return -1;
      }
    char &s = seen[(size_t)b.layer * nh + b.head];
    if (s) {
      set_errorf(fn, "duplicate head block");
      return -1;
    }
    s = 1;
  }
  if (flags & 2u)
    for (int i = 0; i < nht; ++i) {
      const int32_t len = in.get<int32_t>();
      in.take(len >= 0 ? (uint64_t)len : ~0ull);
    }
  if (!in.ok) {
    set_errorf(fn, "truncated strategy state");
    return -1;
  }
  // The token log (flags & 1) is not needed to restore packed rings.
  for (const auto &b : blocks) {
    Mha *m = static_cast<Mha *>(layers[b.layer]);
    std::lock_guard<std::mutex> gm(m->mu);
    Ctx *c = m->heads[b.head];
    std::lock_guard<std::mutex> gc(c->mu);
    const uint8_t *kc = b.data, *vc = b.data + (size_t)b.n * slot_bytes;
    std::vector<float> ks((size_t)b.n), vs((size_t)b.n);
    std::memcpy(ks.data(), b.scales, (size_t)b.n * 4);
    std::memcpy(vs.data(), b.scales + (size_t)b.n * 4, (size_t)b.n * 4);
    if (!write_ring(c, b.n, kc, vc, slot_bytes, ks.data(), vs.data(), fn)) return -1;
  }
  clear_error();
  return 0;
}

}  // extern "C"
