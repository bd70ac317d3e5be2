// The C ABI of layer 1 (include/emeans_hip.h): context, buffers and the
// Device ops, each validated like the reference CPU backend
// (crates/emeans-core/src/core/cpu.rs) before anything is queued.

#include <algorithm>
#include <atomic>
#include <cstring>
#include <deque>
#include <exception>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "emh_internal.h"

namespace {
thread_local std::string g_last_error;

// Device scratch of emh_top1_noalloc: one fixed block per GPU, in the code
// object's device memory, so that the entry point allocates nothing. In host
// code `scratch` names a host-side stand-in, never the device block: only the
// address hipGetSymbolAddress gives (per device, kept in g_scratch) may reach
// a kernel or a copy.
constexpr size_t SCRATCH_BYTES = size_t(32) << 20;
static __device__ __align__(256) char scratch[SCRATCH_BYTES];
constexpr int SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
char* g_scratch[SCRATCH_DEVICES] = {};
// Per device: an event recorded on the stream of the last call that used the
// block (g_scratch_used once one has), which the next call's stream waits
// for, so that calls from different streams or contexts run one after another.
hipEvent_t g_scratch_done[SCRATCH_DEVICES] = {};
bool g_scratch_used[SCRATCH_DEVICES] = {};

// The device address of `scratch` on `device`, looked up once per device with
// that device current (emh_create calls this after hipSetDevice), and the
// device's ordering event.
char* scratch_setup(int device) {
  EMH_ENSURE(device >= 0 && device < SCRATCH_DEVICES, "device %d: at most %d devices", device,
             SCRATCH_DEVICES);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      char m[256];
      snprintf(m, sizeof m, "hipGetSymbolAddress(scratch) on device %d failed: %s", device,
               hipGetErrorString(e));
      throw emh::Failure(m);
    }
    EMH_HIP(hipEventCreateWithFlags(&g_scratch_done[device], hipEventDisableTiming));
    g_scratch[device] = (char*)p;
  }
  return g_scratch[device];
}

template <class F>
int guard(F&& f) {
  try {
    f();
    return EMH_OK;
  } catch (const emh::Invalid& e) {
    g_last_error = e.what();
    return EMH_INVALID;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return EMH_ERROR;
  } catch (...) {
    g_last_error = "unknown error";
    return EMH_ERROR;
  }
}

void use_device(emh_ctx* c) { EMH_HIP(hipSetDevice(c->device)); }

std::atomic<uint64_t> g_serial{0};

// Blocks of freed buffers, kept per device for the next buffer of the same
// size. hipFree waits for every stream on the device, so a loop of small runs
// on several contexts at once (the automatic-k sweeps) would run one context
// at a time. emh_free drains the freeing context's stream; for the work the
// other live contexts on the device had queued by then, it records an event
// on each of their streams, and whichever context takes the block again
// makes its streams wait for those events before its first write.
constexpr size_t KEEP_BLOCK_MAX = size_t(64) << 20;   // larger blocks are freed
constexpr size_t KEEP_DEVICE_MAX = size_t(1) << 30;   // kept bytes per device
struct KeptBlock {
  int device;
  size_t bytes;
  void* ptr;
  std::vector<hipEvent_t> after;
};
std::mutex g_blocks_mu;
std::vector<emh_ctx*> g_live;                 // contexts not yet destroyed
std::deque<KeptBlock> g_kept;                 // oldest first
std::map<int, size_t> g_kept_bytes;           // per device
std::map<int, std::vector<hipEvent_t>> g_spare_events;  // per device, no timing

hipEvent_t spare_event(int device) {  // with g_blocks_mu held, device current
  std::vector<hipEvent_t>& v = g_spare_events[device];
  if (!v.empty()) {
    hipEvent_t e = v.back();
    v.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  EMH_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  return e;
}

// A kept block of exactly `bytes` on c's device, with c's streams ordered
// after the work that may still use it; nullptr if none is kept.
void* take_kept(emh_ctx* c, size_t bytes) {
  std::lock_guard<std::mutex> g(g_blocks_mu);
  for (auto it = g_kept.begin(); it != g_kept.end(); ++it) {
    if (it->device != c->device || it->bytes != bytes) continue;
    // Most have completed by now: a wait between hardware queues is queued
    // only for those that have not. A failed wait leaves the block kept.
    for (hipEvent_t e : it->after) {
      if (hipEventQuery(e) != hipSuccess) {
        (void)hipGetLastError();  // not-ready is no error of the next launch
        EMH_HIP(hipStreamWaitEvent(c->stream, e, 0));
        EMH_HIP(hipStreamWaitEvent(c->copies(), e, 0));
      }
    }
    std::vector<hipEvent_t>& spare = g_spare_events[c->device];
    spare.insert(spare.end(), it->after.begin(), it->after.end());
    void* p = it->ptr;
    g_kept_bytes[c->device] -= bytes;
    g_kept.erase(it);
    return p;
  }
  return nullptr;
}

// Keeps the block of a buffer freed on c (whose stream has been drained), or
// frees it when it is too large. Past the device's limit the oldest kept
// blocks are freed.
void keep_block(emh_ctx* c, void* p, size_t bytes) {
  if (bytes > KEEP_BLOCK_MAX) {
    EMH_HIP(hipFree(p));
    return;
  }
  std::vector<void*> drop;
  std::exception_ptr failed;
  {
    std::lock_guard<std::mutex> g(g_blocks_mu);
    KeptBlock kb{c->device, bytes, p, {}};
    try {
      for (emh_ctx* o : g_live) {
        if (o == c || o->device != c->device) continue;
        for (hipStream_t st : {o->stream, o->copy_stream}) {
          if (!st) continue;  // no copy stream yet: nothing queued there
          hipEvent_t e = spare_event(c->device);
          kb.after.push_back(e);
          EMH_HIP(hipEventRecord(e, st));
        }
      }
    } catch (...) {
      // The block is freed instead (hipFree waits for every stream).
      std::vector<hipEvent_t>& spare = g_spare_events[c->device];
      spare.insert(spare.end(), kb.after.begin(), kb.after.end());
      failed = std::current_exception();
    }
    size_t& total = g_kept_bytes[c->device];
    if (!failed) {
      g_kept.push_back(std::move(kb));
      total += bytes;
    }
    for (auto it = g_kept.begin(); total > KEEP_DEVICE_MAX && it != g_kept.end();) {
      if (it->device != c->device) {
        ++it;
        continue;
      }
      total -= it->bytes;
      drop.push_back(it->ptr);
      for (hipEvent_t e : it->after) g_spare_events[c->device].push_back(e);
      it = g_kept.erase(it);
    }
  }
  if (failed) drop.push_back(p);
  hipError_t first = hipSuccess;
  for (void* q : drop) {
    const hipError_t e = hipFree(q);
    if (first == hipSuccess) first = e;
  }
  if (failed) std::rethrow_exception(failed);
  EMH_HIP(first);
}

// Frees the blocks kept on `device` and its spare events (the last context
// on the device is going).
void release_kept(int device) {
  std::vector<void*> drop;
  std::vector<hipEvent_t> evs;
  {
    std::lock_guard<std::mutex> g(g_blocks_mu);
    for (emh_ctx* o : g_live)
      if (o->device == device) return;
    for (auto it = g_kept.begin(); it != g_kept.end();) {
      if (it->device != device) {
        ++it;
        continue;
      }
      drop.push_back(it->ptr);
      evs.insert(evs.end(), it->after.begin(), it->after.end());
      it = g_kept.erase(it);
    }
    g_kept_bytes[device] = 0;
    std::vector<hipEvent_t>& v = g_spare_events[device];
    evs.insert(evs.end(), v.begin(), v.end());
    v.clear();
  }
  for (void* q : drop) (void)hipFree(q);
  for (hipEvent_t e : evs) (void)hipEventDestroy(e);
}

emh_buf* new_buf(emh_ctx* c, size_t len, int kind) {
  auto* b = new emh_buf;
  b->len = len;
  b->kind = kind;
  b->serial = ++g_serial;
  b->device = c->device;
  if (len > 0 && len * 4 <= KEEP_BLOCK_MAX) {
    try {
      b->ptr = take_kept(c, len * 4);
    } catch (...) {
      delete b;
      throw;
    }
  }
  if (len > 0 && !b->ptr) {
    hipError_t e = hipMalloc(&b->ptr, len * 4);
    if (e != hipSuccess) {
      delete b;
      char m[256];
      snprintf(m, sizeof m, "hipMalloc of %zu bytes failed: %s", len * 4, hipGetErrorString(e));
      throw emh::Failure(m);
    }
  }
  return b;
}

const float* F(const emh_buf* b, const char* what) {
  EMH_ENSURE(b && b->kind == 0, "%s must be an f32 buffer", what);
  return (const float*)b->ptr;
}
float* Fm(emh_buf* b, const char* what) {
  EMH_ENSURE(b && b->kind == 0, "%s must be an f32 buffer", what);
  ++b->gen;  // an output: its contents change
  return (float*)b->ptr;
}
const uint32_t* U(const emh_buf* b, const char* what) {
  EMH_ENSURE(b && b->kind == 1, "%s must be a u32 buffer", what);
  return (const uint32_t*)b->ptr;
}
uint32_t* Um(emh_buf* b, const char* what) {
  EMH_ENSURE(b && b->kind == 1, "%s must be a u32 buffer", what);
  return (uint32_t*)b->ptr;
}

// Errors the kernels record on the device come up at the next wait.
void check_device_flags(emh_ctx* c) {
  uint32_t w[emh::SW_WORDS];
  EMH_HIP(hipMemcpyAsync(w, c->small, sizeof w, hipMemcpyDeviceToHost, c->stream));
  EMH_HIP(hipStreamSynchronize(c->stream));
  bool bad_label = w[emh::SW_BAD_LABEL] != 0, bad_id = w[emh::SW_BAD_ID] != 0;
  if (bad_label || bad_id) {
    emh::launch_fill_u32(c, c->small + emh::SW_BAD_LABEL, 1, 0);
    emh::launch_fill_u32(c, c->small + emh::SW_BAD_ID, 1, 0);
    EMH_HIP(hipStreamSynchronize(c->stream));
    EMH_ENSURE(!bad_label, "scatter_add: label out of range");
    EMH_ENSURE(!bad_id, "row id out of range");
  }
}

// core/mod.rs:432-439 (check_select).
void check_select(const emh_buf* ids, size_t lo, size_t hi, size_t nx) {
  EMH_ENSURE(lo <= hi, "bad row range");
  if (ids)
    EMH_ENSURE(hi <= ids->len, "row range past the ids");
  else
    EMH_ENSURE(hi <= nx, "row range past the data");
}
}  // namespace

namespace emh {
void set_last_error(const std::string& m) { g_last_error = m; }
}  // namespace emh

extern "C" {

const char* emh_last_error(void) { return g_last_error.c_str(); }

int emh_create(int device, emh_ctx** out) {
  return guard([&] {
    EMH_ENSURE(out != nullptr, "out is null");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
      throw emh::Failure("no HIP device");
    EMH_ENSURE(device >= 0 && device < n, "device %d not present (%d devices)", device, n);
    EMH_HIP(hipSetDevice(device));
    hipDeviceProp_t p;
    EMH_HIP(hipGetDeviceProperties(&p, device));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {
      char m[256];
      snprintf(m, sizeof m, "device %d is %s; this library is built for gfx950", device,
               p.gcnArchName);
      throw emh::Failure(m);
    }
    char* block = scratch_setup(device);
    auto* c = new emh_ctx;
    c->device = device;
    c->scratch = block;
    c->cus = p.multiProcessorCount;
    if (const char* s = getenv("EMEANS_HIP_SCREEN")) {
      const int m = atoi(s);
      c->screen = m >= emh::SCREEN_OFF && m <= emh::SCREEN_F16 ? m : emh::SCREEN_BF3;
    }
    try {
      EMH_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
      for (hipEvent_t& e : c->ev_stage) EMH_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
      EMH_HIP(hipMalloc(&c->small, emh::SW_WORDS * 4));
      EMH_HIP(hipMemsetAsync(c->small, 0, emh::SW_WORDS * 4, c->stream));
      EMH_HIP(hipStreamSynchronize(c->stream));
    } catch (...) {
      if (c->small) (void)hipFree(c->small);
      if (c->stream) (void)hipStreamDestroy(c->stream);
      if (c->copy_stream) (void)hipStreamDestroy(c->copy_stream);
      for (hipEvent_t e : c->ev_stage)
        if (e) (void)hipEventDestroy(e);
      delete c;
      throw;
    }
    {
      std::lock_guard<std::mutex> g(g_blocks_mu);
      g_live.push_back(c);
    }
    *out = c;
  });
}

int emh_destroy(emh_ctx* c) {
  return guard([&] {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (c->copy_stream)
      (void)hipStreamSynchronize(c->copy_stream);  // copies may still read pinned staging
    for (emh::Scratch* s : {&c->cand, &c->fblist, &c->order, &c->start, &c->misc, &c->knn_tmp,
                            &c->xnorm, &c->bigj, &c->chunkcnt, &c->tickets,
                            &c->preview_ticket, &c->xsplit, &c->csplit, &c->csplit_norm, &c->csplit_part,
                            &c->xpre, &c->xpre_norm, &c->tsplit, &c->tsplit_part, &c->tally_cnt,
                            &c->klong, &c->trun, &c->kpp, &c->iscore, &c->cnorm})
      s->release();
    for (emh::Pinned* s : {&c->pin_usage, &c->pin_plan, &c->pin_small, &c->pin_order[0],
                           &c->pin_order[1], &c->pin_lab[0], &c->pin_lab[1], &c->pin_sco[0],
                           &c->pin_sco[1], &c->pin_out, &c->pin_stage[0], &c->pin_stage[1],
                           &c->pin_aux})
      s->release();
    if (c->small) (void)hipFree(c->small);
    for (hipEvent_t e : c->ev_pool) (void)hipEventDestroy(e);
    for (hipEvent_t e : c->ev_stage) (void)hipEventDestroy(e);
    {
      std::lock_guard<std::mutex> g(g_blocks_mu);
      g_live.erase(std::remove(g_live.begin(), g_live.end(), c), g_live.end());
    }
    release_kept(c->device);  // when c was the device's last context
    (void)hipStreamDestroy(c->stream);
    if (c->copy_stream) (void)hipStreamDestroy(c->copy_stream);
    delete c;
  });
}

const char* emh_name(const emh_ctx* c) { return c ? c->name.c_str() : "hip-gfx950"; }

int emh_flush(emh_ctx* c) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    (void)hipStreamQuery(c->stream);
  });
}

int emh_sync(emh_ctx* c) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    use_device(c);
    check_device_flags(c);
  });
}

void* emh_stream(emh_ctx* c) { return c ? (void*)c->stream : nullptr; }

// ------------------------------------------------------------------ buffers
static int upload(emh_ctx* c, const void* v, size_t len, int kind, emh_buf** out) {
  return guard([&] {
    EMH_ENSURE(c && out, "null argument");
    EMH_ENSURE(len == 0 || v, "null source");
    use_device(c);
    emh_buf* b = new_buf(c, len, kind);
    if (len > 0) {
      hipError_t e = hipMemcpyAsync(b->ptr, v, len * 4, hipMemcpyHostToDevice, c->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(c->stream);  // the source may go away
      if (e != hipSuccess) {
        (void)hipFree(b->ptr);
        delete b;
        throw emh::Failure(std::string("upload failed: ") + hipGetErrorString(e));
      }
    }
    *out = b;
  });
}

int emh_bind(emh_ctx* c, const float* x, size_t len, emh_buf** out) {
  return upload(c, x, len, 0, out);
}
int emh_upload_f32(emh_ctx* c, const float* v, size_t len, emh_buf** out) {
  return upload(c, v, len, 0, out);
}
int emh_upload_u32(emh_ctx* c, const uint32_t* v, size_t len, emh_buf** out) {
  return upload(c, v, len, 1, out);
}

static int zeros(emh_ctx* c, size_t len, int kind, emh_buf** out) {
  return guard([&] {
    EMH_ENSURE(c && out, "null argument");
    use_device(c);
    emh_buf* b = new_buf(c, len, kind);
    if (len > 0) emh::launch_fill_u32(c, (uint32_t*)b->ptr, len, 0);
    *out = b;
  });
}
int emh_zeros_f32(emh_ctx* c, size_t len, emh_buf** out) { return zeros(c, len, 0, out); }
int emh_zeros_u32(emh_ctx* c, size_t len, emh_buf** out) { return zeros(c, len, 1, out); }

static int write(emh_ctx* c, emh_buf* b, size_t off, const void* v, size_t len, int kind) {
  return guard([&] {
    EMH_ENSURE(c && b && b->kind == kind, "buffer kind mismatch");
    EMH_ENSURE(off + len <= b->len, "write past the buffer");
    if (len == 0) return;
    use_device(c);
    ++b->gen;
    EMH_HIP(hipMemcpyAsync((char*)b->ptr + off * 4, v, len * 4, hipMemcpyHostToDevice,
                           c->stream));
    EMH_HIP(hipStreamSynchronize(c->stream));
  });
}
int emh_write_f32(emh_ctx* c, emh_buf* b, size_t off, const float* v, size_t len) {
  return write(c, b, off, v, len, 0);
}
int emh_write_u32(emh_ctx* c, emh_buf* b, size_t off, const uint32_t* v, size_t len) {
  return write(c, b, off, v, len, 1);
}

static int read(emh_ctx* c, const emh_buf* b, size_t lo, size_t hi, void* dst, int kind) {
  return guard([&] {
    EMH_ENSURE(c && b && b->kind == kind, "buffer kind mismatch");
    EMH_ENSURE(lo <= hi && hi <= b->len, "read past the buffer");
    use_device(c);
    if (hi > lo)
      EMH_HIP(hipMemcpyAsync(dst, (const char*)b->ptr + lo * 4, (hi - lo) * 4,
                             hipMemcpyDeviceToHost, c->stream));
    check_device_flags(c);  // waits
  });
}
int emh_read_f32(emh_ctx* c, const emh_buf* b, size_t lo, size_t hi, float* dst) {
  return read(c, b, lo, hi, dst, 0);
}
int emh_read_u32(emh_ctx* c, const emh_buf* b, size_t lo, size_t hi, uint32_t* dst) {
  return read(c, b, lo, hi, dst, 1);
}

int emh_free(emh_ctx* c, emh_buf* b) {
  return guard([&] {
    if (!b) return;
    std::unique_ptr<emh_buf> hold(b);  // the handle goes, also when the call fails
    void* p = b->owned ? b->ptr : nullptr;
    const bool keep = p && c && !b->exposed && b->device == c->device;
    if (c) {
      use_device(c);
      const hipError_t e = hipStreamSynchronize(c->stream);
      if (e != hipSuccess) {
        if (p) (void)hipFree(p);  // waits for every stream on the device
        EMH_HIP(e);
      }
    }
    // A buffer whose address went out may be in use on streams of the
    // caller's own: hipFree waits for them.
    if (keep)
      keep_block(c, p, b->len * 4);
    else if (p)
      EMH_HIP(hipFree(p));
  });
}

int emh_wrap(emh_ctx* c, void* p, size_t len, int kind, emh_buf** out) {
  return guard([&] {
    EMH_ENSURE(c && out, "null argument");
    EMH_ENSURE(kind == 0 || kind == 1, "kind must be 0 (f32) or 1 (u32)");
    EMH_ENSURE(len == 0 || p, "null pointer");
    auto* b = new emh_buf;
    b->ptr = p;
    b->len = len;
    b->kind = kind;
    b->owned = false;
    b->serial = ++g_serial;
    b->exposed = true;  // foreign memory: written from outside
    *out = b;
  });
}

void* emh_buf_ptr(const emh_buf* b) {
  if (b) b->exposed = true;  // the caller may write it from now on
  return b ? b->ptr : nullptr;
}
size_t emh_buf_len(const emh_buf* b) { return b ? b->len : 0; }

// ---------------------------------------------------------------------- ops
}  // extern "C"

namespace {
// emh_top1's arguments, checked like the reference CPU backend's top1
// (core/cpu.rs:77-104, assign.rs:121-147).
struct Top1Call {
  const float* x;
  size_t nx;
  const uint32_t* ids;
  const float* cents;
  const float* cn;
  uint32_t* lab;
  float* sco;
};
Top1Call check_top1(emh_ctx* c, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                    size_t hi, const emh_buf* cents, const emh_buf* cnorm, size_t k, int metric,
                    emh_buf* labels, emh_buf* scores) {
  EMH_ENSURE(c, "null context");
  EMH_ENSURE(d > 0, "d must be positive");
  EMH_ENSURE(k > 0, "k must be positive");
  EMH_ENSURE(metric == EMH_L2 || metric == EMH_IP, "unknown metric");
  Top1Call t{};
  t.x = F(x, "x");
  t.nx = x->len / d;
  if (ids) t.ids = U(ids, "ids");
  check_select(ids, lo, hi, t.nx);
  EMH_ENSURE(cents && F(cents, "centroids") && cents->len >= k * d, "centroids must be k x d");
  t.cents = (const float*)cents->ptr;
  if (metric == EMH_L2) {
    EMH_ENSURE(cnorm != nullptr, "L2 top1 needs the centroid norms");
    t.cn = F(cnorm, "cnorm");
    EMH_ENSURE(cnorm->len >= k, "cnorm must have k entries");
  }
  t.lab = Um(labels, "labels");
  t.sco = Fm(scores, "scores");
  EMH_ENSURE(hi <= labels->len && hi <= scores->len, "outputs too short");
  return t;
}
}  // namespace

extern "C" {

int emh_top1(emh_ctx* c, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo, size_t hi,
             const emh_buf* cents, const emh_buf* cnorm, size_t k, int metric, emh_buf* labels,
             emh_buf* scores) {
  return guard([&] {
    const Top1Call t = check_top1(c, x, d, ids, lo, hi, cents, cnorm, k, metric, labels, scores);
    use_device(c);
    emh::launch_top1(c, t.x, t.nx, d, t.ids, lo, hi, t.cents, t.cn, k, metric == EMH_IP, t.lab,
                     t.sco);
  });
}

int emh_top1_noalloc(emh_ctx* c, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                     size_t hi, const emh_buf* cents, const emh_buf* cnorm, size_t k, int metric,
                     emh_buf* labels, emh_buf* scores) {
  return guard([&] {
    const Top1Call t = check_top1(c, x, d, ids, lo, hi, cents, cnorm, k, metric, labels, scores);
    if (hi <= lo) return;
    const size_t need = emh::top1_scratch_bytes(c, hi - lo, d, k, metric == EMH_IP);
    EMH_ENSURE(need <= SCRATCH_BYTES,
               "top1_noalloc: %zu rows x k = %zu x d = %zu need %zu bytes of scratch, above the "
               "fixed %zu",
               hi - lo, k, d, need, SCRATCH_BYTES);
    use_device(c);
    // The block is the GPU's, not the context's: hold the lock while queueing,
    // make this stream wait for the previous call's work on the block, and
    // mark this call's end for the next one (also when queueing fails midway).
    // A stream under graph capture takes no part (an event from outside the
    // capture cannot order it): the caller orders its graph's launches.
    std::lock_guard<std::mutex> g(g_scratch_mu);
    const int dv = c->device;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    EMH_HIP(hipStreamIsCapturing(c->stream, &cap));
    const bool order = cap == hipStreamCaptureStatusNone;
    if (order && g_scratch_used[dv])
      EMH_HIP(hipStreamWaitEvent(c->stream, g_scratch_done[dv], 0));
    struct Mark {
      emh_ctx* c;
      int dv;
      bool on;
      ~Mark() {
        if (on && hipEventRecord(g_scratch_done[dv], c->stream) == hipSuccess)
          g_scratch_used[dv] = true;
      }
    } mark{c, dv, order};
    emh::Arena ar{c->scratch, SCRATCH_BYTES, 0};
    emh::launch_top1(c, t.x, t.nx, d, t.ids, lo, hi, t.cents, t.cn, k, metric == EMH_IP, t.lab,
                     t.sco, false, &ar);
  });
}

int emh_screen_margin(emh_ctx* c, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                      size_t hi, const emh_buf* cents, const emh_buf* cnorm, size_t k, int metric,
                      emh_screen_report* out) {
  return guard([&] {
    EMH_ENSURE(out, "null argument");
    // Only the screen's lists are touched: labels and scores need no buffers.
    emh_buf none_u{nullptr, hi, 1, false}, none_f{nullptr, hi, 0, false};
    const Top1Call t = check_top1(c, x, d, ids, lo, hi, cents, cnorm, k, metric, &none_u, &none_f);
    use_device(c);
    emh_screen_report r{};
    emh::screen_margin_top1(c, t.x, t.nx, d, t.ids, lo, hi, t.cents, t.cn, k, metric == EMH_IP,
                            &r);
    *out = r;
  });
}

int emh_screen_margin_topk(emh_ctx* c, const emh_buf* q, size_t m, const emh_buf* data, size_t n,
                           size_t d, int exclude_self, emh_screen_report* out) {
  return guard([&] {
    EMH_ENSURE(c && out, "null argument");
    EMH_ENSURE(d > 0, "d must be positive");
    EMH_ENSURE(!exclude_self || m == n, "exclude_self needs queries == data");
    const float* qp = F(q, "queries");
    const float* dp = F(data, "data");
    EMH_ENSURE(q->len >= m * d && data->len >= n * d, "queries m x d, data n x d");
    use_device(c);
    emh_screen_report r{};
    emh::launch_topk(c, qp, m, dp, n, d, 16, exclude_self != 0, nullptr, nullptr, &r);
    *out = r;
  });
}

int emh_topk_dev(emh_ctx* c, const emh_buf* q, size_t m, const emh_buf* data, size_t n, size_t d,
                 size_t kk, int exclude_self, emh_buf* ids, emh_buf* sims) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    EMH_ENSURE(d > 0, "d must be positive");
    EMH_ENSURE(kk > 0, "k must be positive");
    EMH_ENSURE(kk <= (size_t)emh::KLONG, "topk keeps at most %d neighbours, got %zu", emh::KLONG,
               kk);
    EMH_ENSURE(!exclude_self || m == n, "exclude_self needs queries == data");
    const float* qp = F(q, "queries");
    const float* dp = F(data, "data");
    EMH_ENSURE(q->len >= m * d && data->len >= n * d, "queries m x d, data n x d");
    uint32_t* ip = Um(ids, "ids");
    float* sp = Fm(sims, "sims");
    EMH_ENSURE(ids->len >= m * kk && sims->len >= m * kk, "outputs must hold m x k");
    use_device(c);
    emh::launch_topk(c, qp, m, dp, n, d, kk, exclude_self != 0, ip, sp);
  });
}

int emh_topk(emh_ctx* c, const float* queries, size_t m, const float* data, size_t n, size_t d,
             size_t kk, int exclude_self, uint32_t* ids, float* sims) {
  return guard([&] {
    EMH_ENSURE(c && (m == 0 || (queries && ids && sims)) && (n == 0 || data), "null argument");
    EMH_ENSURE(d > 0 && kk > 0 && kk <= (size_t)emh::KLONG, "need d > 0 and 1 <= k <= %d",
               emh::KLONG);
    EMH_ENSURE(!exclude_self || m == n, "exclude_self needs queries == data");
    if (m == 0) return;
    use_device(c);
    const bool same = queries == data && m == n;
    emh_buf *qb = nullptr, *db = nullptr, *ib = nullptr, *sb = nullptr;
    auto cleanup = [&] {
      for (emh_buf* b : {qb, db, ib, sb})
        if (b && b != qb) emh_free(c, b);
      if (qb) emh_free(c, qb);
    };
    try {
      if (emh_upload_f32(c, queries, m * d, &qb)) throw emh::Failure(g_last_error);
      if (same)
        db = nullptr;
      else if (emh_upload_f32(c, data, n * d, &db))
        throw emh::Failure(g_last_error);
      if (emh_zeros_u32(c, m * kk, &ib) || emh_zeros_f32(c, m * kk, &sb))
        throw emh::Failure(g_last_error);
      emh::launch_topk(c, (const float*)qb->ptr, m, same ? (const float*)qb->ptr
                                                        : (const float*)db->ptr,
                       n, d, kk, exclude_self != 0, (uint32_t*)ib->ptr, (float*)sb->ptr);
      EMH_HIP(hipMemcpyAsync(ids, ib->ptr, m * kk * 4, hipMemcpyDeviceToHost, c->stream));
      EMH_HIP(hipMemcpyAsync(sims, sb->ptr, m * kk * 4, hipMemcpyDeviceToHost, c->stream));
      check_device_flags(c);
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}

int emh_scatter_add(emh_ctx* c, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                    size_t hi, const emh_buf* labels, size_t k, emh_buf* sums, emh_buf* counts,
                    emh_buf* acc) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    EMH_ENSURE(d > 0 && k > 0, "d and k must be positive");
    const float* xp = F(x, "x");
    const size_t nx = x->len / d;
    if (ids) U(ids, "ids");
    check_select(ids, lo, hi, nx);
    const uint32_t* lab = U(labels, "labels");
    EMH_ENSURE(hi <= labels->len, "labels shorter than the selection");
    float* sp = Fm(sums, "sums");
    uint32_t* cp = Um(counts, "counts");
    EMH_ENSURE(sums->len == k * d && counts->len == k, "sums k x d, counts k");
    float* ap = nullptr;
    if (acc) {
      ap = Fm(acc, "acc");
      EMH_ENSURE(acc->len == k * d, "acc must be k x d");
    }
    use_device(c);
    emh::ProfScope prof(c, EMH_PROF_SCATTER, emh::scatter_bytes(hi - lo, k, d, ids, ap),
                        emh::prof_take(c, EMH_PROF_SCATTER));
    emh::launch_scatter(c, xp, nx, d, ids ? (const uint32_t*)ids->ptr : nullptr, lo, hi, lab, k,
                        sp, cp, ap);
  });
}

int emh_row_norms(emh_ctx* c, const emh_buf* m, size_t rows, size_t d, emh_buf* out) {
  return guard([&] {
    EMH_ENSURE(c && d > 0, "bad arguments");
    const float* mp = F(m, "m");
    float* op = Fm(out, "out");
    EMH_ENSURE(m->len >= rows * d && out->len >= rows, "shapes");
    use_device(c);
    emh::launch_row_norms(c, mp, rows, d, op);
  });
}

int emh_normalize_rows(emh_ctx* c, const emh_buf* src, size_t rows, size_t d, emh_buf* dst) {
  return guard([&] {
    EMH_ENSURE(c && d > 0, "bad arguments");
    const float* sp = F(src, "src");
    float* dp = Fm(dst, "dst");
    EMH_ENSURE(src->len >= rows * d && dst->len >= rows * d, "shapes");
    EMH_ENSURE(src->ptr != dst->ptr || rows == 0, "normalize_rows: src and dst must differ");
    use_device(c);
    emh::launch_normalize_rows(c, sp, rows, d, dp);
  });
}

int emh_split(emh_ctx* c, emh_buf* positions, emh_buf* usage, const uint32_t* pairs,
              size_t npairs, size_t d) {
  return guard([&] {
    EMH_ENSURE(c && d > 0, "bad arguments");
    float* pp = Fm(positions, "positions");
    float* up = Fm(usage, "usage");
    const size_t k = usage->len;
    EMH_ENSURE(positions->len == k * d, "positions must be k x d");
    if (npairs == 0) return;
    EMH_ENSURE(pairs != nullptr, "null plan");
    std::vector<uint8_t> seen(k, 0);
    bool independent = true;
    for (size_t q = 0; q < npairs; q++) {
      uint32_t s = pairs[2 * q], t = pairs[2 * q + 1];
      EMH_ENSURE(s < k && t < k, "split ids out of range");
      if (seen[s] || seen[t] || s == t) independent = false;
      seen[s] = seen[t] = 1;
    }
    use_device(c);
    uint32_t* pd = (uint32_t*)c->misc.get(npairs * 8);
    EMH_HIP(hipMemcpyAsync(pd, pairs, npairs * 8, hipMemcpyHostToDevice, c->stream));
    EMH_HIP(hipStreamSynchronize(c->stream));
    emh::launch_split(c, pp, up, pd, npairs, d, independent);
  });
}

int emh_ema_update(emh_ctx* c, emh_buf* positions, emh_buf* usage, const emh_buf* sums,
                   const emh_buf* counts, size_t k, size_t d, float alpha, float decay,
                   int replace) {
  return guard([&] {
    EMH_ENSURE(c && d > 0, "bad arguments");
    float* pp = Fm(positions, "positions");
    float* up = Fm(usage, "usage");
    const float* sp = F(sums, "sums");
    const uint32_t* cp = U(counts, "counts");
    EMH_ENSURE(positions->len == k * d && usage->len == k && sums->len == k * d &&
                   counts->len == k,
               "shapes");
    use_device(c);
    emh::ProfScope prof(c, EMH_PROF_EMA, emh::ema_bytes(k, d), emh::prof_take(c, EMH_PROF_EMA));
    emh::launch_ema(c, pp, up, sp, cp, k, d, alpha, decay, replace);
  });
}

uint64_t emh_fallback_rows(emh_ctx* c) {
  if (!c) return 0;
  uint32_t v = 0;
  if (hipSetDevice(c->device) != hipSuccess) return 0;
  if (hipMemcpyAsync(&v, c->small + emh::SW_FALLBACK_TOTAL, 4, hipMemcpyDeviceToHost,
                     c->stream) != hipSuccess)
    return 0;
  (void)hipStreamSynchronize(c->stream);
  return v;
}

int emh_set_screen(emh_ctx* c, int on) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    EMH_ENSURE(on >= 0 && on <= 3, "screen mode %d: 0 (off), 1 (bf16), 2 (f32) or 3 (fp16)",
               on);
    c->screen = on;
  });
}

int emh_set_exact_below(emh_ctx* c, uint64_t items) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    c->exact_below = (size_t)items;
  });
}

int emh_profile(emh_ctx* c, int on) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    EMH_ENSURE(on >= 0, "profile period %d must be >= 0", on);
    for (int op = 0; op < EMH_PROF_OPS; op++) {
      c->prof[op] = on;
      c->prof_count[op] = 0;
    }
  });
}

int emh_profile_op(emh_ctx* c, int op, int on) {
  return guard([&] {
    EMH_ENSURE(c, "null context");
    EMH_ENSURE(op >= 0 && op < EMH_PROF_OPS, "unknown profiled op %d", op);
    EMH_ENSURE(on >= 0, "profile period %d must be >= 0", on);
    c->prof[op] = on;
    c->prof_count[op] = 0;
  });
}

int emh_profile_read_op(emh_ctx* c, int op, double* ms, uint64_t* instances, double* units) {
  return guard([&] {
    EMH_ENSURE(c && ms && instances && units, "null argument");
    EMH_ENSURE(op >= 0 && op < EMH_PROF_OPS, "unknown profiled op %d", op);
    use_device(c);
    EMH_HIP(hipStreamSynchronize(c->stream));
    // Every timed segment so far goes into its op's totals; the events go
    // back to the pool.
    for (auto& e : c->timed) {
      float m = 0.f;
      EMH_HIP(hipEventElapsedTime(&m, e.a, e.b));
      emh_ctx::ProfSum& s = c->prof_sum[e.op];
      s.ms += m;
      if (e.last) {
        s.units += e.units;
        s.instances++;
      }
    }
    c->timed.clear();
    c->ev_used = 0;
    emh_ctx::ProfSum& s = c->prof_sum[op];
    *ms = s.ms;
    *instances = s.instances;
    *units = s.units;
    s = emh_ctx::ProfSum{};
  });
}

int emh_profile_read(emh_ctx* c, double* ms, uint64_t* launches, double* flop) {
  return emh_profile_read_op(c, EMH_PROF_SCREEN, ms, launches, flop);
}

}  // extern "C"
